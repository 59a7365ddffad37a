#!/bin/bash
# Builds libeureka_moe.so (gfx950) in place. -ffp-contract=off: the exact tier's float ops are
# executed as written; -packed-fp32-ops off: no v_pk_*_f32. Each source compiles to its own object in
# parallel (at most 8 jobs), then one link.
set -euo pipefail
cd "$(dirname "$0")"
FLAGS=(--offload-arch=gfx950 -O3 -std=c++17 -fPIC -ffp-contract=off
       -Xclang -target-feature -Xclang -packed-fp32-ops "$@")
SRCS=(csrc/llb_moe_hip.cpp csrc/llb_moe_table.cpp csrc/llb_moe_gguf.cpp csrc/moe_exact.hip csrc/moe_decode.hip
      csrc/moe_q8.hip csrc/moe_synth.hip csrc/moe_gemm.hip csrc/moe_noalloc.hip)
OBJ=_obj
mkdir -p "$OBJ"
pids=()
for s in "${SRCS[@]}"; do
  o="$OBJ/$(basename "$s").o"
  if [[ "$s" == *.cpp ]]; then hipcc "${FLAGS[@]}" -x hip -c -o "$o" "$s" & else hipcc "${FLAGS[@]}" -c -o "$o" "$s" & fi
  pids+=($!)
done
for p in "${pids[@]}"; do wait "$p"; done
hipcc --offload-arch=gfx950 -fPIC -shared -o libeureka_moe.so "$OBJ"/*.o
# the standalone C host for one layer (driver/moe_layer_drv.c), linked against the library in place, and
# the code object its LLB_LAUNCH loads by name
hipcc --offload-arch=gfx950 -O3 --genco -Xclang -target-feature -Xclang -packed-fp32-ops \
  -o drv_kernels.hsaco driver/drv_kernels.hip
gcc -O2 -std=c11 -D_DEFAULT_SOURCE -Wall -Wextra -o moe_layer_drv driver/moe_layer_drv.c -L. -leureka_moe \
  -Wl,-rpath,'$ORIGIN'
