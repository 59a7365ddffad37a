// moe_noalloc.hip -- llb_moe_hip_forward for callers that cannot allocate (code under graph capture,
// serving loops, harnesses that forbid hipMalloc): the layer's transient state lives in a file-scope
// device array instead of a caller scratch. Each device holds its own copy of the array, at its own
// address, for the life of the process. Host code never passes the array's name (a host-side stand-in,
// not a device address): set-up resolves the device address once per device with hipGetSymbolAddress,
// and the entry point hands that address to the forward as its scratch. Nothing in the array has to
// start at zero (the forward writes every byte it reads), so no call clears it.
#include <hip/hip_runtime.h>
#include <stdio.h>

#include <mutex>

#include "../../include/llb_moe_hip.h"
#include "moe_kernels.h"

static __device__ __align__(256) uint8_t scratch[LLB_MOE_STATIC_SCRATCH_BYTES];

static constexpr int kMaxDev = 64;
static void* g_scratch_ptr[kMaxDev];
static std::mutex g_scratch_mu;

// the array's device address on `device` (current), resolved once
int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDev) return llb_fail_msg(LLB_HIP_EINVAL, "static scratch: device index past 63");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[device]) return 0;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    (void)hipGetLastError();
    char msg[160];
    snprintf(msg, sizeof msg, "static scratch: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    return llb_fail_msg(LLB_HIP_EDEVICE, msg);
  }
  g_scratch_ptr[device] = p;
  return 0;
}

extern "C" int llb_moe_hip_forward_static(const llb_moe_layer* L, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y,
                                          llb_dptr ids, llb_dptr wt, int tier) {
  if (!L) return llb_fail_msg(LLB_HIP_EINVAL, "forward_static: null layer");
  if (tier != LLB_MOE_EXACT && tier != LLB_MOE_Q8)
    return llb_fail_msg(LLB_HIP_EINVAL, "forward_static: the exact and q8 tiers only (the f16 tier makes its side "
                                        "stream on first use)");
  if (L->res == LLB_MOE_RES_STREAM)
    return llb_fail_msg(LLB_HIP_EINVAL, "forward_static: a streamed layer stages its experts through host memory");
  const size_t need = llb_moe_hip_scratch_bytes(L, T, tier);
  if (need > LLB_MOE_STATIC_SCRATCH_BYTES) {
    char msg[160];
    snprintf(msg, sizeof msg, "forward_static: this layer and T need %zu bytes of scratch; the static array holds %u",
             need, (unsigned)LLB_MOE_STATIC_SCRATCH_BYTES);
    return llb_fail_msg(LLB_HIP_EINVAL, msg);
  }
  if (T == 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return llb_fail_msg(LLB_HIP_EDEVICE, "forward_static: hipGetDevice failed");
  }
  const int rc = noalloc_setup(dev);
  if (rc) return rc;
  return llb_moe_hip_forward(L, T, h2, x1, y, ids, wt, (llb_dptr)(uintptr_t)g_scratch_ptr[dev],
                             LLB_MOE_STATIC_SCRATCH_BYTES, tier);
}
