/* llb_moe_hip.h -- C ABI of the MI355X (gfx950) MoE FFN backend.
 *
 * Drop-in boundary for eureka-engine's routed-expert FFN. The reference reaches this path through
 * llb_moe_run (host/llb_host.c:622-724) and, for a prompt chunk, pf_moe (host/llb_pf.h:286-389),
 * both over the backend contract of host/llb_backend.h:1-51 (realised for CUDA in
 * host/llb_backend_cuda.h). This header gives
 *   - that backend contract as plain functions (llb_hip_*),
 *   - the layer entry points (llb_moe_hip_forward: decode, batched decode and prefill), and
 *   - kernel-level entry points that replace the reference kernels one for one, for callers that
 *     keep the reference's launch sequence.
 * Plain pointers and sizes only. Device addresses are llb_dptr (u64), as in host/llb_backend.h:8-10.
 * Every function returns 0 (or a non-zero dptr) on success and a negative code on failure;
 * llb_hip_last_error() names the failure. Launches are queued in call order on the library's
 * stream (llb_hip_set_stream; default the null stream), like the reference's null-stream launches.
 */
#ifndef LLB_MOE_HIP_H
#define LLB_MOE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint64_t llb_dptr; /* host/llb_backend.h:8-10 */

/* error codes */
#define LLB_HIP_OK 0
#define LLB_HIP_EINVAL -1   /* a shape, format or argument outside the path's envelope */
#define LLB_HIP_EDEVICE -2  /* a HIP runtime call failed */
#define LLB_HIP_ESCRATCH -3 /* the scratch buffer is smaller than llb_moe_hip_scratch_bytes */

/* format codes, host/llb_formats.h:4-14 */
#define LLB_FM_F32 0
#define LLB_FM_Q8_0 1
#define LLB_FM_Q4_K 3
#define LLB_FM_Q6_K 4
#define LLB_FM_Q5_K 9

/* numeric tiers */
#define LLB_MOE_EXACT 0 /* the reference's exact tier: bit-identical to its f32 kernels */
#define LLB_MOE_Q8 1    /* expert products on q8_1 activations (LLB_MOE_DP4A / LLB_PREFILL=fast) */
#define LLB_MOE_F16 2   /* grouped expert GEMMs on MFMA, f16 operands, f32 accumulate (prefill) */

/* ---- backend contract (host/llb_backend.h:8-41; CUDA twin host/llb_backend_cuda.h:186-219) ---- */
int llb_hip_init(int device);                                  /* cuInit + context: gpu_load */
const char* llb_hip_last_error(void);
int llb_hip_set_stream(void* hip_stream);                      /* NULL: the null stream */
llb_dptr llb_hip_alloc_zero(size_t bytes);                     /* llb_alloc_zero, llb_backend_cuda.h:186-191 */
int llb_hip_free(llb_dptr p);                                  /* (the reference never frees) */
int llb_hip_zero(llb_dptr p, size_t bytes);                    /* llb_zero */
int llb_hip_copy(llb_dptr d, llb_dptr s, size_t bytes);        /* llb_copy */
int llb_hip_write(llb_dptr d, const void* h, size_t bytes);    /* llb_write, llb_backend_cuda.h:210-213 */
int llb_hip_read(void* h, llb_dptr p, size_t bytes);           /* llb_read, llb_backend_cuda.h:198-201 */
int llb_hip_sync(void);                                        /* llb_sync, llb_backend_cuda.h:216-219 */
int llb_hip_mem_info(size_t* free_bytes, size_t* total_bytes); /* cuMemGetInfo, host/llb_host.c:531 */
/* kernel by name (cuModuleGetFunction, host/llb_backend.h:37-39) and LLB_LAUNCH / LLB_LAUNCH_SM
 * (host/llb_backend.h:11-24, host/llb_backend_cuda.h:7-11,82-99): load a gfx950 code object, look up a
 * kernel, launch gx x gy groups of bx threads with sm bytes of dynamic LDS on the library's stream.
 * args[i] is the address of a host variable holding argument i; na counts them. The C macros over these
 * are in llb_backend_hip.h. */
int llb_hip_module_load(const char* path, uint64_t* module);
int llb_hip_module_function(uint64_t module, const char* name, void** fn);
int llb_hip_launch(void* fn, uint32_t gx, uint32_t gy, uint32_t bx, uint32_t sm, void** args, uint32_t na);
/* with a z grid (the fast prefill's direct cuLaunchKernel, host/llb_pf.h:284-285) */
int llb_hip_launch3(void* fn, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t sm, void** args,
                    uint32_t na);
/* pinned, device-mapped host memory and its device address (cuMemHostAlloc(DEVICEMAP | PORTABLE) +
 * cuMemHostGetDevicePointer, host/llb_host.c:446-489), and its release */
int llb_hip_host_alloc(size_t bytes, void** host, llb_dptr* dev);
int llb_hip_host_free(void* host);
/* host to device in stream order without waiting (cuMemcpyHtoDAsync, host/llb_host.c:691-693) */
int llb_hip_copy_h2d_async(llb_dptr d, const void* h, size_t bytes);
/* graph record / replay: llb_graph_begin / llb_graph_end (host/llb_backend_cuda.h:125-184). Launches
 * between begin and end are captured (not run); launch replays them on the library's stream.
 * No allocation, copy or read may happen inside a capture (the reference bails to eager there). */
int llb_hip_graph_begin(void);
int llb_hip_graph_end(uint64_t* handle);
int llb_hip_graph_launch(uint64_t handle);
int llb_hip_graph_free(uint64_t handle);

/* ---- the layer ----
 * What llb_moe_run reads from a layer's table row (host/llb_host.c:623-627, words of
 * tools/gguf2pack.c:1142-1146) plus the device addresses llb_moe_load resolves
 * (host/llb_host.c:491-586). Stacks are GGUF 3-D [ne][rows][row bytes] verbatim. */
typedef struct {
  uint32_t dm;  /* d_model (LlbShape.d) */
  uint32_t ne;  /* word 27: expert count */
  uint32_t nk;  /* word 30: experts used */
  uint32_t ef;  /* word 28: expert ff */
  uint32_t sf;  /* word 29: shared ff; 0 = no shared expert */
  uint32_t fx;  /* word 26: gate | up << 4 | down << 8, bit 12 fused gate+up */
  uint32_t fsg, fsu, fsd; /* shared gate / up / down formats (words 2..4 >> 28) */
  uint32_t pad;
  llb_dptr router; /* F32 [ne][dm] (word 21) */
  llb_dptr shgate; /* F32 [dm] (word 22); 0 when sf == 0 */
  llb_dptr G, U, D;    /* expert stacks; U ignored when fused (U = G + ef rows, llb_host.c:677) */
  llb_dptr SG, SU, SD; /* shared expert */
  llb_dptr router_bias; /* F32 [ne] added to each router logit, one rounding (0: none). Not in the
                         * reference: the batched-decode workload skews expert load with it */
  llb_dptr PG, PU, PD;    /* packed copies of G, U, D for the f16 tier (llb_moe_hip_pack; 0: none) */
  llb_dptr PSG, PSU, PSD; /* packed copies of SG, SU, SD */
  uint32_t res;           /* residency of G / U / D (LLB_MOE_RES_*; 0 = device, the default) */
  uint32_t own;           /* router, shgate, SG, SU, SD (bits 0..4) that llb_moe_hip_load_layer allocated */
  llb_dptr stream;        /* LLB_MOE_RES_STREAM: the loader's per-layer source (host address; 0 otherwise) */
} llb_moe_layer;

/* ---- the layer's table row (host code) ----
 * w: the layer's 32 raw table.bin words (tools/gguf2pack.c:1142-1146): w[21] router, w[22] shared
 * gate row, w[3..5] shared gate / up / down (offset | fm << 28), w[26] formats, w[27] ne, w[28] ef,
 * w[29] sf, w[30] nk. check: pass_mail's MoE admission (tools/payload-moeany.patch:26-50), 0 or 8.
 * from_table: llb_moe_run's field decode (host/llb_host.c:623-627), base = the layer's Bytes.
 * run_table: both, then llb_moe_hip_forward (the call site's one-line replacement). */
int llb_moe_table_check(const uint32_t* w, uint32_t dm, uint32_t df, uint64_t len);
int llb_moe_layer_from_table(const uint32_t* w, uint32_t dm, llb_dptr base, llb_dptr G, llb_dptr U, llb_dptr D,
                             llb_moe_layer* out);
int llb_moe_run_table(const uint32_t* w, uint32_t dm, uint32_t df, uint64_t len, llb_dptr base, llb_dptr G,
                      llb_dptr U, llb_dptr D, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y, llb_dptr ids,
                      llb_dptr wt, llb_dptr scratch, size_t scratch_bytes, int tier);

/* bytes of scratch llb_moe_hip_forward needs for T tokens at a tier (llb_scratch, host/llb_host.c:634) */
size_t llb_moe_hip_scratch_bytes(const llb_moe_layer* L, uint32_t T, int tier);

/* One MoE FFN layer over T tokens (llb_moe_run for T = 1, pf_moe's contract for a chunk).
 * h2: [T][dm] f32 normalised FFN input; x1: [T][dm] residual (0: none); y: [T][dm] out,
 * y = sum_j wt_j expert_j(h2) + sigmoid(sg) shared(h2) + x1.
 * ids: [T][nk] u32 and wt: [T][nk] f32 out (the routing, as llb_moe_topk writes it).
 * Routing is the exact tier's at every tier. Replaces host/llb_host.c:647-723 / host/llb_pf.h:286-389. */
int llb_moe_hip_forward(const llb_moe_layer* L, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y, llb_dptr ids,
                        llb_dptr wt, llb_dptr scratch, size_t scratch_bytes, int tier);

/* One layer with its input step: x1 = x + z and h2 = rmsnorm(x1) w, as llb_moe_hip_rmsnorm_add computes
 * them (llb_rmsnorm_add, tools/payload-fuse.patch:106-127), then llb_moe_hip_forward(L, T, h2, x1, ...).
 * x1 and h2 ([T][dm]) are written too. For T < 16 the router launch computes the input step itself
 * (each of its blocks recomputes the token's norm), one launch fewer a layer; otherwise the input step
 * runs as its own launch first. The bits are the two calls' either way. No single counterpart in the
 * reference: there llb_rmsnorm_add and llb_moe_run are separate launches (host/llb_host.c:622-724). */
int llb_moe_hip_forward_norm(const llb_moe_layer* L, uint32_t T, llb_dptr x, llb_dptr z, llb_dptr w, float eps,
                             llb_dptr x1, llb_dptr h2, llb_dptr y, llb_dptr ids, llb_dptr wt, llb_dptr scratch,
                             size_t scratch_bytes, int tier);

/* The forward with no scratch argument and no allocation. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The transient state lives in a device array of LLB_MOE_STATIC_SCRATCH_BYTES built into the
 * library (one copy per device, held until the process ends; its address is resolved by llb_hip_init or
 * by the first call on a device). Same bits as llb_moe_hip_forward. Exact and q8 tiers, resident layers
 * (not LLB_MOE_RES_STREAM); a layer and T whose llb_moe_hip_scratch_bytes exceeds the array are refused
 * with LLB_HIP_EINVAL. Every call on a device shares that device's array: calls that overlap on one
 * device (several streams or host threads) race and must be serialised by the caller. */
#define LLB_MOE_STATIC_SCRATCH_BYTES (16u << 20)
int llb_moe_hip_forward_static(const llb_moe_layer* L, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y, llb_dptr ids,
                               llb_dptr wt, int tier);

/* The fused one-launch layer (k_fused: the four stages as work items of one persistent launch with
 * completion counters between phases) is disabled: it hung the GPU twice and the cause is not shown.
 * set_fused(0) is accepted (the three / four-launch path, the only one that runs); set_fused(on != 0)
 * returns LLB_HIP_EINVAL with a message naming the hang. status reads the fused path's timeout flag
 * in a scratch (LLB_HIP_EDEVICE, cleared, when set); with the path disabled it is never set.
 * No counterpart in the reference. */
int llb_moe_hip_set_fused(int on);

/* The q8 tier from 16 tokens on: the int8-MFMA grouped GEMM (k_gemm_i8, the counterpart of the
 * reference's int8 tensor-core prefill pfx_* / llb_mx_*, host/llb_pf.cuh:819-848) when on, per-slot v_dot4
 * GEMVs when off (the same q8_1 numerics class). Off by default: its one GPU run so far faulted, on a cause
 * since fixed (a Q8_0 code load past the stack's last block) and not yet run again. The initial state comes
 * from LLB_MOE_Q8_GEMM=1 in the environment at load. The switch sizes the q8 scratch
 * (llb_moe_hip_scratch_bytes) as well as choosing the kernels: size scratch after setting it, and do not
 * change it while forwards run. q8_gemm returns the current state. No counterpart in the reference (its
 * tier is chosen by LLB_PREFILL at build time). */
int llb_moe_hip_set_q8_gemm(int on);
int llb_moe_hip_q8_gemm(void);
int llb_moe_hip_status(llb_dptr scratch, const llb_moe_layer* L, uint32_t T);

/* ---- GGUF expert stacks: llb_moe_load's residency (host/llb_host.c:446-586) and llb_gg_tensor
 * (host/llb_gguf.c:854-865). open parses a GGUF (v2 / v3) header, every length checked against the
 * file; find returns a tensor's index or -1; tensor_at its name, absolute file offset, bytes (0 for a
 * type this path does not read), ggml type and dims (ne[0] fastest). load_layer fills L->G / U / D for
 * blk.<layer>.ffn_{gate,up,down}_exps (ffn_gate_up_exps when fx bit 12 is set) after checking each
 * tensor's type and bytes against L's formats and shape words, and also router / shgate / SG / SU / SD
 * from ffn_gate_inp, ffn_gate_inp_shexp and ffn_{gate,up,down}_shexp when the file holds them and L
 * does not already point at them. Modes: DEVICE (device memory), HOST (pinned, device-mapped host
 * memory; the kernels read it over the bus), STREAM (the file mapped; llb_moe_hip_forward copies the k
 * chosen experts of each token into device staging slots -- exact tier, one token, no graph capture).
 * Every mode gives the same bits. unload_layer frees what load_layer allocated. */
#define LLB_MOE_RES_DEVICE 0
#define LLB_MOE_RES_HOST 1
#define LLB_MOE_RES_STREAM 2
typedef struct llb_gguf llb_gguf;
llb_gguf* llb_gguf_open(const char* path);
void llb_gguf_close(llb_gguf* g);
uint64_t llb_gguf_count(const llb_gguf* g);
int llb_gguf_find(const llb_gguf* g, const char* name);
int llb_gguf_tensor_at(const llb_gguf* g, uint64_t i, char* name, size_t cap, uint64_t* offset, uint64_t* bytes,
                       uint32_t* type, uint32_t* nd, uint64_t* dims);
int llb_moe_hip_load_layer(llb_gguf* g, uint32_t layer, int mode, llb_moe_layer* L);
/* The table rows a qwen35moe GGUF's header implies, as the reference's sidecar writer makes them
 * (tools/gguf2pack.c:1134-1346; word map :1142-1146): word 0 the layer's trunk bytes, words 1..20 the dense
 * tensors' offsets in the trunk (the shared expert under ffn_gate / up / down), 21 router, 22 shared gate
 * row (offset | format << 28), 26 expert formats (bit 12 fused gate+up, bit 13 set), 27 experts, 28 expert
 * ff, 29 shared ff, 30 experts used. table holds cap rows of 32 words; *nlayers gets the layer count (the
 * trailing nextn blocks left out). The rows decode with llb_moe_layer_from_table. */
int llb_moe_table_from_gguf(const llb_gguf* g, uint32_t* table, uint32_t cap, uint32_t* nlayers);
int llb_moe_hip_unload_layer(llb_moe_layer* L);
/* llb_moe_load's residency choice (host/llb_host.c:532-545): sums the routed stacks of the n layers
 * (layers[i] is L[i]'s block index; each stack checked as load_layer checks it) and picks DEVICE when they
 * fit free device memory less 0.75 GiB, else HOST when they fit MemAvailable less 4 GiB, else STREAM.
 * Environment: LLB_MOE_VRAM / LLB_MOE_RAM (bytes) replace the two capacities (with LLB_MOE_VRAM set no
 * device is queried); LLB_MOE_EXPERTS=device|host|stream forces the mode. Prints the reference's
 * "moe: N layers, experts X GiB -> mode [free VRAM .., MemAvailable ..]" line on stderr. expert_bytes
 * may be null. */
int llb_moe_hip_residency(const llb_gguf* g, const uint32_t* layers, const llb_moe_layer* L, uint32_t n, int* mode,
                          uint64_t* expert_bytes);

/* ---- packed weights for the f16 tier. No counterpart in the reference, whose prefill decodes GGUF
 * blocks where they lie. The grouped GEMM reads each weight tile of 32 rows x 64 columns as one
 * coalesced block when the stacks are re-laid once into tiles in its operand order; the packed copy
 * holds the same codes and f16 scales the GEMM derives from the GGUF blocks, so results are the same
 * bit for bit. pack_bytes: device bytes for packed copies of every stack of L (0 when the f16 tier
 * cannot take L). pack: fills buf (at least pack_bytes) from L's GGUF stacks, on the library stream,
 * and sets L->PG .. L->PSD; layers without them keep working on the GGUF stacks. */
size_t llb_moe_hip_pack_bytes(const llb_moe_layer* L);
int llb_moe_hip_pack(llb_moe_layer* L, llb_dptr buf, size_t bytes);

/* ---- kernel-level entry points ---- */
/* llb_rmsnorm_add (tools/payload-fuse.patch:106-127; host/llb_host.c's gpu_rnadd), the step that makes
 * the router's input, for T rows of n <= 16384 (a multiple of 4 past 512): x1 = x + z, h2 = (x1 s) w, s = 1 / sqrt(sum x1^2 / n +
 * eps), the sum in the reference kernels' tree order. x, z, x1, h2: [T][n] f32 (x1 may be 0); w: [n]. */
int llb_moe_hip_rmsnorm_add(llb_dptr x, llb_dptr z, llb_dptr w, float eps, uint32_t T, uint32_t n, llb_dptr x1,
                            llb_dptr h2);
/* llb_moe_topk block 0 (tools/payload-moeany.patch:311-470) for T tokens: lg [T][lstride] (ne logits,
 * then the shared gate's at index ne when has_sg) -> ids, wt [T][nk], sgo [T] */
int llb_moe_hip_topk(llb_dptr lg, uint32_t lstride, uint32_t T, uint32_t ne, uint32_t nk, uint32_t has_sg,
                     llb_dptr ids, llb_dptr wt, llb_dptr sgo);
/* llb_mx_group (host/llb_pf.cuh:774-817): n = T nk slots -> off [ne+1], xmap [n], inv [n]. scratch:
 * group_scratch_bytes(n, ne) bytes (the histogram + scan pair's per-block expert counts). */
int llb_moe_hip_group(llb_dptr ids, uint32_t n, uint32_t nk, uint32_t ne, llb_dptr off, llb_dptr xmap, llb_dptr inv,
                      llb_dptr scratch, size_t scratch_bytes);
size_t llb_moe_hip_group_scratch_bytes(uint32_t n, uint32_t ne);
/* The dispatch permutation's kernels: off (the default), one block an expert scanning every slot (O(ne n));
 * on, a device histogram and prefix scan (two launches, O(n + ne n / 1024), ne <= 1024): per-block stable
 * counts by wave ballots, then per-expert offsets by a scan over blocks and experts, then placement. Both
 * give the same off / xmap / inv (the stable order). The scan pair is off until it has run on a GPU.
 * No counterpart in the reference (llb_mx_group is one fixed kernel). */
int llb_moe_hip_set_group_scan(int on);
int llb_moe_hip_group_scan(void);
/* The one-token decode's routing inside its gate / up launch: off (the default), the 1024-thread top-k
 * with seven barriers; on, for ne <= 256 and nk <= 16, a variant with four barriers (a key's place in its
 * 64-expert group and a candidate's rank counted in registers by readlane). Same ids, weights and bits.
 * Off until the variant has run on a GPU. No counterpart in the reference. */
int llb_moe_hip_set_lean_topk(int on);
int llb_moe_hip_lean_topk(void);
/* pf_q8x (tools/pf27/pfmm.cuh:39-54): n f32 (n % 32 == 0) -> q int8 [n], ds float2 {d, s} [n / 32] */
int llb_moe_hip_q8_1(llb_dptr x, uint32_t n, llb_dptr q, llb_dptr ds);
/* rows of a stack dequantized to f32 (the decoders the kernels use; q8g_w / q4k_w / q6k_w / q5k_w) */
int llb_moe_hip_dequant(uint32_t fm, llb_dptr W, uint32_t rows, uint32_t cols, llb_dptr out);
/* y[i] = (float)exp((double)x[i]), the exp every softmax, SwiGLU and sigmoid of the path uses (attn_exp,
 * tools/payload-attn.patch:57-59; hf_exp, tools/qwen35_engine.c:46-50): for parity checks */
int llb_moe_hip_exp(llb_dptr x, uint64_t n, llb_dptr y);

/* ---- per-stage timing (no counterpart in the reference; its LLB_STEP_US times whole steps,
 * host/llb_host.c:2873-2891): on = 1 resets and starts a tally of HIP-event intervals around each
 * stage of llb_moe_hip_forward (at most 64 per stage between reads); read syncs and returns the mean
 * microseconds and counts per stage (eager launches only: nothing is timed inside a graph capture).
 * llb_hip_spin(us) queues a kernel that holds the stream for us microseconds (bounded), so the launches
 * behind it run back to back and the intervals measure the kernels. Stage names: llb_moe_hip_stage_name. */
int llb_hip_spin(uint32_t us);
int llb_moe_hip_timing(int on);
int llb_moe_hip_timing_read(double* mean_us, long* counts, int n);
const char* llb_moe_hip_stage_name(int stage);

/* ---- synthetic data (benchmarks and tests): element i of stream s is a normal(0, sigma)
 * from a hash of (seed, s, i); quantized rows use this project's quantizers ---- */
int llb_moe_hip_gen_gauss(uint64_t seed, uint64_t stream, uint64_t i0, uint64_t n, float sigma, llb_dptr out);
int llb_moe_hip_gen_rows(uint32_t fm, uint64_t seed, uint64_t stream, uint64_t r0, uint64_t nr, uint32_t cols,
                         float sigma, llb_dptr out);

#ifdef __cplusplus
}
#endif
#endif
