/* moe_oracle.h -- CPU restatement of eureka-engine's MoE FFN hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (eureka-engine_amd/) includes,
 * links or calls this code; tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it as the checker the HIP path is compared against.
 *
 * Numeric classes (reference: tools/payload-moeany.patch:78-84, host/llb_pf.cuh:447-455):
 *   exact  f32 activations, f32 dequant, every op rounded once in a declared order;
 *          the GPU exact tier must reproduce it bit for bit.
 *   q8     routed and shared expert products on q8_1 activations (llb_mx_*, pf_q8x):
 *          tolerance class.
 *   f64    float64 recompute from the same dequantized weights and ids
 *          (reports/metal-catchup/tools/mx_ref.py:44-57 semantics): tolerance checks.
 * Build with -O2 -ffp-contract=off (no FMA contraction anywhere in this file).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* format codes, host/llb_formats.h:4-14 */
#define MO_F32 0u
#define MO_Q8_0 1u /* GGUF blocks [f16 d][i8 q x32], as expert stacks keep them */
#define MO_Q4_K 3u
#define MO_Q6_K 4u
#define MO_Q5_K 9u

/* dot orders of the exact tier */
#define MO_ORDER_STRIDE 0 /* moe_dot / llb_gemv_any: 32 lanes strided, xor tree */
#define MO_ORDER_TREE 1   /* llb_warp / kp_pair: balanced tree over 2^cdepth groups */

typedef struct {
  uint32_t dm, ne, nk, ef, sf;   /* d_model, experts, top-k, expert ff, shared ff (0: none) */
  uint32_t fg, fu, fd;           /* routed gate / up / down formats */
  uint32_t fsg, fsu, fsd;        /* shared gate / up / down formats */
  const float* router;           /* [ne][dm] f32 */
  const float* shgate;           /* [dm] f32 (NULL when sf == 0) */
  const uint8_t* G;              /* [ne][ef] rows of dm cols, format fg */
  const uint8_t* U;              /* [ne][ef] rows of dm cols, format fu */
  const uint8_t* D;              /* [ne][dm] rows of ef cols, format fd */
  const uint8_t* SG;             /* [sf] rows of dm cols */
  const uint8_t* SU;             /* [sf] rows of dm cols */
  const uint8_t* SD;             /* [dm] rows of sf cols */
  const float* router_bias;      /* [ne] added to each logit (NULL: none); batched-decode expert skew */
} mo_layer;

/* ---- formats ---- */
float mo_f16(uint32_t h);                       /* llb_f16, tools/quant-fix.patch:11-21 */
uint16_t mo_f32_to_f16(float f);                /* round to nearest even */
uint64_t mo_row_bytes(uint32_t fm, uint32_t cols); /* LLB_FM_RB, host/llb_formats.h:16 */
int mo_deq_row(uint32_t fm, const uint8_t* row, uint32_t cols, float* out);
int mo_quant_row(uint32_t fm, const float* x, uint32_t cols, uint8_t* out);

/* ---- synthetic data (also produced on the device by the product's generator) ---- */
float mo_gauss(uint64_t seed, uint64_t stream, uint64_t i, float sigma);
void mo_gauss_fill(uint64_t seed, uint64_t stream, uint64_t i0, uint64_t n, float sigma, float* out);
/* rows [r0, r0+nr) of a quantized matrix whose fp32 source is mo_gauss(seed, stream, r * cols + c) */
int mo_gen_rows(uint32_t fm, uint64_t seed, uint64_t stream, uint64_t r0, uint64_t nr, uint32_t cols,
                float sigma, uint8_t* out);

/* ---- dots ---- */
uint32_t mo_cdepth(uint32_t cols);
int mo_tuned(uint32_t fm, uint32_t cols);
float mo_dot_stride(uint32_t fm, const uint8_t* row, uint32_t cols, const float* x);
float mo_dot_tree(uint32_t fm, const uint8_t* row, uint32_t cols, const float* x);
/* llb_kgemv's choice for one row: the tree where a tuned body applies, else llb_gemv_any */
float mo_gemv_row(uint32_t fm, const uint8_t* row, uint32_t cols, const float* x);
float mo_exp(float x);
float mo_silu_mul(float g, float u);
float mo_sigmoid(float x);
void mo_renorm(float* wt, uint32_t nk);
float mo_combine(const float* v, const float* wt, uint32_t nk, int shared, float hv, float sgo, float res);

/* ---- routing ---- */
void mo_router(const mo_layer* L, const float* h2, float* lg, float* sg);
void mo_topk(const float* lg, uint32_t ne, uint32_t nk, float sg, uint32_t* ids, float* wt, float* sgo);
/* the dispatch permutation over n = T*nk slots, host/llb_pf.cuh:774-817 */
void mo_group(const uint32_t* ids, uint32_t n, uint32_t nk, uint32_t ne, uint32_t* off, uint32_t* xmap,
              uint32_t* inv);

/* ---- the layer ----
 * T tokens, h2/x1/y [T][dm]; ids/wt [T][nk]; sgo [T]. nthreads 1 = scalar, >1 OpenMP rows.
 * Returns 0 on success, <0 on a shape or format the path does not take. */
int mo_moe_exact(const mo_layer* L, uint32_t T, const float* h2, const float* x1, float* y, uint32_t* ids,
                 float* wt, float* sgo, int nthreads);
/* act [T*nk][ef] of the exact tier (gate/up/SwiGLU only), for kernel-level checks */
int mo_moe_exact_act(const mo_layer* L, uint32_t T, const float* h2, const uint32_t* ids, float* act);
int mo_moe_q8(const mo_layer* L, uint32_t T, const float* h2, const float* x1, float* y, uint32_t* ids,
              float* wt, float* sgo, int nthreads);
/* float64 recompute given ids (from the exact tier): y64 [T][dm] without residual */
int mo_moe_f64(const mo_layer* L, uint32_t T, const float* h2, const uint32_t* ids, double* y64);

/* q8_1 activations, pf_q8x / ref_q8x: per 32 values d = amax / 127, q = round(x / d), s = sum x */
void mo_q8_1(const float* x, uint32_t n, int8_t* q, float* d, float* s);
/* llb_rmsnorm_add (tools/payload-fuse.patch:106-127): x1 = x + z (x1 may be NULL), h2 = (x1 s) w,
 * s = 1 / sqrt(tree sum of x1^2 / n + eps), returned */
float mo_rmsnorm_add(const float* x, const float* z, const float* w, float eps, uint32_t n, float* x1, float* h2);
float mo_dot_q8(uint32_t fm, const uint8_t* row, uint32_t cols, const int8_t* q, const float* d,
                const float* s);

#ifdef __cplusplus
}
#endif
#endif
