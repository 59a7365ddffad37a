// moe_kernels.h -- kernel argument blocks and launchers shared by the HIP sources and the C-ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

enum { ST_ROUTE, ST_TOPK, ST_GU, ST_DN, ST_Q8X, ST_NSTAGE };
// Stage timing. A stage other than ST_Q8X is one kernel: stage_begin arms it, and the next launch
// made through LAUNCH_K takes the armed event pair, which hipExtLaunchKernelGGL has the GPU record
// around that kernel alone (no launch gap in the figure). ST_Q8X (several kernels) records plain
// stream events around them.
bool stage_armed(hipEvent_t* a, hipEvent_t* b);
#define LAUNCH_K(K, G, B, S, ST, ...)                                                   \
  do {                                                                                   \
    hipEvent_t ea_, eb_;                                                                 \
    if (stage_armed(&ea_, &eb_)) hipExtLaunchKernelGGL(K, G, B, S, ST, ea_, eb_, 0, __VA_ARGS__); \
    else hipLaunchKernelGGL(K, G, B, S, ST, __VA_ARGS__);                                \
  } while (0)
void stage_begin(int s);
void stage_end(int s);

// Kernel attributes (the dynamic-LDS limit) are per device: a launch site keeps a mask of the devices
// it has set them on. dev_bit() is the current device's bit (devices past 63: 0, set up every time).
#include <atomic>
inline uint64_t dev_bit() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return d >= 0 && d < 64 ? 1ull << d : 0;
}
inline bool dev_needs_setup(const std::atomic<uint64_t>& mask, uint64_t bit) { return !bit || !(mask.load() & bit); }

struct TreeSeg {
  const uint8_t* W;  // rows of `cols` columns
  uint32_t fm;
  uint64_t rb;       // row bytes
  uint32_t rows;
  float* out;        // out[t * ostride + row]
  uint32_t ostride;
  const float* bias; // added to row's dot (null: none)
};
struct TreeArgs {
  TreeSeg seg[4];
  uint32_t nseg;
  uint32_t cols;
  const float* x;  // [T][xstride]
  uint32_t T, xstride, tch;
  // the input step inside (T < 16; nz set): x is the pre-norm input, x1 = x + nz, h2 = (x1 s) nw with
  // s = 1 / sqrt(sum x1^2 / cols + eps); blocks of row block 0 store x1o / h2o for the later stages
  const float* nz;
  const float* nw;
  float eps;
  float* x1o;
  float* h2o;
#ifdef MOE_DEC_STAMPS
  unsigned long long* stamps;
#endif
};
struct TopkArgs {
  const float* lg;  // [T][lstride]: ne logits, then the shared gate's when has_sg
  uint32_t lstride, ne, nk, has_sg, sf;
  uint32_t* ids;
  float* wt;
  float* sgo;
};
struct GuArgs {
  const uint8_t *G, *U;
  uint64_t rbg, rbu;
  uint64_t es;  // expert stride of G and U in bytes (fused stacks: 2 ef rows)
  uint32_t dm, ef, nk;
  const float* h2;  // [T][dm]
  const uint32_t* ids;
  float* act;  // [T nk][ef]
};
struct DnArgs {
  const uint8_t* D;
  uint64_t rbd;
  const uint8_t* SD;
  uint64_t rbs;
  uint32_t dm, ef, nk, sf, rw;
  const float* act;
  const float* gsu;  // [T][2 sf]: the shared gate then up dots (sa = silu(g) u is formed in the kernel)
  const uint32_t* ids;
  const float* wt;
  const float* sgo;
  const float* x1;  // nullable
  float* y;
};

// the one-token decode layer (moe_decode.hip)
struct DecGuArgs {
  const uint8_t *G, *U;   // routed gate / up rows (one format, dm = 2048 columns, 16-aligned)
  uint64_t es;            // expert stride of G and U in bytes
  const uint8_t *SG, *SU; // the shared expert's gate / up rows (tree order), null when sf == 0
  uint32_t dm, ef, nk, sf;
  uint32_t nrb;           // routed blocks (the shared expert's follow)
  const float* h2;        // [dm]
  float* act;             // [nk][ef] (SwiGLU applied)
  float* gsu;             // [2 sf]: shared gate, then up dots
  float* sa;              // [sf]: the shared expert's SwiGLU
  TopkArgs tk;            // the token's logits in, ids / wt / sgo out
  // the down launch's rows, touched into this XCD's L2 for the down block of the same XCD (0: none)
  const uint8_t* D;
  uint64_t rbd;
  const uint8_t* SD;
  uint64_t rbs;
  uint32_t ndb;           // down blocks (DN_RB outputs each)
  uint32_t lean;          // 1: top-k by topk_block4 (ne <= 256, four barriers)
#ifdef MOE_DEC_STAMPS
  unsigned long long* stamps;
#endif
};
struct DecDnArgs {
  const uint8_t* D;
  uint64_t rbd;
  const uint8_t* SD;
  uint64_t rbs;
  uint32_t dm, ef, nk, sf;
  const float* act;  // [nk][ef]
  const float* sa;   // [sf]: the shared expert's SwiGLU
  const uint32_t* ids;
  const float* wt;
  const float* sgo;
  const float* x1;  // nullable
  float* y;
  uint32_t stage_bytes, xw_bytes;  // LDS a wave stages its rows / activations in, set by the launcher
#ifdef MOE_DEC_STAMPS
  unsigned long long* stamps;
#endif
};
#ifdef MOE_DEC_STAMPS
extern unsigned long long* g_dec_stamps;
#endif
int launch_router(const TreeArgs& a, uint32_t nq, hipStream_t st);
// q8: the q8 tier's dots (q8_1 activations, v_dot4) in place of the exact tier's f32 orders
int launch_gu_dec(DecGuArgs a, uint32_t f, uint32_t fs, bool q8, hipStream_t st);
int launch_dn_dec(DecDnArgs a, uint32_t fd, uint32_t fs, bool q8, hipStream_t st);
size_t dn_dec_lds(uint32_t nk, uint32_t ef, uint32_t sf, uint64_t rbd, uint64_t rbs, uint32_t dm, bool shared, bool q8,
                  uint32_t* stage_bytes, uint32_t* xw_bytes);

struct FusedArgs {
  TreeArgs tr;
  TopkArgs tk;
  GuArgs gu;
  DnArgs dn;
  uint32_t T, nR, nG, nD;
  uint32_t rpt;  // tree items a token (4 waves x 2 rows an item)
  uint32_t dpt;  // down items a token
  uint32_t np;   // gate / up row pairs an item
  uint32_t spin; // 100 MHz ticks a wait may take before it records an error
  uint32_t* ctr; // 6 counters in the scratch, cleared by launch_fused before each launch
};
int launch_fused(const FusedArgs& f, uint32_t fg, uint32_t fd, uint32_t fs, uint32_t nsp, uint32_t grid, hipStream_t st);
bool fused_supported(uint32_t fg, uint32_t fd, uint32_t fs, uint32_t nsp);
int launch_tree_rows(const TreeArgs& a, uint32_t nsp, hipStream_t st);
uint32_t dn_rows(uint32_t nk, uint32_t ef, uint32_t sf);
int launch_topk(const TopkArgs& a, uint32_t T, hipStream_t st);
uint32_t tree_rows_per_wave(uint32_t nsp);
int launch_gu_topk(const GuArgs& a, const TopkArgs& k, uint32_t fg, uint32_t fu, uint32_t nslots, hipStream_t st);
int launch_gu_exact(const GuArgs& a, uint32_t fg, uint32_t fu, uint32_t nslots, hipStream_t st);
int launch_dn_exact(const DnArgs& a, uint32_t fd, uint32_t fs, uint32_t T, hipStream_t st);
struct Q8Args {
  const uint8_t *G, *U, *D, *SG, *SU, *SD;
  uint64_t rbg, rbu, rbd, es, rbsg, rbsu, rbs;
  uint32_t fg, fu, fd, fsg, fsu, fsd;
  uint32_t dm, ef, nk, sf, rw;
  const float* h2;   // [T][dm] activations (quantized in LDS by the gate / up kernel for few tokens)
  const int8_t* hq;  // [T][dm] q8_1 of h2
  const float2* hd;  // [T][dm / 32]
  const uint32_t* ids;
  const float* wt;
  const float* sgo;
  float* act;        // [T nk][ef]
  int8_t* aq;        // [T nk][ef]
  float2* ad;
  float* sa;         // [T][sf]
  int8_t* sq;
  float2* sd2;
  const float* x1;
  float* y;
};
// the q8 tier's gate / up + SwiGLU (shared expert rows ride along); tk: route inside the launch (T = 1);
// lq: quantize the token's activations in LDS instead of reading hq / hd
int launch_gu_q8(const Q8Args& a, const TopkArgs* tk, uint32_t nslot, uint32_t T, bool lq, hipStream_t st);
struct GemmArgs {
  const uint8_t* W0;  // weights (gate / the one matrix), rows of K columns
  const uint8_t* W1;  // up (mode 0)
  uint64_t es, rb;    // expert stride, row bytes
  uint32_t K, N, M;   // M: rows when there is no tile list (the shared expert)
  uint32_t arows;     // rows of A (the bound of its buffer loads)
  const _Float16* A;  // activations, f16 rows of K
  const uint32_t* xmap;   // slot -> A row (mode 0), or null: slot itself
  const uint32_t* off;    // [ne + 1] slot offsets, or null: M rows, no experts (the shared expert)
  uint32_t ne;            // experts (<= 1024) when off is set
  void* out;          // mode 0: f16 [slots][N]; mode 1: f32 [slots][N], or f16 with o16
  uint32_t o16;       // mode 1: f16 outputs
  float* spill;       // o16: f32 [slots][N], written only where the f16 output is +-inf (|v| past 65504)
  const uint8_t* P0;  // packed W0 (null: read the GGUF rows)
  const uint8_t* P1;  // packed W1 (mode 0)
  uint64_t pes;       // packed expert stride
};
int launch_moe_gemm(const GemmArgs& g, uint32_t fm, uint32_t mode, uint32_t grid_y, hipStream_t st);
// the q8 tier's grouped GEMM on int8 MFMA (many tokens): q8_1 activations against the GGUF codes
struct GemmQ8Args {
  const uint8_t* W0;   // GGUF rows: gate (mode 0) or the one matrix (mode 1)
  const uint8_t* W1;   // up rows (mode 0)
  uint64_t es, rb;     // expert stride, row bytes
  uint32_t K, N, M;    // columns (K % 32 == 0), weight rows (mode 0: features), rows when off is null
  const int8_t* A;     // q8_1 codes, rows of K
  const float2* Ad;    // {d, s} a row's 32-column block
  const uint32_t* xmap;  // slot -> A row, or null: the slot itself
  const uint32_t* off;   // [ne + 1] slot offsets, or null (M rows, no experts: the shared expert)
  uint32_t ne;
  float* out;          // mode 0: SwiGLU [slots][N]; mode 1: [slots][N]
};
int launch_gemm_i8(const GemmQ8Args& g, uint32_t fm, uint32_t mode, uint32_t grid_y, hipStream_t st);
int launch_combine_f32(const float* out, const uint32_t* inv, const float* wt, uint32_t nk, const float* shd,
                       const float* sgo, const float* x1, float* y, uint32_t dm, uint32_t T, hipStream_t st);
// cnt: group_cnt_bytes(n, ne) of scratch for the histogram + scan pair (used when it is switched on;
// null keeps k_group)
int launch_group(const uint32_t* ids, uint32_t n, uint32_t nk, uint32_t ne, uint32_t* off, uint32_t* xmap,
                 uint32_t* inv, const float* x, _Float16* x16, uint64_t nx, hipStream_t st, uint32_t* cnt);
size_t group_cnt_bytes(uint32_t n, uint32_t ne);
void moe_set_group_scan(bool on);
bool moe_group_scan_enabled();
int launch_q8_1(const float* x, uint32_t n, int8_t* q, float2* ds, hipStream_t st);
uint32_t gemm_bm();
int llb_fail_msg(int code, const char* msg);  // sets llb_hip_last_error's text, returns code
// the static scratch's device address on the current device, resolved once (moe_noalloc.hip)
int noalloc_setup(int device);
hipStream_t llb_cur_stream();
// stream residency (llb_moe_gguf.cpp): stage_done waits for a token's uploads (the staging is reused)
int stream_done();
int launch_rmsnorm_add(const float* x, const float* z, const float* w, float eps, uint32_t T, uint32_t n, float* x1,
                       float* h2, hipStream_t st);
uint64_t pack_bytes(uint32_t fm, uint32_t R, uint32_t K);
int launch_pack(uint32_t fm, const uint8_t* W, uint64_t es, uint64_t rb, uint32_t R, uint32_t K, uint32_t ne,
                uint8_t* P, hipStream_t st);
int launch_combine(const _Float16* out, const float* spill, const uint32_t* inv, const float* wt, uint32_t nk, const float* shd,
                   const float* sgo, const float* x1, float* y, uint32_t dm, uint32_t T, hipStream_t st);
int launch_exp(const float* x, float* y, uint64_t n, hipStream_t st);
int launch_dequant(uint32_t fm, const uint8_t* W, uint64_t rb, uint32_t rows, uint32_t cols, float* out,
                   hipStream_t st);
