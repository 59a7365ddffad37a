// moe_gemm.hip -- the grouped-GEMM tier for many tokens (prefill, large batches): the expert products
// on CDNA4 MFMA (v_mfma_f32_32x32x16_f16, f32 accumulate). The reference's fast prefill
// (host/llb_pf.h:286-389, pfx_* on int8 mma.sync) groups slots by expert and runs one GEMM per
// expert over its slots; so does this. Weight tiles are dequantized with the exact tier's decoders
// (a 32-column span at a time) and rounded to f16 into LDS; activations are f16. Tolerance class.
//
// Per expert e (slots off[e] .. off[e+1], rows of the slot-ordered activations):
//   gate / up   act[s][n] = silu(G_e[n] . x_s) (U_e[n] . x_s), x_s = h2 of token xmap[s]
//   down        out[s][r] = D_e[r] . act[s]
// then y[t] = (sum over ranks j, in order, wt[t][j] out[inv[t nk + j]]) + sgo[t] shd[t] + x1[t].
// The shared expert is the same two GEMMs over all T tokens (one "expert", identity map).
//
// Block tile: BM = 128 slots x BN = 64 outputs (x2 matrices for gate / up), K in steps of BK = 128.
// Wave w computes rows 32 w .. 32 w + 31 of the tile, both 32-column halves, each matrix.
#include "../../include/llb_moe_hip.h"
#include "moe_dev.h"
#include "moe_kernels.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define GM_BM 128
#define GM_BN 64
#define GM_BK 128
#define GM_LD (GM_BK + 8)  // halves per LDS row: the pad spreads a wave's 16-byte row reads over banks

// f32 rows -> f16 rows (the activations' one conversion)
__global__ void __launch_bounds__(256) k_to_f16(const float* __restrict__ x, _Float16* __restrict__ y, u64 n) {
  const u64 i = ((u64)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 3 < n) {
    const float4 v = *(const float4*)(x + i);
    y[i] = (_Float16)v.x; y[i + 1] = (_Float16)v.y; y[i + 2] = (_Float16)v.z; y[i + 3] = (_Float16)v.w;
  } else {
    for (u64 k = i; k < n; k++) y[k] = (_Float16)x[k];
  }
}

// the tile list: for each expert, ceil(M_e / BM) tiles (e << 16 | tile index); count in *ntiles
__global__ void __launch_bounds__(1024) k_tiles(const u32* __restrict__ off, u32 ne, u32* __restrict__ tiles,
                                                u32* __restrict__ ntiles) {
  __shared__ u32 part[1024];
  const u32 t = threadIdx.x;
  // experts t, t + 1024, ... (ne may exceed 1024): each thread counts its experts' tiles
  u32 mine = 0;
  for (u32 e = t; e < ne; e += 1024) mine += (off[e + 1] - off[e] + GM_BM - 1) / GM_BM;
  part[t] = mine;
  __syncthreads();
  for (u32 s = 1; s < 1024; s <<= 1) {  // inclusive scan
    const u32 v = t >= s ? part[t - s] : 0u;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  u32 at = part[t] - mine;
  for (u32 e = t; e < ne; e += 1024) {
    const u32 nt = (off[e + 1] - off[e] + GM_BM - 1) / GM_BM;
    for (u32 k = 0; k < nt; k++) tiles[at++] = e << 16 | k;
  }
  if (t == 1023) *ntiles = part[1023];
}

// MODE 0: gate / up with the SwiGLU epilogue, A = f16 rows of x gathered through xmap, out f16 act.
// MODE 1: down, A = f16 act rows (slot order), out f32.
template <u32 F, u32 MODE>
__global__ void __launch_bounds__(256) k_moe_gemm(GemmArgs g) {
  extern __shared__ _Float16 lds[];
  constexpr u32 NB = MODE == 0 ? 2u : 1u;
  _Float16* As = lds;                      // [BM][LD]
  _Float16* Bs = lds + GM_BM * GM_LD;      // [NB][BN][LD]
  u32 e, m0, base, M;
  if (g.tiles) {
    if (blockIdx.y >= *g.ntiles) return;
    const u32 tv = g.tiles[blockIdx.y];
    e = tv >> 16;
    m0 = (tv & 0xffffu) * GM_BM;
    base = g.off[e];
    M = g.off[e + 1] - base;
  } else {
    e = 0;
    m0 = blockIdx.y * GM_BM;
    base = 0;
    M = g.M;
    if (m0 >= M) return;
  }
  const u32 n0 = blockIdx.x * GM_BN, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const u8* W0 = g.W0 + (u64)e * g.es;
  const u8* W1 = MODE == 0 ? g.W1 + (u64)e * g.es : nullptr;
  f32x16 acc[NB][2];
#pragma unroll
  for (u32 b = 0; b < NB; b++)
#pragma unroll
    for (u32 h = 0; h < 2; h++)
#pragma unroll
      for (u32 i = 0; i < 16; i++) acc[b][h][i] = 0.0f;

  for (u32 k0 = 0; k0 < g.K; k0 += GM_BK) {
    // A: BM rows x BK halves, 16-byte chunks (8 halves): 2048 chunks, 8 a thread
#pragma unroll
    for (u32 q = 0; q < GM_BM * GM_BK / 8 / 256; q++) {
      const u32 c = tid + 256 * q, r = c / (GM_BK / 8), kc = c % (GM_BK / 8);
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m0 + r < M) {
        const u64 s = base + m0 + r;
        const u64 src = MODE == 0 ? (g.xmap ? (u64)g.xmap[s] : s) : s;
        v = *(const uint4*)(g.A + src * g.K + k0 + 8 * kc);
      }
      *(uint4*)(As + r * GM_LD + 8 * kc) = v;
    }
    // B: NB x BN rows x BK columns of weights, a 32-column span a task
    for (u32 it = tid; it < NB * GM_BN * (GM_BK / 32); it += 256) {
      const u32 b = it / (GM_BN * (GM_BK / 32)), rr = (it / (GM_BK / 32)) % GM_BN, sp = it % (GM_BK / 32);
      float wv[32];
      Span<F>::w((b == 0 ? W0 : W1) + (u64)(n0 + rr) * g.rb, k0 + 32 * sp, wv);
      _Float16* dst = Bs + (b * GM_BN + rr) * GM_LD + 32 * sp;
#pragma unroll
      for (u32 q = 0; q < 4; q++) {
        h8 hv;
#pragma unroll
        for (u32 i = 0; i < 8; i++) hv[i] = (_Float16)wv[8 * q + i];
        *(h8*)(dst + 8 * q) = hv;
      }
    }
    __syncthreads();
#pragma unroll
    for (u32 ks = 0; ks < GM_BK / 16; ks++) {
      const h8 a = *(const h8*)(As + (32 * w + (l & 31)) * GM_LD + 16 * ks + 8 * (l >> 5));
#pragma unroll
      for (u32 b = 0; b < NB; b++)
#pragma unroll
        for (u32 h = 0; h < 2; h++) {
          const h8 bv = *(const h8*)(Bs + (b * GM_BN + 32 * h + (l & 31)) * GM_LD + 16 * ks + 8 * (l >> 5));
          acc[b][h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bv, acc[b][h], 0, 0, 0);
        }
    }
    __syncthreads();
  }
  // epilogue: acc[..][i] is row 8 (i / 4) + 4 (l / 32) + i % 4 of the wave's 32, column l % 32
#pragma unroll
  for (u32 h = 0; h < 2; h++)
#pragma unroll
    for (u32 i = 0; i < 16; i++) {
      const u32 row = 32 * w + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3), col = n0 + 32 * h + (l & 31);
      if (m0 + row >= M) continue;
      const u64 s = base + m0 + row;
      if (MODE == 0) {
        const float gv = acc[0][h][i], uv = acc[NB - 1][h][i];
        ((_Float16*)g.out)[s * g.N + col] = (_Float16)(gv / (1.0f + __expf(-gv)) * uv);
      } else {
        ((float*)g.out)[s * g.N + col] = acc[0][h][i];
      }
    }
}

// y[t][r] = (sum_j, rank order, wt[t][j] out[inv[t nk + j]][r]) + sgo[t] shd[t][r] + x1[t][r]
__global__ void __launch_bounds__(256) k_combine(const float* __restrict__ out, const u32* __restrict__ inv,
                                                 const float* __restrict__ wt, u32 nk, const float* __restrict__ shd,
                                                 const float* __restrict__ sgo, const float* __restrict__ x1,
                                                 float* __restrict__ y, u32 dm) {
  const u32 t = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
  if (r >= dm) return;
  float mo = 0.0f;
  for (u32 j = 0; j < nk; j++) {
    const float v = out[(u64)inv[(u64)t * nk + j] * dm + r];
    mo = j == 0 ? v * wt[(u64)t * nk] : mo + v * wt[(u64)t * nk + j];
  }
  const u64 o = (u64)t * dm + r;
  const float res = x1 ? x1[o] : 0.0f;
  y[o] = shd ? (mo + shd[o] * sgo[t]) + res : mo + res;
}

// ---------------------------------------------------------------- launchers

size_t gemm_lds(u32 mode) { return ((size_t)GM_BM * GM_LD + (size_t)(mode == 0 ? 2 : 1) * GM_BN * GM_LD) * 2; }

// more than 64 KiB of dynamic LDS has to be allowed per kernel (gfx950 has 160 KiB a CU)
template <u32 F, u32 MODE> static void gemm_go(const GemmArgs& g, dim3 grid, size_t sm, hipStream_t st) {
  static bool set = false;
  if (!set) {
    (void)hipFuncSetAttribute((const void*)k_moe_gemm<F, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
    set = true;
  }
  hipLaunchKernelGGL((k_moe_gemm<F, MODE>), grid, dim3(256), sm, st, g);
}

int launch_moe_gemm(const GemmArgs& g, u32 fm, u32 mode, u32 grid_y, hipStream_t st) {
  if (g.K % GM_BK || g.N % GM_BN) return -1;
  const dim3 grid(g.N / GM_BN, grid_y);
  const size_t sm = gemm_lds(mode);
#define GM_L(F) \
  if (fm == F) { \
    if (mode == 0) gemm_go<F, 0>(g, grid, sm, st); \
    else gemm_go<F, 1>(g, grid, sm, st); \
    return 0; \
  }
  GM_L(FM_Q8_0) GM_L(FM_Q4_K) GM_L(FM_Q6_K) GM_L(FM_Q5_K)
#undef GM_L
  return -1;
}

int launch_to_f16(const float* x, _Float16* y, u64 n, hipStream_t st) {
  hipLaunchKernelGGL(k_to_f16, dim3((u32)((n / 4 + 255) / 256 + 1)), dim3(256), 0, st, x, y, n);
  return 0;
}
int launch_tiles(const u32* off, u32 ne, u32* tiles, u32* ntiles, hipStream_t st) {
  hipLaunchKernelGGL(k_tiles, dim3(1), dim3(1024), 0, st, off, ne, tiles, ntiles);
  return 0;
}
int launch_combine(const float* out, const u32* inv, const float* wt, u32 nk, const float* shd, const float* sgo,
                   const float* x1, float* y, u32 dm, u32 T, hipStream_t st) {
  hipLaunchKernelGGL(k_combine, dim3((dm + 255) / 256, T), dim3(256), 0, st, out, inv, wt, nk, shd, sgo, x1, y, dm);
  return 0;
}
u32 gemm_bm() { return GM_BM; }
