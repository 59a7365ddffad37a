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
#include "../../include/llb_moe_hip.h"
#include "moe_dev.h"
#include "moe_kernels.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define GM_BM 256  // slots a tile (an expert's slots split into tiles of this many)

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

// ---- the grouped GEMM. Block tile: BM = 256 slots x 128 weight rows (mode 0: 64 gate + 64 up
// features, mode 1: 128 features), K in steps of 64, eight waves of 64 x 64 (2 x 2 MFMA 32x32x16
// tiles; in mode 0 one wave's gate and up tiles cover the same 32 features, so the SwiGLU epilogue
// pairs them in registers). A tile of 256 slots holds a whole expert at prefill sizes, so each weight
// tile is read once. LDS holds two stages of A and B (f16, rows padded to 72 halves): while the
// MFMAs run on one stage, the next three tiles' A rows and raw weight half-spans are in flight into
// registers; after the MFMAs one tile is dequantized into the other stage. One barrier a k-tile.
#define G2_BK 64
#define G2_LD 72
#define G2_BN 128                                  // weight rows a tile
#define G2_STAGE ((GM_BM + G2_BN) * G2_LD)         // halves: A [256][72] then B [128][72]

// XCD-aware order: the hardware deals block b to XCD b % 8, so block b takes m-tile
// 8 ((b / 8) / NT) + b % 8 and feature tile (b / 8) % NT: an m-tile's NT feature tiles all run on
// one XCD and read its activation rows from that XCD's L2 (1-D grid, 8 NT ceil(tiles / 8) blocks)
template <u32 F, u32 MODE>
__global__ void __launch_bounds__(512) k_moe_gemm2(GemmArgs g, u32 NT) {
  extern __shared__ _Float16 lds[];
  const u32 bi = blockIdx.x >> 3, tile = 8 * (bi / NT) + (blockIdx.x & 7), ntile = bi % NT;
  u32 e, m0, base, M;
  if (g.tiles) {
    if (tile >= *g.ntiles) return;
    const u32 tv = g.tiles[tile];
    e = tv >> 16;
    m0 = (tv & 0xffffu) * GM_BM;
    base = g.off[e];
    M = g.off[e + 1] - base;
  } else {
    e = 0;
    m0 = tile * GM_BM;
    base = 0;
    M = g.M;
    if (m0 >= M) return;
  }
  constexpr u32 NF = MODE == 0 ? 64u : 128u;  // output features a block
  const u32 n0 = ntile * NF, tid = threadIdx.x, w = tid >> 6, l = tid & 63, wm = w >> 1, wn = w & 1;
  // A: 256 rows x 64 halves a k-tile, 16-byte chunks c = tid + 512 i (i < 4): row c / 8, chunk c % 8.
  // Buffer loads bounded by A's size: a row past the expert's slots gets an offset past the bound, so
  // its load returns zeros without touching memory, and every load stays unconditional (a load under a
  // branch makes the compiler wait for all of them)
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)g.A, (short)0, (int)(g.arows * g.K * 2u), 0x00020000);
  u32 aoff[4], src[4];
#pragma unroll
  for (u32 i = 0; i < 4; i++) src[i] = base + m0 + min((tid + 512 * i) >> 3, M - m0 - 1);  // a live slot
  if (MODE == 0 && g.xmap) {  // slot -> token row, the four reads in flight together
#pragma unroll
    for (u32 i = 0; i < 4; i++) src[i] = g.xmap[src[i]];
  }
#pragma unroll
  for (u32 i = 0; i < 4; i++) {
    const u32 c = tid + 512 * i, r = c >> 3;
    aoff[i] = m0 + r < M ? (src[i] * g.K + 8 * (c & 7)) * 2u : 0x80000000u;
  }
  // B: 128 rows x 64 columns a k-tile; thread: row tid / 4, span (tid / 2) % 2, half tid % 2
  const u32 br = tid >> 2, bs = (tid >> 1) & 1, bj = tid & 1;
  const u8* brow;
  if (MODE == 0) brow = (br < 64 ? g.W0 + (u64)(n0 + br) * g.rb : g.W1 + (u64)(n0 + br - 64) * g.rb) + (u64)e * g.es;
  else brow = g.W0 + (u64)e * g.es + (u64)(n0 + br) * g.rb;
  // a wave whose 64 rows are all past the expert's slots skips its MFMAs (wave-uniform)
  const bool live = m0 + 64 * wm < M;

  // three register slots keep k-tiles t + 2 .. t + 4 in flight while tile t is multiplied (slot of
  // tile u: u % 3); compile-time slot choice keeps them in registers
  struct Slot {
    uint4 a[4];
    Half<F> h;
  };
  Slot s0, s1, s2;
  const u32 nk = g.K / G2_BK;
  auto load = [&](Slot& s, u32 t) {
    const u32 k0 = min(t, nk - 1) * G2_BK;  // past the end: a repeat of the last tile, never stored
#pragma unroll
    for (u32 i = 0; i < 4; i++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(arsrc, (int)(aoff[i] + 2 * k0), 0, 0);
      s.a[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    s.h.ld(brow, k0 + 32 * bs, bj);
  };
  auto store = [&](const Slot& s, u32 t) {
    _Float16* As = lds + (t & 1) * G2_STAGE;
    _Float16* Bs = As + GM_BM * G2_LD;
    const u32 k0 = t * G2_BK;
#pragma unroll
    for (u32 i = 0; i < 4; i++) {
      const u32 c = tid + 512 * i;
      *(uint4*)(As + (c >> 3) * G2_LD + 8 * (c & 7)) = s.a[i];
    }
    u32 o[8];
    half_f16<F>(s.h, k0 + 32 * bs, bj, o);
    _Float16* d = Bs + br * G2_LD + 32 * bs + 16 * bj;
    *(uint4*)d = make_uint4(o[0], o[1], o[2], o[3]);
    *(uint4*)(d + 8) = make_uint4(o[4], o[5], o[6], o[7]);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (u32 a = 0; a < 2; a++)
#pragma unroll
    for (u32 b = 0; b < 2; b++)
#pragma unroll
      for (u32 i = 0; i < 16; i++) acc[a][b][i] = 0.0f;
  // B rows of this wave's two 32-column tiles
  const u32 bro0 = MODE == 0 ? 32 * wn : 64 * wn, bro1 = MODE == 0 ? 64 + 32 * wn : 64 * wn + 32;
  auto mma = [&](u32 t) {
    if (!live) return;
    const _Float16* As = lds + (t & 1) * G2_STAGE;
    const _Float16* Bs = As + GM_BM * G2_LD;
#pragma unroll
    for (u32 ks = 0; ks < G2_BK / 16; ks++) {
      const u32 ko = 16 * ks + 8 * (l >> 5);
      const h8 a0 = *(const h8*)(As + (64 * wm + (l & 31)) * G2_LD + ko);
      const h8 a1 = *(const h8*)(As + (64 * wm + 32 + (l & 31)) * G2_LD + ko);
      const h8 b0 = *(const h8*)(Bs + (bro0 + (l & 31)) * G2_LD + ko);
      const h8 b1 = *(const h8*)(Bs + (bro1 + (l & 31)) * G2_LD + ko);
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, acc[1][1], 0, 0, 0);
    }
  };
  // iteration t: multiply tile t, store tile t + 1 (its slot) into the other stage, refill that
  // slot with tile t + 4, one barrier. The steady-state loop runs while three tiles follow, so its
  // stores and loads are unconditional; the last one to three iterations only multiply and store.
  auto step = [&](Slot& s, u32 t) {
    mma(t);
    store(s, t + 1);
    load(s, t + 4);
    __syncthreads();
  };
  auto tail = [&](const Slot& s, u32 t) {
    mma(t);
    if (t + 1 < nk) store(s, t + 1);
    __syncthreads();
  };
  load(s0, 0);
  load(s1, 1);
  load(s2, 2);
  store(s0, 0);
  load(s0, 3);
  __syncthreads();
  u32 t = 0;
  for (; t + 4 <= nk; t += 3) {
    step(s1, t);
    step(s2, t + 1);
    step(s0, t + 2);
  }
  // 1 .. 3 tiles left; their slots continue the rotation
  tail(s1, t);
  if (t + 1 < nk) tail(s2, t + 1);
  if (t + 2 < nk) tail(s0, t + 2);
  // epilogue: acc[a][b][i] is row 64 wm + 32 a + 8 (i / 4) + 4 (l / 32) + i % 4 of the tile,
  // column l % 32 of B tile b
#pragma unroll
  for (u32 a = 0; a < 2; a++)
#pragma unroll
    for (u32 i = 0; i < 16; i++) {
      const u32 row = 64 * wm + 32 * a + 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
      if (m0 + row >= M) continue;
      const u64 s = base + m0 + row;
      if (MODE == 0) {
        const float gv = acc[a][0][i], uv = acc[a][1][i];
        ((_Float16*)g.out)[s * g.N + n0 + 32 * wn + (l & 31)] = (_Float16)(gv / (1.0f + __expf(-gv)) * uv);
      } else {
#pragma unroll
        for (u32 b = 0; b < 2; b++) ((float*)g.out)[s * g.N + n0 + 64 * wn + 32 * b + (l & 31)] = acc[a][b][i];
      }
    }
}

// y[t][r] = (sum_j, rank order, wt[t][j] out[inv[t nk + j]][r]) + sgo[t] shd[t][r] + x1[t][r]
__global__ void __launch_bounds__(256) k_combine(const float* __restrict__ out, const u32* __restrict__ inv,
                                                 const float* __restrict__ wt, u32 nk, const float* __restrict__ shd,
                                                 const float* __restrict__ sgo, const float* __restrict__ x1,
                                                 float* __restrict__ y, u32 dm) {
  // four outputs a thread (dm % 4 == 0); the token's slot rows and weights read once into LDS; the
  // slot values of up to eight ranks in flight at once, summed in rank order
  __shared__ u32 srow[64];
  __shared__ float swt[64];
  const u32 t = blockIdx.y, r = 4 * (blockIdx.x * 256 + threadIdx.x);
  if (threadIdx.x < nk) {
    srow[threadIdx.x] = inv[(u64)t * nk + threadIdx.x];
    swt[threadIdx.x] = wt[(u64)t * nk + threadIdx.x];
  }
  __syncthreads();
  if (r >= dm) return;
  float4 mo = make_float4(0.f, 0.f, 0.f, 0.f);
  for (u32 j0 = 0; j0 < nk; j0 += 8) {
    float4 v[8];
#pragma unroll
    for (u32 j = 0; j < 8; j++)
      if (j0 + j < nk) v[j] = *(const float4*)(out + (u64)srow[j0 + j] * dm + r);
#pragma unroll
    for (u32 j = 0; j < 8; j++) {
      if (j0 + j >= nk) break;
      const float w = swt[j0 + j];
      if (j0 + j == 0) {
        mo = make_float4(v[j].x * w, v[j].y * w, v[j].z * w, v[j].w * w);
      } else {
        mo.x = mo.x + v[j].x * w; mo.y = mo.y + v[j].y * w; mo.z = mo.z + v[j].z * w; mo.w = mo.w + v[j].w * w;
      }
    }
  }
  const u64 o = (u64)t * dm + r;
  const float4 res = x1 ? *(const float4*)(x1 + o) : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 yv;
  if (shd) {
    const float4 s = *(const float4*)(shd + o);
    const float g = sgo[t];
    yv = make_float4((mo.x + s.x * g) + res.x, (mo.y + s.y * g) + res.y, (mo.z + s.z * g) + res.z, (mo.w + s.w * g) + res.w);
  } else {
    yv = make_float4(mo.x + res.x, mo.y + res.y, mo.z + res.z, mo.w + res.w);
  }
  *(float4*)(y + o) = yv;
}

// ---------------------------------------------------------------- launchers

template <u32 F, u32 MODE> static void gemm2_go(const GemmArgs& g, dim3 grid, size_t sm, hipStream_t st) {
  static bool set = false;
  if (!set) {
    (void)hipFuncSetAttribute((const void*)k_moe_gemm2<F, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
    set = true;
  }
  LAUNCH_K((k_moe_gemm2<F, MODE>), grid, dim3(512), sm, st, g, g.N / (MODE == 0 ? 64u : 128u));
}

int launch_moe_gemm(const GemmArgs& g, u32 fm, u32 mode, u32 grid_y, hipStream_t st) {
  const u32 nf = mode == 0 ? 64u : 128u;
  // A's buffer loads take 32-bit offsets below 2^31 (dead rows use 2^31)
  if (g.K % G2_BK || g.N % nf || fm == FM_F32 || (u64)g.arows * g.K * 2 >= (1ull << 31)) return -1;
  const dim3 grid(8 * (g.N / nf) * ((grid_y + 7) / 8));
  const size_t sm = (size_t)2 * G2_STAGE * 2;
#define G2_L(F) \
  if (fm == F) { \
    if (mode == 0) gemm2_go<F, 0>(g, grid, sm, st); \
    else gemm2_go<F, 1>(g, grid, sm, st); \
    return 0; \
  }
  G2_L(FM_Q8_0) G2_L(FM_Q4_K) G2_L(FM_Q6_K) G2_L(FM_Q5_K)
#undef G2_L
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
  if (dm % 4 || nk > 64) return -1;
  hipLaunchKernelGGL(k_combine, dim3((dm / 4 + 255) / 256, T), dim3(256), 0, st, out, inv, wt, nk, shd, sgo, x1, y, dm);
  return 0;
}
u32 gemm_bm() { return GM_BM; }
