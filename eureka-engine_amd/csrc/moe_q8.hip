// moe_q8.hip -- the q8 tier (the reference's LLB_MOE_DP4A decode tier and LLB_PREFILL=fast
// numerics, host/llb_pf.cuh:447-620): expert products on q8_1 activations. A 32-column block's
// dot is an int8 dot product (v_dot4_i32_i8) scaled in f32: Q4_K / Q5_K (d sc) xd acc - (dmin m) xs,
// Q6_K d xd (sc0 a0 + sc1 a1), Q8_0 d xd acc. Routing stays the exact tier's. Tolerance class.
// Also the dispatch permutation (llb_mx_group) and the q8_1 quantizer (pf_q8x).
#include <stdlib.h>

#include "../../include/llb_moe_hip.h"
#include "moe_dev.h"
#include <atomic>
#include "moe_kernels.h"
#include "moe_q8dot.h"

// ---------------------------------------------------------------- q8_1 (pf_q8x)

// one thread an element; lanes 32 h .. 32 h + 31 of a wave form one block: d = amax / 127,
// q = round(x / d) (0 when amax = 0), s = sum x
__global__ void __launch_bounds__(256) k_q8_1(const float* __restrict__ x, u32 n, signed char* __restrict__ q,
                                              float2* __restrict__ ds) {
  const u64 i = (u64)blockIdx.x * 256 + threadIdx.x;
  float d, sum;
  const signed char c = q8_1_lane(i < n ? x[i] : 0.0f, d, sum);
  if (i < n) q[i] = c;
  if (i < n && (threadIdx.x & 31) == 0) ds[i >> 5] = make_float2(d, sum);
}

int launch_q8_1(const float* x, uint32_t n, int8_t* q, float2* ds, hipStream_t st) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_q8_1, dim3((n + 255) / 256), dim3(256), 0, st, x, n, (signed char*)q, ds);
  return 0;
}

// ---------------------------------------------------------------- dispatch (llb_mx_group)

// block e of ne: off[e] = #{slots with id < e}; then e's slots in ascending slot order, each
// wave's ballot giving a slot its rank: xmap[pos] = slot / nk, inv[slot] = pos. Deterministic.
// the dispatch permutation (llb_mx_group, host/llb_pf.cuh:774-817): slots of expert e in slot order.
// Block e; thread t scans its contiguous slots: ids below e (the expert's offset)
// and equal to e (its hits); an exclusive scan of the hits over the block gives each thread its first
// position, and it writes its hits in slot order -- the stable order, with one scan a block.
// Blocks past ne (when x16 is set) convert the activations to f16 for the grouped GEMM instead, 8
// values a thread (nx % 8 == 0): the two jobs are independent and share one launch.
__global__ void __launch_bounds__(256) k_group(const u32* __restrict__ ids, u32 n, u32 nk, u32 ne, u32* __restrict__ off,
                                               u32* __restrict__ xmap, u32* __restrict__ inv,
                                               const float* __restrict__ x, _Float16* __restrict__ x16, u64 nx) {
  __shared__ u32 wl[4], wh[4];
  if (blockIdx.x >= ne) {
    const u64 i = ((u64)(blockIdx.x - ne) * 256 + threadIdx.x) * 8;
    if (i < nx) {
      const float4 a = *(const float4*)(x + i), b = *(const float4*)(x + i + 4);
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
      const h8 v = {(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                    (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
      *(h8*)(x16 + i) = v;
    }
    return;
  }
  const u32 e = blockIdx.x, t = threadIdx.x, w = t >> 6, L = t & 63;
  // thread t scans the contiguous slots [t per, t per + per), per a multiple of 4 (16-byte loads)
  const u32 per = ((n + 255) / 256 + 3) & ~3u, i0 = min(t * per, n), i1 = min(i0 + per, n);
  // up to 64 slots a thread: all its ids in registers from one round of loads, reused by the scatter
  // below; a partial last quad holds ~0 past n (never an expert: it counts neither below nor at e)
  const bool reg = per <= 64 && ((uintptr_t)ids & 15) == 0;
  uint4 v[16];
  u32 lt = 0, hit = 0;
  if (reg) {
#pragma unroll
    for (u32 q = 0; q < 16; q++) {
      const u32 i = i0 + 4 * q;
      uint4 x = make_uint4(~0u, ~0u, ~0u, ~0u);
      if (4 * q < per && i < i1) {
        if (i + 4 <= i1) {
          x = *(const uint4*)(ids + i);
        } else {
          x.x = ids[i];
          if (i + 1 < i1) x.y = ids[i + 1];
          if (i + 2 < i1) x.z = ids[i + 2];
        }
      }
      v[q] = x;
    }
#pragma unroll
    for (u32 q = 0; q < 16; q++) {
      const uint4 x = v[q];
      lt += (x.x < e ? 1u : 0u) + (x.y < e ? 1u : 0u) + (x.z < e ? 1u : 0u) + (x.w < e ? 1u : 0u);
      hit += (x.x == e ? 1u : 0u) + (x.y == e ? 1u : 0u) + (x.z == e ? 1u : 0u) + (x.w == e ? 1u : 0u);
    }
  } else {
    for (u32 i = i0; i < i1; i++) {
      const u32 x = ids[i];
      lt += x < e ? 1u : 0u;
      hit += x == e ? 1u : 0u;
    }
  }
  // inclusive scan of hit across the wave, sum of lt
  u32 inc = hit, lsum = lt;
#pragma unroll
  for (u32 m = 1; m < 64; m <<= 1) {
    const u32 o = __shfl_up(inc, m, 64);
    if (L >= m) inc += o;
    lsum += __shfl_xor(lsum, m, 64);
  }
  if (L == 63) wh[w] = inc;
  if (L == 0) wl[w] = lsum;
  __syncthreads();
  const u32 base = wl[0] + wl[1] + wl[2] + wl[3];
  u32 pos = base + inc - hit;
  for (u32 k = 0; k < w; k++) pos += wh[k];
  if (t == 0) {
    off[e] = base;
    if (e + 1 == ne) off[ne] = n;
  }
  if (hit && reg) {
#pragma unroll
    for (u32 q = 0; q < 16; q++) {
      const u32 xs[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
      for (u32 c = 0; c < 4; c++) {
        if (xs[c] == e) {  // only slots below i1 can hold e
          const u32 i = i0 + 4 * q + c;
          xmap[pos] = i / nk;
          inv[i] = pos;
          pos++;
        }
      }
    }
  } else if (hit) {
    for (u32 i = i0; i < i1; i++) {
      if (ids[i] == e) {
        xmap[pos] = i / nk;
        inv[i] = pos;
        pos++;
      }
    }
  }
}

// ---- the same permutation as a device histogram and prefix scan (two launches, O(n + nb ne) work)
//
// Slot i lives in block b = i / GS_SLOTS, wave w = (i % GS_SLOTS) / 256, round r = (i % 256) / 64, lane
// L = i % 64, so (b, w, r, L) ascending is slot order. k_group_count: within each round a wave gives every
// lane its rank among the round's lanes of the same expert (lanes below it, by ballot: one pass per
// distinct expert in the round, leader = the lowest lane left) plus the wave's running count of that expert
// (LDS, wave-private); after the four rounds the block turns its per-wave counts into per-wave exclusive
// prefixes, writes its per-expert totals cnt[b][e] and each slot's rank inside the block into inv[i].
// k_group_place: every block sums cnt over blocks for its experts (those before it, and all), scans the
// totals over experts (off[e] = slots with id < e), and places its slots: pos = off[e] + (slots of e in
// earlier blocks) + rank, xmap[pos] = i / nk, inv[i] = pos. Ids >= ne (never produced by routing) get no
// position, as in k_group. Blocks past nb convert the activations to f16 as k_group's do.
constexpr u32 GS_SLOTS = 1024;
__global__ void __launch_bounds__(256) k_group_count(const u32* __restrict__ ids, u32 n, u32 ne, u32* __restrict__ cnt,
                                                     u32* __restrict__ inv) {
  extern __shared__ u32 wc[];  // [4][ne]
  const u32 t = threadIdx.x, L = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
  for (u32 i = t; i < 4 * ne; i += 256) wc[i] = 0u;
  __syncthreads();
  u32* mine = wc + w * ne;
  const u32 s0 = blockIdx.x * GS_SLOTS + w * 256;
  const u64 below = L ? (~0ull >> (64 - L)) : 0ull;  // lanes under this one
  u32 rk[4], ev[4];
#pragma unroll
  for (u32 r = 0; r < 4; r++) {
    const u32 i = s0 + 64 * r + L;
    const u32 e = i < n ? ids[i] : 0xFFFFFFFFu;
    const bool ok = e < ne;
    u64 act = __ballot(ok);
    u32 my = 0;
    while (act) {  // wave-uniform: one pass per distinct expert of the round
      const u32 ld = (u32)__builtin_ctzll(act);
      const u32 ee = (u32)__builtin_amdgcn_readlane((int)e, (int)ld);
      const bool same = ok && e == ee;
      const u64 m = __ballot(same);
      const u32 base = mine[ee];
      if (same) my = base + (u32)__builtin_popcountll(m & below);
      if (L == ld) mine[ee] = base + (u32)__builtin_popcountll(m);
      // the next pass (or round) may read this count: keep the LDS store ahead of it
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
      act &= ~m;
    }
    rk[r] = my;
    ev[r] = ok ? e : 0xFFFFFFFFu;
  }
  __syncthreads();
  for (u32 e = t; e < ne; e += 256) {
    const u32 a0 = wc[e], a1 = wc[ne + e], a2 = wc[2 * ne + e], a3 = wc[3 * ne + e];
    wc[e] = 0u;
    wc[ne + e] = a0;
    wc[2 * ne + e] = a0 + a1;
    wc[3 * ne + e] = a0 + a1 + a2;
    cnt[(u64)blockIdx.x * ne + e] = a0 + a1 + a2 + a3;
  }
  __syncthreads();
#pragma unroll
  for (u32 r = 0; r < 4; r++) {
    const u32 i = s0 + 64 * r + L;
    if (ev[r] != 0xFFFFFFFFu) inv[i] = mine[ev[r]] + rk[r];
  }
}

__global__ void __launch_bounds__(256) k_group_place(const u32* __restrict__ ids, u32 n, u32 nk, u32 ne, u32 nb,
                                                     const u32* __restrict__ cnt, u32* __restrict__ off,
                                                     u32* __restrict__ xmap, u32* __restrict__ inv,
                                                     const float* __restrict__ x, _Float16* __restrict__ x16, u64 nx) {
  __shared__ u32 base[1024];
  __shared__ u32 wsum[4];
  if (blockIdx.x >= nb) {
    const u64 i = ((u64)(blockIdx.x - nb) * 256 + threadIdx.x) * 8;
    if (i < nx) {
      const float4 a = *(const float4*)(x + i), b = *(const float4*)(x + i + 4);
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
      const h8 v = {(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                    (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
      *(h8*)(x16 + i) = v;
    }
    return;
  }
  const u32 t = threadIdx.x, L = t & 63, w = t >> 6, b = blockIdx.x;
  // thread t: experts 4 t .. 4 t + 3 (ne <= 1024), each summed over the blocks before this one and over all
  u32 tot[4], bef[4], own = 0;
#pragma unroll
  for (u32 j = 0; j < 4; j++) {
    const u32 e = 4 * t + j;
    u32 a = 0, c = 0;
    if (e < ne)
      for (u32 k = 0; k < nb; k++) {
        const u32 v = cnt[(u64)k * ne + e];
        a += k < b ? v : 0u;
        c += v;
      }
    bef[j] = a;
    tot[j] = c;
    own += c;
  }
  // exclusive scan of the threads' totals (expert order): within the wave, then the waves before
  u32 inc = own;
#pragma unroll
  for (u32 m = 1; m < 64; m <<= 1) {
    const u32 o = __shfl_up(inc, m, 64);
    if (L >= m) inc += o;
  }
  if (L == 63) wsum[w] = inc;
  __syncthreads();
  u32 pre = inc - own;
  for (u32 k = 0; k < w; k++) pre += wsum[k];
#pragma unroll
  for (u32 j = 0; j < 4; j++) {
    const u32 e = 4 * t + j;
    if (e < ne) {
      base[e] = pre + bef[j];
      if (b == 0) off[e] = pre;
    }
    pre += tot[j];
  }
  if (b == 0 && t == 0) off[ne] = n;
  __syncthreads();
  const u32 s0 = b * GS_SLOTS;
#pragma unroll
  for (u32 q = 0; q < 4; q++) {
    const u32 i = s0 + 256 * q + t;
    if (i < n) {
      const u32 e = ids[i];
      if (e < ne) {
        const u32 pos = base[e] + inv[i];
        inv[i] = pos;
        xmap[pos] = i / nk;
      }
    }
  }
}

// the permutation's choice: 0 k_group (per-expert scans), 1 the histogram + scan pair. Off (0) by default
// until the pair has run on the GPU.
static std::atomic<int> g_group_scan{0};
void moe_set_group_scan(bool on) { g_group_scan.store(on ? 1 : 0); }
bool moe_group_scan_enabled() { return g_group_scan.load() != 0; }
size_t group_cnt_bytes(uint32_t n, uint32_t ne) {
  return (size_t)((n + GS_SLOTS - 1) / GS_SLOTS) * ne * 4;
}

int launch_group(const uint32_t* ids, uint32_t n, uint32_t nk, uint32_t ne, uint32_t* off, uint32_t* xmap,
                 uint32_t* inv, const float* x, _Float16* x16, uint64_t nx, hipStream_t st, uint32_t* cnt) {
  if (x16 && nx % 8) return -1;
  const u64 nconv = x16 ? (nx + 2047) / 2048 : 0;
  if (cnt && n && ne <= 1024 && moe_group_scan_enabled()) {  // (no slots: k_group writes the all-zero offsets)
    const u32 nb = (n + GS_SLOTS - 1) / GS_SLOTS;
    if (nb + nconv > 0x7fffffffull) return -1;
    hipLaunchKernelGGL(k_group_count, dim3(nb), dim3(256), 4 * ne * 4, st, ids, n, ne, cnt, inv);
    hipLaunchKernelGGL(k_group_place, dim3((u32)(nb + nconv)), dim3(256), 0, st, ids, n, nk, ne, nb, cnt, off, xmap,
                       inv, x, x16, nx);
    return 0;
  }
  if (ne + nconv > 0x7fffffffull) return -1;
  hipLaunchKernelGGL(k_group, dim3((u32)(ne + nconv)), dim3(256), 0, st, ids, n, nk, ne, off, xmap, inv, x, x16, nx);
  return 0;
}

// ---------------------------------------------------------------- decode-shaped kernels (per slot)

// down + combine (llb_mx_dn + llb_mx_comb): rw rows of token blockIdx.y, tasks (j, r). With lq (few
// tokens) the block quantizes its token's act and shared activations to q8_1 in LDS itself -- the
// same q8_1_lane steps as k_q8_1, so the same bits -- instead of a launch of k_q8_1 before it.
__global__ void __launch_bounds__(256) k_dn_q8(Q8Args a, u32 lq) {
  extern __shared__ float4 dsm[];  // part [64]; with lq: aq [nk ef], sq [sf], ad [nk ef / 32], sd [sf / 32]
  float* part = (float*)dsm;
  const u32 t = blockIdx.y, nt = a.nk + (a.sf ? 1u : 0u);
  // act in LDS or in memory: separate call sites keep each pointer's address space (no flat loads)
  const u32 na = a.nk * a.ef;
  signed char* laq = (signed char*)(part + 64);
  signed char* lsq = laq + na;
  float2* lad = (float2*)(lsq + a.sf);
  float2* lsd = lad + na / 32;
  if (lq) {
    q8_1_block256<32>(a.act + (u64)t * na, na, laq, lad);
    if (a.sf) q8_1_block256<16>(a.sa + (u64)t * a.sf, a.sf, lsq, lsd);
    __syncthreads();
  }
  const u32 g = threadIdx.x >> 2, p = threadIdx.x & 3;
  if (g < a.rw * nt) {
    const u32 j = g / a.rw, rl = g % a.rw, r = blockIdx.x * a.rw + rl;
    if (r < a.dm) {
      float v;
      if (j < a.nk) {
        const u64 e = a.ids[(u64)t * a.nk + j];
        const u8* row = a.D + (e * a.dm + r) * a.rbd;
        if (lq) v = row_q8_fm(a.fd, row, a.ef, laq + (u64)j * a.ef, lad + (u64)j * (a.ef / 32), p);
        else v = row_q8_fm(a.fd, row, a.ef, a.aq + ((u64)t * a.nk + j) * a.ef, a.ad + ((u64)t * a.nk + j) * (a.ef / 32), p);
      } else {
        const u8* row = a.SD + (u64)r * a.rbs;
        if (lq) v = row_q8_fm(a.fsd, row, a.sf, lsq, lsd, p);
        else v = row_q8_fm(a.fsd, row, a.sf, a.sq + (u64)t * a.sf, a.sd2 + (u64)t * (a.sf / 32), p);
      }
      if (p == 0) part[g] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < a.rw) {
    const u32 r = blockIdx.x * a.rw + threadIdx.x;
    if (r < a.dm) {
      const float* wt = a.wt + (u64)t * a.nk;
      float mo = 0.0f;
      for (u32 j = 0; j < a.nk; j++) {
        const float v = part[j * a.rw + threadIdx.x];
        mo = j == 0 ? v * wt[0] : mo + v * wt[j];
      }
      const float res = a.x1 ? a.x1[(u64)t * a.dm + r] : 0.0f;
      a.y[(u64)t * a.dm + r] = a.sf ? (mo + part[a.nk * a.rw + threadIdx.x] * a.sgo[t]) + res : mo + res;
    }
  }
}

// ---------------------------------------------------------------- the q8 layer

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }
static uint64_t rbytes(uint32_t fm, uint32_t cols) {
  return fm == FM_Q8_0 ? (uint64_t)cols / 32 * 34 : fm == FM_Q4_K ? (uint64_t)cols / 256 * 144
       : fm == FM_Q6_K ? (uint64_t)cols / 256 * 210 : fm == FM_Q5_K ? (uint64_t)cols / 256 * 176 : 0;
}

// many tokens: the grouped GEMM path on int8 MFMA (moe_q8_gemm below)
#define Q8_GEMM_T 16u
struct Q8GemmLayout {
  size_t hq, hd, off, xmap, inv, gcnt, act, aq, ad, out, sa, sq, sd, shd, total;
};
static Q8GemmLayout q8_gemm_layout(const llb_moe_layer* L, uint32_t T) {
  Q8GemmLayout g;
  const size_t n = (size_t)T * L->nk;
  size_t o = 0;
  g.hq = o; o += al((size_t)T * L->dm);
  g.hd = o; o += al((size_t)T * L->dm / 32 * 8);
  g.off = o; o += al(((size_t)L->ne + 1) * 4);
  g.xmap = o; o += al(n * 4);
  g.inv = o; o += al(n * 4);
  g.gcnt = o; o += al(group_cnt_bytes((uint32_t)n, L->ne));
  g.act = o; o += al(n * L->ef * 4);
  g.aq = o; o += al(n * L->ef);
  g.ad = o; o += al(n * L->ef / 32 * 8);
  g.out = o; o += al(n * L->dm * 4);
  g.sa = o; o += al((size_t)T * L->sf * 4 + 4);
  g.sq = o; o += al((size_t)T * L->sf + 4);
  g.sd = o; o += al((size_t)T * L->sf / 32 * 8 + 8);
  g.shd = o; o += al((size_t)T * L->dm * 4);
  g.total = o;
  return g;
}
// The int8-MFMA path is switched by llb_moe_hip_set_q8_gemm (its initial state: LLB_MOE_Q8_GEMM=1 in the
// environment at load time, else off). It is off by default until it has run on the GPU: its first run
// faulted (its Q8_0 code loads read 4 bytes past the stack's last block, fixed since), and the fixed code
// has not run yet. Off, the q8 tier keeps its per-slot kernels at every T. The switch is read at scratch
// sizing and at each forward; a forward whose scratch was sized with the switch off and that runs with it
// on is refused by the forward's scratch check.
static std::atomic<int> g_q8_gemm{[] {
  const char* e = getenv("LLB_MOE_Q8_GEMM");
  return e && e[0] == '1' ? 1 : 0;
}()};
void moe_q8_set_gemm(bool on) { g_q8_gemm.store(on ? 1 : 0); }
bool moe_q8_gemm_enabled() { return g_q8_gemm.load() != 0; }
static bool q8_gemm_on() { return moe_q8_gemm_enabled(); }
static bool q8_gemm_ok(const llb_moe_layer* L, uint32_t T) {
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15;
  const uint32_t fd = L->fx >> 8 & 15;
  // launch_gemm_i8 takes K-quant rows of whole 256-column super-blocks only (down: K = ef; shared down: sf)
  const bool kd = fd == FM_Q8_0 || L->ef % 256 == 0, ks = !L->sf || L->fsd == FM_Q8_0 || L->sf % 256 == 0;
  return q8_gemm_on() && T >= Q8_GEMM_T && fg == fu && (!L->sf || L->fsg == L->fsu) && L->ef % 128 == 0 && L->sf % 128 == 0 &&
         L->dm % 256 == 0 && L->ne <= 1024 && kd && ks;
}
size_t moe_q8_scratch(const llb_moe_layer* L, uint32_t T) {
  const size_t n = (size_t)T * L->nk;
  const size_t gemv = al((size_t)T * L->dm) + al((size_t)T * L->dm / 32 * 8) + al(n * L->ef * 4) + al(n * L->ef) +
                      al(n * L->ef / 32 * 8) + al((size_t)T * L->sf * 4 + 4) + al((size_t)T * L->sf + 4) +
                      al((size_t)T * L->sf / 32 * 8 + 8);
  const size_t gm = q8_gemm_ok(L, T) ? q8_gemm_layout(L, T).total : 0;
  return gemv > gm ? gemv : gm;
}

// the q8 tier for many tokens: x to q8_1; the slots grouped by expert; the gate / up GEMM (int8 MFMA,
// SwiGLU in the epilogue); act to q8_1; the down GEMM; the shared expert as one more "expert" over the T
// tokens; the rank-order combine with the shared gate and the residual
static int moe_q8_gemm(const llb_moe_layer* L, uint32_t T, const float* h2, const float* x1, float* y,
                       const uint32_t* ids, const float* wt, const float* sgo, uint8_t* sc, hipStream_t st) {
  const Q8GemmLayout q = q8_gemm_layout(L, T);
  const uint32_t fg = L->fx & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  const uint32_t n = T * L->nk;
  int8_t* hq = (int8_t*)(sc + q.hq);
  float2* hd = (float2*)(sc + q.hd);
  uint32_t* off = (uint32_t*)(sc + q.off);
  uint32_t* xmap = (uint32_t*)(sc + q.xmap);
  uint32_t* inv = (uint32_t*)(sc + q.inv);
  float* act = (float*)(sc + q.act);
  int8_t* aq = (int8_t*)(sc + q.aq);
  float2* ad = (float2*)(sc + q.ad);
  float* out = (float*)(sc + q.out);
  const uint64_t rbg = rbytes(fg, L->dm), rbd = rbytes(fd, L->ef);
  stage_begin(ST_Q8X);
  int rc = launch_q8_1(h2, T * L->dm, hq, hd, st);
  if (!rc) rc = launch_group(ids, n, L->nk, L->ne, off, xmap, inv, nullptr, nullptr, 0, st, (uint32_t*)(sc + q.gcnt));
  stage_end(ST_Q8X);
  if (rc) return rc;
  const uint32_t maxt = n / gemm_bm() + L->ne + 1;  // >= sum over experts of ceil(M_e / 64)
  GemmQ8Args g{};
  g.W0 = (const uint8_t*)(uintptr_t)L->G;
  g.W1 = fz ? g.W0 + (uint64_t)L->ef * rbg : (const uint8_t*)(uintptr_t)L->U;
  g.es = (uint64_t)(fz ? 2 : 1) * L->ef * rbg;
  g.rb = rbg;
  g.K = L->dm;
  g.N = L->ef;
  g.A = hq;
  g.Ad = hd;
  g.xmap = xmap;
  g.off = off;
  g.ne = L->ne;
  g.out = act;
  stage_begin(ST_GU);
  rc = launch_gemm_i8(g, fg, 0, maxt, st);
  stage_end(ST_GU);
  if (rc) return rc;
  if ((rc = launch_q8_1(act, n * L->ef, aq, ad, st))) return rc;
  GemmQ8Args d{};
  d.W0 = (const uint8_t*)(uintptr_t)L->D;
  d.es = (uint64_t)L->dm * rbd;
  d.rb = rbd;
  d.K = L->ef;
  d.N = L->dm;
  d.A = aq;
  d.Ad = ad;
  d.off = off;
  d.ne = L->ne;
  d.out = out;
  stage_begin(ST_DN);
  rc = launch_gemm_i8(d, fd, 1, maxt, st);
  stage_end(ST_DN);
  if (rc) return rc;
  const float* shd = nullptr;
  if (L->sf) {
    float* sa = (float*)(sc + q.sa);
    int8_t* sq = (int8_t*)(sc + q.sq);
    float2* sd = (float2*)(sc + q.sd);
    const uint32_t mt = (T + gemm_bm() - 1) / gemm_bm();
    GemmQ8Args s{};
    s.W0 = (const uint8_t*)(uintptr_t)L->SG;
    s.W1 = (const uint8_t*)(uintptr_t)L->SU;
    s.rb = rbytes(L->fsg, L->dm);
    s.K = L->dm;
    s.N = L->sf;
    s.M = T;
    s.A = hq;
    s.Ad = hd;
    s.out = sa;
    if ((rc = launch_gemm_i8(s, L->fsg, 0, mt, st))) return rc;
    if ((rc = launch_q8_1(sa, T * L->sf, sq, sd, st))) return rc;
    GemmQ8Args sd2{};
    sd2.W0 = (const uint8_t*)(uintptr_t)L->SD;
    sd2.rb = rbytes(L->fsd, L->sf);
    sd2.K = L->sf;
    sd2.N = L->dm;
    sd2.M = T;
    sd2.A = sq;
    sd2.Ad = sd;
    sd2.out = (float*)(sc + q.shd);
    if ((rc = launch_gemm_i8(sd2, L->fsd, 1, mt, st))) return rc;
    shd = sd2.out;
  }
  return launch_combine_f32(out, inv, wt, L->nk, shd, sgo, x1, y, L->dm, T, st);
}

// few tokens: each kernel quantizes the activations it reads in LDS (no q8_1 launches); more: the
// q8_1 launches, once for all blocks
#define Q8_LOCAL_T 8u

int moe_q8_forward(const llb_moe_layer* L, uint32_t T, const float* h2, const float* x1, float* y, const uint32_t* ids,
                   const float* wt, const float* sgo, const TopkArgs* tk, uint8_t* sc, hipStream_t st) {
  if (!tk && q8_gemm_ok(L, T)) return moe_q8_gemm(L, T, h2, x1, y, ids, wt, sgo, sc, st);
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  Q8Args a{};
  const size_t n = (size_t)T * L->nk;
  size_t o = 0;
  a.hq = (const int8_t*)(sc + o); o += al((size_t)T * L->dm);
  a.hd = (const float2*)(sc + o); o += al((size_t)T * L->dm / 32 * 8);
  a.act = (float*)(sc + o); o += al(n * L->ef * 4);
  a.aq = (int8_t*)(sc + o); o += al(n * L->ef);
  a.ad = (float2*)(sc + o); o += al(n * L->ef / 32 * 8);
  a.sa = (float*)(sc + o); o += al((size_t)T * L->sf * 4 + 4);
  a.sq = (int8_t*)(sc + o); o += al((size_t)T * L->sf + 4);
  a.sd2 = (float2*)(sc + o);
  a.rbg = rbytes(fg, L->dm);
  a.rbu = rbytes(fu, L->dm);
  a.rbd = rbytes(fd, L->ef);
  a.es = (uint64_t)(fz ? 2 : 1) * L->ef * a.rbg;
  a.G = (const uint8_t*)(uintptr_t)L->G;
  a.U = fz ? a.G + (uint64_t)L->ef * a.rbg : (const uint8_t*)(uintptr_t)L->U;
  a.D = (const uint8_t*)(uintptr_t)L->D;
  a.SG = (const uint8_t*)(uintptr_t)L->SG;
  a.SU = (const uint8_t*)(uintptr_t)L->SU;
  a.SD = (const uint8_t*)(uintptr_t)L->SD;
  a.rbsg = L->sf ? rbytes(L->fsg, L->dm) : 0;
  a.rbsu = L->sf ? rbytes(L->fsu, L->dm) : 0;
  a.rbs = L->sf ? rbytes(L->fsd, L->sf) : 0;
  a.fg = fg; a.fu = fu; a.fd = fd; a.fsg = L->fsg; a.fsu = L->fsu; a.fsd = L->fsd;
  a.dm = L->dm; a.ef = L->ef; a.nk = L->nk; a.sf = L->sf;
  a.rw = 64 / (L->nk + (L->sf ? 1 : 0));
  a.ids = ids;
  a.wt = wt;
  a.x1 = x1;
  a.y = y;
  a.sgo = sgo;
  // (the in-LDS quantizers hold 16 / 32 values a thread: dm, sf <= 4096, nk ef <= 8192)
  const bool lq = T <= Q8_LOCAL_T && L->dm <= 4096 && (size_t)L->nk * L->ef <= 8192 && L->sf <= 4096;
  // top-k inside the gate / up launch takes one token
  if (tk && (T != 1 || !lq)) return -1;
  if (!lq) {
    stage_begin(ST_Q8X);
    launch_q8_1(h2, T * L->dm, (int8_t*)a.hq, (float2*)a.hd, st);
    stage_end(ST_Q8X);
  }
  a.h2 = h2;
  stage_begin(ST_GU);
  int rc = launch_gu_q8(a, tk, (u32)n, T, lq, st);
  stage_end(ST_GU);
  if (rc) return rc;
  if (!lq) {
    launch_q8_1(a.act, (uint32_t)(n * L->ef), a.aq, a.ad, st);
    if (L->sf) launch_q8_1(a.sa, T * L->sf, a.sq, a.sd2, st);
  }
  const size_t lsm = 256 + (lq ? (size_t)L->nk * L->ef * 5 / 4 + (size_t)L->sf * 5 / 4 : 0);
  if (lsm > 65536) return -1;
  stage_begin(ST_DN);
  LAUNCH_K(k_dn_q8, dim3((L->dm + a.rw - 1) / a.rw, T), dim3(256), lsm, st, a, (u32)lq);
  stage_end(ST_DN);
  return 0;
}

// ---------------------------------------------------------------- zero fill (llb_zero)

// bytes [p, p + n) to zero by vector stores: the 16-byte-aligned body as uint4, the unaligned head and
// tail as bytes. A kernel, not a memset, so that a graph capture records a kernel node (memset nodes have
// given wrong results on replay). Grid-stride over the body, every store inside [p, p + n).
__global__ void __launch_bounds__(256) k_zero(u8* __restrict__ p, u64 n) {
  const u64 a = (u64)(uintptr_t)p, b0 = ((a + 15) & ~15ull) - a;  // head bytes before the aligned body
  const u64 head = b0 < n ? b0 : n, body = (n - head) / 16, tail0 = head + 16 * body;
  const u64 i0 = (u64)blockIdx.x * 256 + threadIdx.x, step = (u64)gridDim.x * 256;
  for (u64 i = i0; i < body; i += step) *(uint4*)(p + head + 16 * i) = make_uint4(0u, 0u, 0u, 0u);
  if (i0 < head) p[i0] = 0;
  if (i0 < n - tail0) p[tail0 + i0] = 0;
}
int launch_zero(void* p, uint64_t n, hipStream_t st) {
  if (n == 0) return 0;
  const u64 units = (n + 15) / 16, blocks = (units + 255) / 256;
  hipLaunchKernelGGL(k_zero, dim3((u32)(blocks < 4096 ? (blocks ? blocks : 1) : 4096)), dim3(256), 0, st, (u8*)p, (u64)n);
  return 0;
}

// ---------------------------------------------------------------- a bounded stall (timing aid)

__global__ void k_spin(u64 ticks) {
  const u64 t0 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}
int launch_spin(uint32_t us, hipStream_t st) {
  hipLaunchKernelGGL(k_spin, dim3(1), dim3(64), 0, st, (u64)us * 100u);
  return 0;
}
