// moe_exact.hip -- the exact tier of the MoE FFN on gfx950: f32 activations, f32 dequant, each
// float op rounded once in the reference's order, so the outputs are the bits of the reference's
// exact CUDA kernels (llb_warp / kp_pair router and shared gate-up, llb_moe_topk, llb_moe_gu,
// llb_moe_dn; tools/remap.patch:116-171, tools/payload-kpair.patch, tools/payload-moeany.patch:
// 311-594) and of the CPU oracle that restates them.
//
// Two dot orders, both re-mapped onto 64-wide waves:
//   tree    (router, shared gate / up): 2^cdepth group leaves (a group = 4 columns), balanced
//           pairwise tree. A whole wave takes a row: lane L holds the contiguous leaves
//           [L S, L S + S), sums them by an in-lane tree, then the xor butterfly 1 .. 32 finishes
//           the same tree across lanes.
//   stride  (routed experts, shared down): 32 "virtual lanes", lane v summing groups v, v + 32,
//           ... then the xor tree 16 .. 1. A row takes 4 physical lanes, each holding 8 virtual
//           lanes: per 256-column unit, lane p decodes the 32-column spans 32 p and 128 + 32 p
//           (virtual lanes 8 p .. 8 p + 7's groups), so a lane decodes whole Q4_K / Q6_K
//           sub-blocks and a Q8_0 block per span. Levels 16 and 8 of the tree cross lanes
//           (lane ^ 2, lane ^ 1), levels 4, 2, 1 stay in registers.
#include "moe_dev.h"
#include "moe_kernels.h"

// ---------------------------------------------------------------- tree rows (router, shared)

template <u32 NSP>
DEV float tree_row_lane(const float* w, const float* __restrict__ x, u32 c0base) {
  float s[NSP];
#pragma unroll
  for (u32 q = 0; q < NSP; q++) {
    const float* xv = x + c0base + 32 * q;
    float l[8];
#pragma unroll
    for (u32 g = 0; g < 8; g++) l[g] = leaf4(w + 32 * q + 4 * g, *(const float4*)(xv + 4 * g));
    s[q] = ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
  }
#pragma unroll
  for (u32 st = 1; st < NSP; st <<= 1)
#pragma unroll
    for (u32 q = 0; q < NSP; q += 2 * st) s[q] = s[q] + s[q + st];
  return s[0];
}

template <u32 NSP>
DEV void span_any(u32 fm, const u8* rp, u32 c0, float* w) {
  switch (fm) {
    case FM_F32: Span<FM_F32>::w(rp, c0, w); break;
    case FM_Q4_K: Span<FM_Q4_K>::w(rp, c0, w); break;
    case FM_Q6_K: Span<FM_Q6_K>::w(rp, c0, w); break;
    default: Span<FM_Q5_K>::w(rp, c0, w); break;
  }
}

// every tree row of the layer in one launch (router, shared gate logit, shared gate, shared up):
// one wave a row, blockDim 256 (4 rows), grid (ceil(rows / 4), ceil(T / tch))
template <u32 NSP>
__global__ void __launch_bounds__(256) k_tree_rows(TreeArgs a) {
  u32 row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const u32 L = threadIdx.x & 63;
  u32 sgi = 0;
  while (sgi < a.nseg && row >= a.seg[sgi].rows) { row -= a.seg[sgi].rows; sgi++; }
  if (sgi >= a.nseg) return;
  const TreeSeg sg = a.seg[sgi];
  const u32 c0 = 32 * NSP * L;
  const bool live = c0 < a.cols;  // pad leaves past cols count +0
  float w[32 * NSP];
  const u8* rp = sg.W + (u64)row * sg.rb;
#pragma unroll
  for (u32 q = 0; q < NSP; q++) {
    if (live) span_any<NSP>(sg.fm, rp, c0 + 32 * q, w + 32 * q);
    else
#pragma unroll
      for (u32 i = 0; i < 32; i++) w[32 * q + i] = 0.0f;
  }
  const u32 t0 = blockIdx.y * a.tch, t1 = min(a.T, t0 + a.tch);
  for (u32 t = t0; t < t1; t++) {
    float v = 0.0f;
    if (live) v = tree_row_lane<NSP>(w, a.x + (u64)t * a.xstride, c0);  // else every leaf is a +0 pad
    v = tree64_asc(v);
    if (L == 0) sg.out[(u64)t * sg.ostride + row] = v;
  }
}

// ---------------------------------------------------------------- top-k (llb_moe_topk)

// (value, index) of the larger p, ties to the lower index
DEV void amax_step(float& bv, u32& bi, float ov, u32 oi) {
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}
// the best (p, e) of the wave on every lane: pairs at xor 1, 2, then lanes + 4, 8 of the row, then
// the other row and half (any pairing gives the same maximum; ties resolve by index)
DEV void wave_amax(float& bv, u32& bi) {
  amax_step(bv, bi, dppf<DPP_XOR1>(bv), dppu<DPP_XOR1>(bi));
  amax_step(bv, bi, dppf<DPP_XOR2>(bv), dppu<DPP_XOR2>(bi));
  amax_step(bv, bi, dppf<DPP_UP4>(bv), dppu<DPP_UP4>(bi));
  amax_step(bv, bi, dppf<DPP_XOR8>(bv), dppu<DPP_XOR8>(bi));
  // lanes 0 mod 16 now hold their row's best; take rows 0..3's through readlane
  float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
  u32 i0 = (u32)__builtin_amdgcn_readlane((int)bi, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16)
    amax_step(v0, i0, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), r)),
              (u32)__builtin_amdgcn_readlane((int)bi, r));
  bv = v0;
  bi = i0;
}

// one wave a token (ne <= 1024), llb_moe_topk's arithmetic: mx = max; v = exp(l - mx); the sum in
// the 1024-thread block's order (thread t = expert t: each 32-expert group by the xor tree 16 .. 1,
// then the group sums in order); p = v (1 / sum); the k largest p, ties to the lower index;
// wt_j = p / max(sum of the k p in rank order, 2^-14); sgo = sigmoid(sg)
__global__ void __launch_bounds__(64) k_topk(TopkArgs a) {
  const u32 t = blockIdx.x, L = threadIdx.x;
  const float* lg = a.lg + (u64)t * a.lstride;
  const u32 ni = (a.ne + 63) / 64;
  float p[16];
  float mx = bits_f(0xFF800000u);
#pragma unroll
  for (u32 i = 0; i < 16; i++) {
    const u32 e = L + 64 * i;
    const bool ok = i < ni && e < a.ne;
    p[i] = ok ? lg[e] : 0.0f;
    if (ok) mx = fmaxf(mx, p[i]);
  }
  {
    u32 dummy = 0;
    wave_amax(mx, dummy);
  }
  float tot = 0.0f;
#pragma unroll
  for (u32 i = 0; i < 16; i++) {
    if (i < ni) {
      const u32 e = L + 64 * i;
      p[i] = e < a.ne ? exp_f(p[i] - mx) : 0.0f;
      const float s = tree32_desc(p[i]);
      tot = tot + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
      if (64 * i + 32 < a.ne) tot = tot + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
    }
  }
  const float inv = 1.0f / tot;
#pragma unroll
  for (u32 i = 0; i < 16; i++) p[i] = (i < ni && L + 64 * i < a.ne) ? p[i] * inv : -1.0f;
  u32* ids = a.ids + (u64)t * a.nk;
  float* wt = a.wt + (u64)t * a.nk;
  float s = 0.0f, mine = 0.0f;
  for (u32 j = 0; j < a.nk; j++) {
    float bv = -1.0f;
    u32 bi = 0xffffffffu;
#pragma unroll
    for (u32 i = 0; i < 16; i++)
      if (p[i] > bv) { bv = p[i]; bi = L + 64 * i; }
    wave_amax(bv, bi);
#pragma unroll
    for (u32 i = 0; i < 16; i++)
      if (L + 64 * i == bi) p[i] = -2.0f;
    s = s + bv;          // the rank-order sum, uniform across the wave
    if (L == j) mine = bv;
    if (L == 0) ids[j] = bi;
  }
  s = s < 6.103515625e-5f ? 6.103515625e-5f : s;
  if (L < a.nk) wt[L] = mine / s;
  if (L == 0) {
    const float sg = a.has_sg ? lg[a.ne] : 0.0f;
    a.sgo[t] = 1.0f / (1.0f + exp_f(-sg));
  }
}

// ---------------------------------------------------------------- stride rows (experts)
//
// moe_dot's order for a row: virtual lane v of 32 sums the leaves v, v + 32, ... in order, then
// the xor tree 16 .. 1. The leaves themselves are independent values, so a block first has every
// thread decode 32-column spans (all loads issued up front) into leaves in LDS, then replays the
// sequential sums, 32 threads a row, and finishes with the butterfly inside each 32-lane half.

template <u32 F>
DEV void span_leaves(const u8* __restrict__ row, u32 c0, const float* __restrict__ x, float* lv) {
  float4 xv[8];  // x first: its loads fly with the weights', not after the decode
#pragma unroll
  for (u32 g = 0; g < 8; g++) xv[g] = ((const float4*)(x + c0))[g];
  float w[32];
  Span<F>::w(row, c0, w);
#pragma unroll
  for (u32 g = 0; g < 8; g++) lv[g] = leaf4(w + 4 * g, xv[g]);
}
DEV void span_leaves_fm(u32 f, const u8* row, u32 c0, const float* x, float* lv) {
  switch (f) {
    case FM_Q8_0: span_leaves<FM_Q8_0>(row, c0, x, lv); break;
    case FM_Q4_K: span_leaves<FM_Q4_K>(row, c0, x, lv); break;
    case FM_Q6_K: span_leaves<FM_Q6_K>(row, c0, x, lv); break;
    default: span_leaves<FM_Q5_K>(row, c0, x, lv); break;
  }
}
DEV void store_leaves(float* dst, const float* lv) {
  ((float4*)dst)[0] = make_float4(lv[0], lv[1], lv[2], lv[3]);
  ((float4*)dst)[1] = make_float4(lv[4], lv[5], lv[6], lv[7]);
}
// lane v (0..31 of a 32-lane half) over ng leaves: the sequential sum, then the xor tree 16 .. 1;
// the row's dot is on lane v = 0
DEV float stride_sum(const float* lv, u32 ng, u32 v) {
  float acc = 0.0f;
  for (u32 g = v; g < ng; g += 32) acc = acc + lv[g];
  return tree32_desc(acc);
}

// gate + up + SwiGLU (llb_moe_gu): a block takes np (gate, up) row pairs of one slot, 2 np rows of
// dm columns. Leaves [2 np][dm / 4] in LDS; gate rows even, up rows odd.
template <u32 FG, u32 FU>
__global__ void __launch_bounds__(256) k_gu_exact(GuArgs a, u32 np) {
  extern __shared__ float lv[];
  const u32 task0 = blockIdx.x * np, slot = task0 / a.ef, r0 = task0 % a.ef;
  const u32 t = slot / a.nk;
  const float* x = a.h2 + (u64)t * a.dm;
  const u64 e = a.ids[slot];
  const u32 ns = a.dm / 32, ng = a.dm / 4, items = 2 * np * ns;
  for (u32 it = threadIdx.x; it < items; it += 256) {
    const u32 rr = it / ns, sp = it % ns, row = r0 + (rr >> 1);
    float l[8];
    if ((rr & 1) == 0) span_leaves<FG>(a.G + e * a.es + row * a.rbg, 32 * sp, x, l);
    else span_leaves<FU>(a.U + e * a.es + row * a.rbu, 32 * sp, x, l);
    store_leaves(lv + rr * ng + 8 * sp, l);
  }
  __syncthreads();
  const u32 rr = threadIdx.x >> 5, v = threadIdx.x & 31;
  float s = 0.0f;
  if (rr < 2 * np) s = stride_sum(lv + rr * ng, ng, v);
  const float u = xpeer32(s);  // the up row sits in the other half of the wave
  if (rr < 2 * np && (rr & 1) == 0 && v == 0) a.act[(u64)slot * a.ef + r0 + (rr >> 1)] = silu_mul(s, u);
}

// down + rank-order combine + gated shared expert + residual (llb_moe_dn): rw rows of one token a
// block; task j < nk is routed expert ids[j]'s row against act_j, j = nk the shared expert's down
// row against sa (computed here from the shared gate / up logits)
template <u32 FD, u32 FS>
__global__ void __launch_bounds__(256) k_dn_exact(DnArgs a) {
  extern __shared__ float sm[];
  const u32 t = blockIdx.y, nt = a.nk + (FS ? 1u : 0u);
  const u32 nge = a.ef / 4, ngs = a.sf / 4, per_row = a.nk * nge + (FS ? ngs : 0u);
  float* lv = sm;                                  // [rw][nk ef / 4 + sf / 4]
  float* sa = sm + a.rw * per_row;                 // [sf]
  float* part = sa + (FS ? a.sf : 0u);             // [rw][nt]
  if (FS) {
    const float* g = a.gsu + (u64)t * 2 * a.sf;
    for (u32 i = threadIdx.x; i < a.sf; i += 256) sa[i] = silu_mul(g[i], g[a.sf + i]);
    __syncthreads();
  }
  const float* act = a.act + (u64)t * a.nk * a.ef;
  const u32 nse = a.ef / 32, nss = a.sf / 32, spr = a.nk * nse + (FS ? nss : 0u);
  const u32 items = a.rw * spr;
  for (u32 it = threadIdx.x; it < items; it += 256) {
    const u32 rl = it / spr, q = it % spr, r = min(blockIdx.x * a.rw + rl, a.dm - 1);
    float l[8];
    if (q < a.nk * nse) {
      const u32 j = q / nse, sp = q % nse;
      const u64 e = a.ids[(u64)t * a.nk + j];
      span_leaves<FD>(a.D + (e * a.dm + r) * a.rbd, 32 * sp, act + (u64)j * a.ef, l);
      store_leaves(lv + rl * per_row + j * nge + 8 * sp, l);
    } else {
      const u32 sp = q - a.nk * nse;
      span_leaves<FS ? FS : FM_Q4_K>(a.SD + (u64)r * a.rbs, 32 * sp, sa, l);
      store_leaves(lv + rl * per_row + a.nk * nge + 8 * sp, l);
    }
  }
  __syncthreads();
  const u32 sums = a.rw * nt * 32;
  for (u32 q = threadIdx.x; q < ((sums + 63) & ~63u); q += 256) {
    const u32 k = q >> 5, v = q & 31;  // k = rl nt + j
    float s = 0.0f;
    if (q < sums) {
      const u32 rl = k / nt, j = k % nt;
      const float* base = lv + rl * per_row + j * nge;
      s = stride_sum(base, j < a.nk ? nge : ngs, v);
    } else {
      s = stride_sum(lv, 0, v);  // keeps the shuffles of a partial wave uniform
    }
    if (q < sums && v == 0) part[k] = s;
  }
  __syncthreads();
  if (threadIdx.x < a.rw) {
    const u32 r = blockIdx.x * a.rw + threadIdx.x;
    if (r < a.dm) {
      const float* wt = a.wt + (u64)t * a.nk;
      const float* pr = part + threadIdx.x * nt;
      float mo = 0.0f;
      for (u32 j = 0; j < a.nk; j++) mo = j == 0 ? pr[0] * wt[0] : mo + pr[j] * wt[j];
      const float res = a.x1 ? a.x1[(u64)t * a.dm + r] : 0.0f;
      a.y[(u64)t * a.dm + r] = FS ? (mo + pr[a.nk] * a.sgo[t]) + res : mo + res;
    }
  }
}

// ---------------------------------------------------------------- dequant (parity of the decoders)

template <u32 F>
__global__ void __launch_bounds__(256) k_dequant(const u8* __restrict__ W, u64 rb, u32 rows, u32 cols,
                                                 float* __restrict__ out) {
  const u64 i = (u64)blockIdx.x * 256 + threadIdx.x, ns = cols / 32;
  if (i >= (u64)rows * ns) return;
  const u64 r = i / ns;
  const u32 c0 = (u32)(i % ns) * 32;
  float w[32];
  Span<F>::w(W + r * rb, c0, w);
  float* o = out + r * cols + c0;
#pragma unroll
  for (u32 k = 0; k < 32; k++) o[k] = w[k];
}

// ---------------------------------------------------------------- launchers

#define FM_CASES(X) X(FM_Q8_0) X(FM_Q4_K) X(FM_Q6_K) X(FM_Q5_K)

int launch_tree_rows(const TreeArgs& a, u32 nsp, hipStream_t st) {
  u32 rows = 0;
  for (u32 i = 0; i < a.nseg; i++) rows += a.seg[i].rows;
  if (rows == 0) return 0;
  dim3 grid((rows + 3) / 4, (a.T + a.tch - 1) / a.tch);
  if (nsp == 1) { hipLaunchKernelGGL((k_tree_rows<1>), grid, dim3(256), 0, st, a); return 0; }
  if (nsp == 2) { hipLaunchKernelGGL((k_tree_rows<2>), grid, dim3(256), 0, st, a); return 0; }
  if (nsp == 4) { hipLaunchKernelGGL((k_tree_rows<4>), grid, dim3(256), 0, st, a); return 0; }
  return -1;
}

int launch_topk(const TopkArgs& a, u32 T, hipStream_t st) {
  hipLaunchKernelGGL(k_topk, dim3(T), dim3(64), 0, st, a);
  return 0;
}

int launch_gu_exact(const GuArgs& a, u32 fg, u32 fu, u32 nslots, hipStream_t st) {
  if (fg != fu) return -1;
  const u32 np = a.dm >= 4096 ? 1u : 2u;  // 2 np rows of dm / 32 spans: about one span a thread
  dim3 grid(nslots * a.ef / np);
  const size_t sm = (size_t)2 * np * (a.dm / 4) * 4;
#define GU_L(F) \
  if (fg == F) { hipLaunchKernelGGL((k_gu_exact<F, F>), grid, dim3(256), sm, st, a, np); return 0; }
  FM_CASES(GU_L)
#undef GU_L
  return -1;
}

// rows a down block takes: about 512 span items (two a thread), at least one row
u32 dn_rows(u32 nk, u32 ef, u32 sf) {
  const u32 spr = nk * (ef / 32) + sf / 32;
  u32 rw = 512 / spr;
  return rw < 1 ? 1 : rw > 8 ? 8 : rw;
}

int launch_dn_exact(const DnArgs& a, u32 fd, u32 fs, u32 T, hipStream_t st) {
  dim3 grid((a.dm + a.rw - 1) / a.rw, T);
  const u32 nt = a.nk + (fs ? 1u : 0u);
  const size_t sm = ((size_t)a.rw * (a.nk * a.ef / 4 + (fs ? a.sf / 4 : 0)) + (fs ? a.sf : 0) + a.rw * nt) * 4;
#define DN_L(FD, FS) \
  if (fd == FD && fs == FS) { hipLaunchKernelGGL((k_dn_exact<FD, FS>), grid, dim3(256), sm, st, a); return 0; }
#define DN_FS(FD) DN_L(FD, 0u) DN_L(FD, FM_Q4_K) DN_L(FD, FM_Q6_K) DN_L(FD, FM_Q5_K)
  FM_CASES(DN_FS)
#undef DN_FS
#undef DN_L
  return -1;
}

int launch_dequant(u32 fm, const u8* W, u64 rb, u32 rows, u32 cols, float* out, hipStream_t st) {
  const u64 n = (u64)rows * (cols / 32);
  dim3 grid((u32)((n + 255) / 256));
#define DQ_L(F) \
  if (fm == F) { hipLaunchKernelGGL((k_dequant<F>), grid, dim3(256), 0, st, W, rb, rows, cols, out); return 0; }
  FM_CASES(DQ_L) DQ_L(FM_F32)
#undef DQ_L
  return -1;
}
