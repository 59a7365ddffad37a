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

template <u32 F, u32 NSP>
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

// one wave a row, blockDim 256 (4 rows), grid (ceil(rows / 4), ceil(T / tch))
template <u32 F, u32 NSP>
__global__ void __launch_bounds__(256) k_tree_rows(TreeArgs a, u32 seg_id) {
  const TreeSeg sg = a.seg[seg_id];
  const u32 row = blockIdx.x * 4 + (threadIdx.x >> 6), L = threadIdx.x & 63;
  if (row >= sg.rows) return;
  const u32 c0 = 32 * NSP * L;
  const bool live = c0 < a.cols;  // pad leaves past cols count +0
  float w[32 * NSP];
  const u8* rp = sg.W + (u64)row * sg.rb;
#pragma unroll
  for (u32 q = 0; q < NSP; q++) {
    if (live) Span<F>::w(rp, c0 + 32 * q, w + 32 * q);
    else
#pragma unroll
      for (u32 i = 0; i < 32; i++) w[32 * q + i] = 0.0f;
  }
  const u32 t0 = blockIdx.y * a.tch, t1 = min(a.T, t0 + a.tch);
  for (u32 t = t0; t < t1; t++) {
    float v = 0.0f;
    if (live) v = tree_row_lane<F, NSP>(w, a.x + (u64)t * a.xstride, c0);  // else every leaf is a +0 pad
#pragma unroll
    for (u32 m = 1; m < 64; m <<= 1) v = v + __shfl_xor(v, m, 64);
    if (L == 0) sg.out[(u64)t * sg.ostride + row] = v;
  }
}

// ---------------------------------------------------------------- top-k (llb_moe_topk)

// one wave a token (ne <= 1024): the softmax in llb_moe_topk's order, the top k by p (ties to
// the lower index), the renormalisation with the 2^-14 clamp, sgo = sigmoid(sg); then the shared
// expert's sa = silu(g_s) u_s
__global__ void __launch_bounds__(64) k_topk(TopkArgs a) {
  __shared__ float wsum[32];
  const u32 t = blockIdx.x, L = threadIdx.x;
  const float* lg = a.lg + (u64)t * a.lstride;
  float p[16];
  float mx = bits_f(0xFF800000u);
#pragma unroll
  for (u32 i = 0; i < 16; i++) {
    const u32 e = L + 64 * i;
    p[i] = e < a.ne ? lg[e] : 0.0f;
    if (e < a.ne) mx = fmaxf(mx, p[i]);
  }
#pragma unroll
  for (u32 m = 32; m > 0; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  // v_e = exp(l_e - mx); per 32-expert group the xor tree 16 .. 1, then the group sums in order
#pragma unroll
  for (u32 i = 0; i < 16; i++) {
    const u32 e = L + 64 * i;
    p[i] = e < a.ne ? exp_f(p[i] - mx) : 0.0f;
    if (64 * i < a.ne) {
      float s = p[i];
#pragma unroll
      for (u32 m = 16; m > 0; m >>= 1) s = s + __shfl_xor(s, m, 64);
      if ((L & 31) == 0) wsum[2 * i + (L >> 5)] = s;
    }
  }
  __syncthreads();
  float tot = 0.0f;
  const u32 nw = (a.ne + 31) / 32;
  for (u32 w = 0; w < nw; w++) tot = tot + wsum[w];
  const float inv = 1.0f / tot;
#pragma unroll
  for (u32 i = 0; i < 16; i++) p[i] = L + 64 * i < a.ne ? p[i] * inv : -1.0f;
  float wv[64];
  u32* ids = a.ids + (u64)t * a.nk;
  for (u32 j = 0; j < a.nk; j++) {
    float bv = -1.0f;
    u32 bi = 0xffffffffu;
#pragma unroll
    for (u32 i = 0; i < 16; i++)
      if (p[i] > bv) { bv = p[i]; bi = L + 64 * i; }
#pragma unroll
    for (u32 m = 32; m > 0; m >>= 1) {
      const float ov = __shfl_xor(bv, m, 64);
      const u32 oi = __shfl_xor(bi, m, 64);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
#pragma unroll
    for (u32 i = 0; i < 16; i++)
      if (L + 64 * i == bi) p[i] = -2.0f;
    if (j < 64) wv[j] = bv;
    if (L == 0) ids[j] = bi;
  }
  if (L == 0) {
    float s = 0.0f;
    for (u32 j = 0; j < a.nk; j++) s = s + wv[j];
    s = s < 6.103515625e-5f ? 6.103515625e-5f : s;
    float* wt = a.wt + (u64)t * a.nk;
    for (u32 j = 0; j < a.nk; j++) wt[j] = wv[j] / s;
    const float sg = a.has_sg ? lg[a.ne] : 0.0f;
    a.sgo[t] = 1.0f / (1.0f + exp_f(-sg));
  }
  if (a.sf) {
    const float* g = a.gsu + (u64)t * 2 * a.sf;
    float* sa = a.sa + (u64)t * a.sf;
    for (u32 i = L; i < a.sf; i += 64) sa[i] = silu_mul(g[i], g[a.sf + i]);
  }
}

// ---------------------------------------------------------------- stride rows (experts)

// lane p (of the row's 4) over the row: returns the row's dot in moe_dot's order on every lane
template <u32 F>
DEV float stride_row(const u8* __restrict__ row, u32 cols, const float* xs, u32 p) {
  float acc[8];
#pragma unroll
  for (u32 j = 0; j < 8; j++) acc[j] = 0.0f;
  const u32 nu = cols >> 8;
  for (u32 s = 0; s < nu; s++) {
#pragma unroll
    for (u32 h = 0; h < 2; h++) {
      const u32 c0 = 256 * s + 128 * h + 32 * p;
      float w[32];
      Span<F>::w(row, c0, w);
#pragma unroll
      for (u32 j = 0; j < 8; j++) acc[j] = acc[j] + leaf4(w + 4 * j, *(const float4*)(xs + c0 + 4 * j));
    }
  }
#pragma unroll
  for (u32 j = 0; j < 8; j++) acc[j] = acc[j] + __shfl_xor(acc[j], 2, 64);
#pragma unroll
  for (u32 j = 0; j < 8; j++) acc[j] = acc[j] + __shfl_xor(acc[j], 1, 64);
  const float b0 = acc[0] + acc[4], b1 = acc[1] + acc[5], b2 = acc[2] + acc[6], b3 = acc[3] + acc[7];
  return (b0 + b2) + (b1 + b3);
}

DEV float stride_row_fm(u32 f, const u8* row, u32 cols, const float* xs, u32 p) {
  switch (f) {
    case FM_Q8_0: return stride_row<FM_Q8_0>(row, cols, xs, p);
    case FM_Q4_K: return stride_row<FM_Q4_K>(row, cols, xs, p);
    case FM_Q6_K: return stride_row<FM_Q6_K>(row, cols, xs, p);
    default: return stride_row<FM_Q5_K>(row, cols, xs, p);
  }
}

// gate + up + SwiGLU (llb_moe_gu): 128 threads = 16 (gate, up) row pairs of one slot. Wave w's
// lane groups 0..7 take gate rows, 8..15 the same up rows; lane ^ 32 pairs them.
template <u32 FG, u32 FU>
__global__ void __launch_bounds__(128) k_gu_exact(GuArgs a) {
  extern __shared__ float xs[];
  const u32 task0 = blockIdx.x * 16, slot = task0 / a.ef, r0 = task0 % a.ef;
  const u32 t = slot / a.nk;
  const float* x = a.h2 + (u64)t * a.dm;
  for (u32 i = threadIdx.x; i < a.dm / 4; i += 128) ((float4*)xs)[i] = ((const float4*)x)[i];
  __syncthreads();
  const u32 L = threadIdx.x & 63, q = L >> 2, p = L & 3;
  const u32 row = r0 + 8 * (threadIdx.x >> 6) + (q & 7);
  const u64 e = a.ids[slot];
  float v;
  if (q < 8) v = stride_row<FG>(a.G + e * a.es + row * a.rbg, a.dm, xs, p);
  else v = stride_row<FU>(a.U + e * a.es + row * a.rbu, a.dm, xs, p);
  const float u = __shfl_xor(v, 32, 64);
  if (q < 8 && p == 0) a.act[(u64)slot * a.ef + row] = silu_mul(v, u);
}

// down + rank-order combine + gated shared expert + residual (llb_moe_dn): 256 threads = 64
// lane groups; rw rows of one token a block, task (j, r) for j < nk (routed) and j = nk (shared)
template <u32 FD, u32 FS>
__global__ void __launch_bounds__(256) k_dn_exact(DnArgs a) {
  extern __shared__ float xs[];  // act of the token's nk slots, then sa
  __shared__ float part[64];
  const u32 t = blockIdx.y, nt = a.nk + (FS ? 1u : 0u);
  const float* act = a.act + (u64)t * a.nk * a.ef;
  for (u32 i = threadIdx.x; i < a.nk * a.ef / 4; i += 256) ((float4*)xs)[i] = ((const float4*)act)[i];
  if (FS) {
    const float* sa = a.sa + (u64)t * a.sf;
    for (u32 i = threadIdx.x; i < a.sf / 4; i += 256) ((float4*)(xs + a.nk * a.ef))[i] = ((const float4*)sa)[i];
  }
  __syncthreads();
  const u32 g = threadIdx.x >> 2, p = threadIdx.x & 3;
  if (g < a.rw * nt) {
    const u32 j = g / a.rw, rl = g % a.rw, r = blockIdx.x * a.rw + rl;
    if (r < a.dm) {
      float v;
      if (j < a.nk) {
        const u64 e = a.ids[(u64)t * a.nk + j];
        v = stride_row<FD>(a.D + (e * a.dm + r) * a.rbd, a.ef, xs + j * a.ef, p);
      } else {
        v = stride_row<FS ? FS : FM_Q4_K>(a.SD + (u64)r * a.rbs, a.sf, xs + a.nk * a.ef, p);
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
      float y;
      if (FS) y = (mo + part[a.nk * a.rw + threadIdx.x] * a.sgo[t]) + res;
      else y = mo + res;
      a.y[(u64)t * a.dm + r] = y;
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

int launch_tree_rows(const TreeArgs& a, u32 seg, u32 fm, u32 nsp, hipStream_t st) {
  if (a.seg[seg].rows == 0) return 0;
  dim3 grid((a.seg[seg].rows + 3) / 4, (a.T + a.tch - 1) / a.tch);
#define TREE_L(F, N) \
  if (fm == F && nsp == N) { hipLaunchKernelGGL((k_tree_rows<F, N>), grid, dim3(256), 0, st, a, seg); return 0; }
  TREE_L(FM_F32, 1) TREE_L(FM_F32, 2) TREE_L(FM_F32, 4)
  TREE_L(FM_Q4_K, 1) TREE_L(FM_Q4_K, 2) TREE_L(FM_Q4_K, 4)
  TREE_L(FM_Q6_K, 1) TREE_L(FM_Q6_K, 2) TREE_L(FM_Q6_K, 4)
  TREE_L(FM_Q5_K, 1) TREE_L(FM_Q5_K, 2) TREE_L(FM_Q5_K, 4)
#undef TREE_L
  return -1;
}

int launch_topk(const TopkArgs& a, u32 T, hipStream_t st) {
  hipLaunchKernelGGL(k_topk, dim3(T), dim3(64), 0, st, a);
  return 0;
}

int launch_gu_exact(const GuArgs& a, u32 fg, u32 fu, u32 nslots, hipStream_t st) {
  if (fg != fu) return -1;
  dim3 grid(nslots * a.ef / 16);
  const size_t sm = (size_t)a.dm * 4;
#define GU_L(F) \
  if (fg == F) { hipLaunchKernelGGL((k_gu_exact<F, F>), grid, dim3(128), sm, st, a); return 0; }
  FM_CASES(GU_L)
#undef GU_L
  return -1;
}

int launch_dn_exact(const DnArgs& a, u32 fd, u32 fs, u32 T, hipStream_t st) {
  dim3 grid((a.dm + a.rw - 1) / a.rw, T);
  const size_t sm = ((size_t)a.nk * a.ef + a.sf) * 4;
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
