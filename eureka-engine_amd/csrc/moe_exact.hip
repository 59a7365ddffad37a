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
#include "moe_q8dot.h"

// phase timestamps for latency studies: a build that defines MOE_PHASE_T gets (block 0, thread 0)
// wall-clock stamps (100 MHz) in moe_phase_t[]; the library build compiles them away
#ifdef MOE_PHASE_T
__device__ unsigned long long moe_phase_t[64];
#define PHASE(i) \
  do { if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) moe_phase_t[i] = __builtin_amdgcn_s_memrealtime(); } while (0)
// per-block start / end stamps of kernel k: moe_blk_t[k][block][0 | 1] (blocks < 4096, grid x only)
__device__ unsigned long long moe_blk_t[4][4096][2];
#define BSTAMP(k, i) \
  do { if (threadIdx.x == 0 && blockIdx.x < 4096 && blockIdx.y == 0) moe_blk_t[k][blockIdx.x][i] = __builtin_amdgcn_s_memrealtime(); } while (0)
// stamp i once v has arrived (the asm takes v as an input, so the wait for it comes first)
#define PHASE_AFTER(i, v) do { __asm__ volatile("" :: "v"(v)); PHASE(i); } while (0)
// the stamps to the host: phase [64], blk [4][4096][2]
extern "C" int moe_phase_read(unsigned long long* phase, unsigned long long* blk) {
  if (hipMemcpyFromSymbol(phase, HIP_SYMBOL(moe_phase_t), sizeof moe_phase_t) != hipSuccess) return -1;
  return hipMemcpyFromSymbol(blk, HIP_SYMBOL(moe_blk_t), sizeof moe_blk_t) == hipSuccess ? 0 : -1;
}
#else
#define PHASE_AFTER(i, v) do {} while (0)
#define PHASE(i) do {} while (0)
#define BSTAMP(k, i) do {} while (0)
#endif

// ---------------------------------------------------------------- tree rows (router, shared)

// lanes of one wave exchanging words through LDS: a wave's LDS operations complete in issue order,
// so only the compiler must not move them across this point
#define WAVE_SYNC() do { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); __builtin_amdgcn_wave_barrier(); } while (0)

DEV void span_any(u32 fm, const u8* rp, u32 c0, float* w) {
  switch (fm) {
    case FM_F32: Span<FM_F32>::w(rp, c0, w); break;
    case FM_Q4_K: Span<FM_Q4_K>::w(rp, c0, w); break;
    case FM_Q6_K: Span<FM_Q6_K>::w(rp, c0, w); break;
    default: Span<FM_Q5_K>::w(rp, c0, w); break;
  }
}

// rows a wave: the lane's x span is loaded once for them, every row's loads in flight together
// (2 spans of weights a lane at most)
template <u32 NSP> constexpr u32 tree_rpw() { return NSP >= 2 ? 1u : 2u; }
u32 tree_rows_per_wave(u32 nsp) { return nsp >= 2 ? 1u : 2u; }

// every tree row of the layer in one launch (router, shared gate logit, shared gate, shared up):
// a wave takes tree_rpw<NSP>() consecutive rows (of the concatenated segments); blockDim 64, grid
// (ceil(rows / tree_rpw<NSP>()), T). The tree has 64 NQ leaves (NQ = 8 NSP), leaf i = columns
// 4 i .. 4 i + 3 (+0 past cols).
//  * F32 rows (router, shared gate logit) load coalesced: lane L holds leaves 64 q + L (q < NQ);
//    the tree's first six levels pair lanes (tree64_asc, exact on lane 0), the rest pair q in the lane.
//  * quantized rows decode whole spans: lane L holds the contiguous leaves [NQ L, NQ L + NQ); the
//    first log2 NQ levels are in the lane, the last six across lanes.
// x is loaded coalesced and reaches the second layout through LDS (lanes padded 4 floats apart).
// The rows' segments are looked up first, then all their loads go out, then each row is reduced.
template <u32 NQ> DEV float tree_in_lane(float* n) {
#pragma unroll
  for (u32 st = 1; st < NQ; st <<= 1)
#pragma unroll
    for (u32 q = 0; q < NQ; q += 2 * st) n[q] = n[q] + n[q + st];
  return n[0];
}
template <u32 NSP>
DEV void tree_body(const TreeArgs& a, u32 bx, u32 t, u32 L, float* xsh) {
  PHASE(24);
  constexpr u32 RPW = tree_rpw<NSP>(), NQ = 8 * NSP, LS = 4 * NQ + 4;
  const u32 nl4 = a.cols / 4;
  const float4* x4 = (const float4*)(a.x + (u64)t * a.xstride);
  float4 xc[NQ];
  if (a.nz) {
    // llb_rmsnorm_add's arithmetic (k_rmsnorm_add) on this layout: x1 = x + z; the squares' sum is the
    // balanced pairwise tree in column order over 64 NQ float4 groups (2^cdepth leaves, +0 pads) -- in
    // the group, then six levels across lanes (group 64 q + L), then over q in the lane -- the same
    // tree k_rmsnorm_add sums; s = 1 / sqrt(sum / cols + eps), h2 = (x1 s) w
    const float4* z4 = (const float4*)(a.nz + (u64)t * a.xstride);
    const float4* w4 = (const float4*)a.nw;
    float4 v[NQ], wv[NQ];
#pragma unroll
    for (u32 q = 0; q < NQ; q++) {
      const bool in = 64 * q + L < nl4;
      const float4 xa = in ? x4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 za = in ? z4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
      wv[q] = in ? w4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
      v[q] = make_float4(xa.x + za.x, xa.y + za.y, xa.z + za.z, xa.w + za.w);
    }
    float n[NQ];
#pragma unroll
    for (u32 q = 0; q < NQ; q++)
      n[q] = tree64_asc((v[q].x * v[q].x + v[q].y * v[q].y) + (v[q].z * v[q].z + v[q].w * v[q].w));
    const float sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, tree_in_lane<NQ>(n))));
    const float s = 1.0f / __builtin_sqrtf(sum / (float)a.cols + a.eps);  // correctly rounded, as k_rmsnorm_add
#pragma unroll
    for (u32 q = 0; q < NQ; q++)
      xc[q] = make_float4((v[q].x * s) * wv[q].x, (v[q].y * s) * wv[q].y, (v[q].z * s) * wv[q].z, (v[q].w * s) * wv[q].w);
    if (bx == 0) {
#pragma unroll
      for (u32 q = 0; q < NQ; q++) {
        if (64 * q + L < nl4) {
          ((float4*)(a.x1o + (u64)t * a.xstride))[64 * q + L] = v[q];
          ((float4*)(a.h2o + (u64)t * a.xstride))[64 * q + L] = xc[q];
        }
      }
    }
  } else {
#pragma unroll
    for (u32 q = 0; q < NQ; q++) xc[q] = 64 * q + L < nl4 ? x4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  u32 row[RPW], sgi[RPW];
#pragma unroll
  for (u32 k = 0; k < RPW; k++) {
    u32 r = bx * RPW + k, s = 0;
    while (s < a.nseg && r >= a.seg[s].rows) { r -= a.seg[s].rows; s++; }
    row[k] = r;
    sgi[k] = s;  // nseg: past the last row
  }
  const u32 c0 = 32 * NSP * L;
  const bool live = c0 < a.cols;
  float4 wr[RPW][NQ];
#pragma unroll
  for (u32 k = 0; k < RPW; k++) {
    if (sgi[k] >= a.nseg) continue;
    const TreeSeg& sg = a.seg[sgi[k]];
    const u8* rp = sg.W + (u64)row[k] * sg.rb;
    if (sg.fm == FM_F32) {
#pragma unroll
      for (u32 q = 0; q < NQ; q++) wr[k][q] = 64 * q + L < nl4 ? ((const float4*)rp)[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
#pragma unroll
      for (u32 q = 0; q < NSP; q++) {
        float w[32];
        if (live) span_any(sg.fm, rp, c0 + 32 * q, w);
        else
#pragma unroll
          for (u32 i = 0; i < 32; i++) w[i] = 0.0f;
#pragma unroll
        for (u32 g = 0; g < 8; g++) wr[k][8 * q + g] = make_float4(w[4 * g], w[4 * g + 1], w[4 * g + 2], w[4 * g + 3]);
      }
    }
  }
  // the contiguous layout of x for quantized rows
#pragma unroll
  for (u32 q = 0; q < NQ; q++) {
    const u32 li = 64 * q + L;
    *(float4*)(xsh + (li / NQ) * LS + 4 * (li % NQ)) = xc[q];
  }
  WAVE_SYNC();
  PHASE(25);
#pragma unroll
  for (u32 k = 0; k < RPW; k++) {
    if (sgi[k] >= a.nseg) break;
    const TreeSeg& sg = a.seg[sgi[k]];
    float v;
    if (sg.fm == FM_F32) {
      float n[NQ];
#pragma unroll
      for (u32 q = 0; q < NQ; q++) n[q] = tree64_asc(leaf4((const float*)&wr[k][q], xc[q]));
      v = tree_in_lane<NQ>(n);
    } else {
      float n[NQ];
#pragma unroll
      for (u32 q = 0; q < NQ; q++) n[q] = leaf4((const float*)&wr[k][q], *(const float4*)(xsh + L * LS + 4 * q));
      v = tree64_asc(live ? tree_in_lane<NQ>(n) : 0.0f);  // a dead lane's leaves are all +0 pads
    }
    if (L == 0) sg.out[(u64)t * sg.ostride + row[k]] = sg.bias ? v + sg.bias[row[k]] : v;
  }
  PHASE(26);
}
template <u32 NSP> constexpr u32 tree_lds() { return 64 * (32 * NSP + 4); }  // floats
template <u32 NSP>
__global__ void __launch_bounds__(64) k_tree_rows(TreeArgs a) {
  __shared__ float xsh[tree_lds<NSP>()];
  BSTAMP(0, 0);
  tree_body<NSP>(a, blockIdx.x, blockIdx.y, threadIdx.x, xsh);
  BSTAMP(0, 1);
}

// Many tokens (prefill, batches): a block of four waves takes 4 RW consecutive rows (RW = 4 for rows of
// one span a lane, 2 for two) and tiles of TT tokens. A tile's x rows are staged in LDS once (coalesced
// loads, lanes padded 4 floats apart), each token's x read from LDS once for a wave's RW rows; each wave
// holds its rows' weights in registers (lane L: the contiguous leaves [NQ L, NQ L + NQ)) and reduces
// them against every token: the in-lane levels, then tree64_asc -- the same tree as tree_body, so the
// same sums.
// A block walks `ntb` consecutive tiles of TT tokens (grid.y = ceil(T / (TT ntb))) with its rows'
// weights held in registers the whole time: weights are read once per TT ntb tokens, and the next
// tile's x loads are in flight while the current tile is reduced. The wave index is made uniform so
// the segment table and the row pointers come through scalar loads, ahead of every vector load.
template <u32 NSP, u32 TT>
DEV void tree_mt_load_x(const TreeArgs& a, u32 tid, u32 t0, float4* xl) {
  constexpr u32 NQ = 8 * NSP, XJ = TT * 64 * NQ / 256;
  const u32 nl4 = a.cols / 4;
#pragma unroll
  for (u32 j = 0; j < XJ; j++) {  // tokens past T and columns past cols are zeros
    const u32 i = tid + 256 * j, tt = i / (64 * NQ), li = i % (64 * NQ), t = t0 + tt;
    xl[j] = (t < a.T && li < nl4) ? ((const float4*)(a.x + (u64)t * a.xstride))[li] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}
template <u32 NSP, u32 TT, u32 RW>
__global__ void __launch_bounds__(256) k_tree_rows_mt(TreeArgs a, u32 ntb) {
  constexpr u32 NQ = 8 * NSP, LS = 4 * NQ + 4;
  constexpr u32 XJ = TT * 64 * NQ / 256;  // float4 staging loads a thread
  static_assert(XJ * 256 == TT * 64 * NQ, "whole float4s a thread");
  constexpr u32 LS4 = LS / 4;
  extern __shared__ float4 xsh4[];  // [TT][64 lanes][LS floats]
  const u32 tid = threadIdx.x, L = tid & 63;
  const u32 w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // this wave's RW rows: segment, row in it, output and bias (wave-uniform)
  const u32 c0 = 32 * NSP * L;
  const bool live = c0 < a.cols;
  const u8* wp[RW];
  float* op[RW];
  u32 fm[RW], ost[RW];
  bool has[RW], hb[RW];
  float bia[RW];
#pragma unroll
  for (u32 k = 0; k < RW; k++) {
    u32 r = blockIdx.x * 4 * RW + RW * w + k, s = 0;
    while (s < a.nseg && r >= a.seg[s].rows) { r -= a.seg[s].rows; s++; }
    has[k] = s < a.nseg;  // false: past the last row
    const TreeSeg& sg = a.seg[has[k] ? s : 0];
    wp[k] = sg.W + (u64)r * sg.rb;
    fm[k] = sg.fm;
    op[k] = sg.out + r;
    ost[k] = sg.ostride;
    hb[k] = has[k] && sg.bias;
    bia[k] = hb[k] ? sg.bias[r] : 0.0f;
    has[k] = has[k] && sg.out != nullptr;
  }
  const u32 tb = blockIdx.y * TT * ntb;
  float wr[RW][32 * NSP];
#pragma unroll
  for (u32 k = 0; k < RW; k++) {
    const bool ok = live && has[k];
#pragma unroll
    for (u32 q = 0; q < NSP; q++) {
      if (ok) {
        if (fm[k] == FM_F32) {
          const float4* p = (const float4*)(wp[k] + 4 * (c0 + 32 * q));
#pragma unroll
          for (u32 g = 0; g < 8; g++) *(float4*)(wr[k] + 32 * q + 4 * g) = p[g];
        } else {
          span_any(fm[k], wp[k], c0 + 32 * q, wr[k] + 32 * q);
        }
      } else {
#pragma unroll
        for (u32 i = 0; i < 32; i++) wr[k][32 * q + i] = 0.0f;
      }
    }
  }
  float4 xl[XJ];
  tree_mt_load_x<NSP, TT>(a, tid, tb, xl);
  for (u32 j = 0; j < ntb; j++) {
    const u32 t0 = tb + j * TT;
    if (t0 >= a.T) break;  // block-uniform
    if (j) __syncthreads();  // every wave is done with the previous tile's x
#pragma unroll
    for (u32 jj = 0; jj < XJ; jj++) {
      const u32 i = tid + 256 * jj, tt = i / (64 * NQ), li = i % (64 * NQ);
      xsh4[tt * 64 * LS4 + (li / NQ) * LS4 + li % NQ] = xl[jj];
    }
    __syncthreads();
    if (j + 1 < ntb && t0 + TT < a.T) tree_mt_load_x<NSP, TT>(a, tid, t0 + TT, xl);  // next tile in flight
    // every token of the tile (rows past T are zeros, their sums never stored): the in-lane levels
    // first, then the six cross-lane levels of all RW TT sums together -- independent chains, so the
    // DPP and permlane latencies overlap -- and one store block
    float v[TT][RW];
#pragma unroll
    for (u32 tt = 0; tt < TT; tt++) {
      float4 xv[NQ];
#pragma unroll
      for (u32 q = 0; q < NQ; q++) xv[q] = xsh4[tt * 64 * LS4 + L * LS4 + q];
#pragma unroll
      for (u32 k = 0; k < RW; k++) {
        float n[NQ];
#pragma unroll
        for (u32 q = 0; q < NQ; q++) n[q] = leaf4(wr[k] + 4 * q, xv[q]);
        v[tt][k] = live ? tree_in_lane<NQ>(n) : 0.0f;  // a dead lane's leaves are +0 pads
      }
    }
#pragma unroll
    for (u32 tt = 0; tt < TT; tt++)
#pragma unroll
      for (u32 k = 0; k < RW; k++) v[tt][k] = tree64_asc(v[tt][k]);
    if (L == 0) {
#pragma unroll
      for (u32 tt = 0; tt < TT; tt++)
#pragma unroll
        for (u32 k = 0; k < RW; k++)
          if (has[k] && t0 + tt < a.T) op[k][(u64)(t0 + tt) * ost[k]] = hb[k] ? v[tt][k] + bia[k] : v[tt][k];
    }
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
  // every lane holds its row's best: the other row of the pair, then the other half
  {
    const auto v = __builtin_amdgcn_permlane16_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto i = __builtin_amdgcn_permlane16_swap(bi, bi, false, false);
    float v0 = __uint_as_float(v[0]);
    u32 i0 = i[0];
    amax_step(v0, i0, __uint_as_float(v[1]), i[1]);
    bv = v0;
    bi = i0;
  }
  {
    const auto v = __builtin_amdgcn_permlane32_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto i = __builtin_amdgcn_permlane32_swap(bi, bi, false, false);
    float v0 = __uint_as_float(v[0]);
    u32 i0 = i[0];
    amax_step(v0, i0, __uint_as_float(v[1]), i[1]);
    bv = v0;
    bi = i0;
  }
}

// LDS of topk_body256 (floats): p [1024], sums / tau / count / lane maxima [128], chosen p [64],
// candidates [256 + 256], the chosen experts [64] (u32)
#define TOPK_SIDS (1024 + 128 + 64 + 512)
#define TOPK_LDS (TOPK_SIDS + 64)
// one block of 256 a token (ne <= 1024), llb_moe_topk's arithmetic: mx = max; v = exp(l - mx); the
// sum in the 1024-thread block's order (expert e on thread e: each 32-expert group by the xor tree
// 16 .. 1, then the group sums in order); p = v (1 / sum). Selection by rank instead of k argmax
// rounds: rank(e) = #{e' : p_e' > p_e, or p_e' = p_e and e' < e} is the round in which repeated
// argmax (ties to the lower index) would take e, so the experts with rank < k are the top k in that
// order -- independent compares, no serial chain. wt_j = p / max(sum of the k p in rank order,
// 2^-14); sgo = sigmoid(sg). Thread t holds experts t, t + 256, t + 512, t + 768.
// a token's routing out of topk_body256's LDS into ids / wt / sgo (the renormalised weights as
// llb_moe_topk: the rank-order sum of the chosen p, clamped at 2^-14, divides each)
DEV void topk_write(const TopkArgs& a, u32 t, const float* sm) {
  const u32 tid = threadIdx.x;
  const float* wv = sm + 1152;
  const u32* ids = (const u32*)(sm + TOPK_SIDS);
  if (tid < 64) {
    float s = 0.0f;
    for (u32 j = 0; j < a.nk; j++) s = s + wv[j];
    s = s < 6.103515625e-5f ? 6.103515625e-5f : s;
    if (tid < a.nk) {
      a.wt[(u64)t * a.nk + tid] = wv[tid] / s;
      a.ids[(u64)t * a.nk + tid] = ids[tid];
    }
    if (tid == 0) {
      const float sg = a.has_sg ? a.lg[(u64)t * a.lstride + a.ne] : 0.0f;
      a.sgo[t] = 1.0f / (1.0f + exp_f(-sg));
    }
  }
}
DEV void topk_body256(const TopkArgs& a, u32 t, float* sm, bool wr) {
  float* ps = sm;               // [ne] p
  float* red = sm + 1024;       // [32] group sums / wave maxima, [32] tau, [40] count, [64..128) lane maxima
  float* wv = sm + 1152;        // [64] the chosen p by rank, then [256] + [256] candidates
  const u32 tid = threadIdx.x, L = tid & 63, w = tid >> 6;
  PHASE(0);
  const float* lg = a.lg + (u64)t * a.lstride;
  const u32 ni = (a.ne + 255) / 256;
  float p[4];
  float mx = bits_f(0xFF800000u);
#pragma unroll
  for (u32 i = 0; i < 4; i++) {
    const u32 e = tid + 256 * i;
    p[i] = (i < ni && e < a.ne) ? lg[e] : 0.0f;
    if (i < ni && e < a.ne) mx = fmaxf(mx, p[i]);
  }
  PHASE(1);
  {
    u32 dummy = 0;
    wave_amax(mx, dummy);
  }
  if (L == 0) red[w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  PHASE(2);
#pragma unroll
  for (u32 i = 0; i < 4; i++) {
    if (i < ni) {
      const u32 e = tid + 256 * i;
      p[i] = e < a.ne ? exp_f(p[i] - mx) : 0.0f;
      const float s = tree32_desc(p[i]);
      if ((L & 31) == 0) red[(tid >> 5) + 8 * i] = s;  // group (e / 32)
    }
  }
  __syncthreads();
  float tot = 0.0f;
  const u32 ng = (a.ne + 31) / 32;
  for (u32 g = 0; g < ng; g++) tot = tot + red[g];
  const float inv = 1.0f / tot;
#pragma unroll
  for (u32 i = 0; i < 4; i++) {
    const u32 e = tid + 256 * i;
    if (i < ni && e < a.ne) { p[i] = p[i] * inv; ps[e] = p[i]; }
  }
  __syncthreads();
  PHASE(3);
  // Selection in wave 0 alone (no block barriers inside). tau = the nk-th largest of the 64 strided
  // maxima m_l = max p[l + 64 j]: at least nk values are >= tau, so the nk-th largest value is >= tau
  // and every expert of the top k has p >= tau. The experts with p >= tau (the candidates) are
  // compacted by ballot and ranked among themselves; ranks below nk are the top k in order. More
  // than 64 candidates (heavy ties) fall back to a rank over every expert, block-wide.
  u32* ids = (u32*)(sm + TOPK_SIDS);  // [nk] in LDS; copied out when wr
  u32* cnt = (u32*)(red + 40);
  float* cv = wv + 64;                 // [64] candidate p
  u32* ci = (u32*)(cv + 256);          // [64] candidate expert
  float* lm = red + 64;                // [64] lane maxima
  if (w == 0) {
    // Order keys: (bits of p) << 32 | ~e. p >= 0, so its bits order like p; a larger key is a larger
    // p, then a lower index. -inf (and NaN) map to key 0, below every real p. tau comes from the 64
    // lane maxima by a radix select over their bits; the (at most 64) candidates are ranked by counting.
    u64* kk = (u64*)cv;  // [64] candidate keys
    if (L < a.nk) ids[L] = 0;  // a valid expert whatever happens below (NaN logits rank nothing)
    const u32 nj = (a.ne + 63) / 64;
    float pv[16];
#pragma unroll
    for (u32 j = 0; j < 16; j++) pv[j] = (j < nj && L + 64 * j < a.ne) ? ps[L + 64 * j] : -1.0f;  // p >= 0
    float m = pv[0];
#pragma unroll
    for (u32 j = 1; j < 16; j++)
      if (j < nj) m = fmaxf(m, pv[j]);
    // tau only has to be a lower bound of the nk-th largest p that leaves few candidates: the largest t
    // on a grid of 2^16 (sign, exponent and the top 7 mantissa bits of p >= 0, whose bits order like
    // its value) with at least nk lane maxima >= t -- so at least nk experts have p >= t -- by a
    // bitwise radix select over the maxima's top 16 bits (-inf and NaN lanes as 0)
    const u32 mb = (L < a.ne && m >= 0.0f) ? __float_as_uint(m) : 0u;
    PHASE(40);
    u32 tb = 0;
#pragma unroll
    for (int bit = 31; bit >= 16; bit--) {
      const u32 c = tb | (1u << bit);
      if ((u32)__popcll(__ballot(mb >= c)) >= a.nk) tb = c;
    }
    const float tau = __uint_as_float(tb);
    kk[L] = 0ull;
    WAVE_SYNC();
    PHASE(41);
    u32 base = 0;
#pragma unroll
    for (u32 j = 0; j < 16; j++) {
      if (j < nj) {
        const bool c = pv[j] >= tau;  // -1 (past ne) never is
        const u64 bal = __ballot(c);
        const u32 pos = base + __builtin_amdgcn_mbcnt_hi((u32)(bal >> 32), __builtin_amdgcn_mbcnt_lo((u32)bal, 0u));
        if (c && pos < 64) kk[pos] = ((u64)__float_as_uint(pv[j]) << 32) | (0xFFFFFFFFu - (L + 64 * j));
        base += (u32)__popcll(bal);
      }
    }
    WAVE_SYNC();
    PHASE(42);
    if (base <= 64) {
      // a candidate's rank is the number of larger keys among the candidates (keys are distinct: the
      // index is in the low word), read as LDS broadcasts; ranks below nk are the top k in order
      const u64 mine = kk[L];
      const u32 mhi = (u32)(mine >> 32), mlo = (u32)mine;
      u32 rk = 0;
      for (u32 j = 0; j < base; j++) {  // lane j's key, read across the wave (no LDS round trip)
        const u64 o = (u64)(u32)__builtin_amdgcn_readlane((int)mhi, (int)j) << 32 |
                      (u32)__builtin_amdgcn_readlane((int)mlo, (int)j);
        rk += o > mine ? 1u : 0u;
      }
      if (L < base && rk < a.nk) {  // fewer than nk candidates (NaN logits): the other slots keep expert 0
        ids[rk] = 0xFFFFFFFFu - (u32)mine;
        wv[rk] = __uint_as_float((u32)(mine >> 32));
      }
    }
    PHASE(43);
    if (L == 0) *cnt = base;
  }
  __syncthreads();
  if (*cnt > 64) {
    // heavy ties: rank over every expert
    u32 rk[4] = {0, 0, 0, 0};
    for (u32 q = 0; q < a.ne; q++) {
      const float v = ps[q];
#pragma unroll
      for (u32 i = 0; i < 4; i++) rk[i] += (v > p[i] || (v == p[i] && q < tid + 256 * i));
    }
#pragma unroll
    for (u32 i = 0; i < 4; i++) {
      const u32 e = tid + 256 * i;
      if (i < ni && e < a.ne && rk[i] < a.nk) { ids[rk[i]] = e; wv[rk[i]] = p[i]; }
    }
  }
  __syncthreads();
  PHASE(4);
  if (wr) topk_write(a, t, sm);
  PHASE(5);
}

__global__ void __launch_bounds__(256) k_topk(TopkArgs a) {
  __shared__ float sm[TOPK_LDS];
  topk_body256(a, blockIdx.x, sm, true);
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
// dm columns. x goes to LDS once; thread t owns span t % ns and walks rows t / ns, t / ns + 256 / ns,
// ... (gate rows even, up rows odd), so its slice of x is read once. Leaves [2 np][dm / 4] in LDS.
template <u32 FG, u32 FU>
DEV void gu_body(const GuArgs& a, u32 np, u32 bx, float* sm) {
  float* xs = sm;              // [dm]
  float* lv = sm + a.dm;       // [2 np][dm / 4]
  PHASE(8);
  const u32 task0 = bx * np, slot = task0 / a.ef, r0 = task0 % a.ef;
  const u32 t = slot / a.nk;
  const float* x = a.h2 + (u64)t * a.dm;
  for (u32 i = threadIdx.x; i < a.dm / 4; i += 256) ((float4*)xs)[i] = ((const float4*)x)[i];
  const u64 e = a.ids[slot];
  const u32 ns = a.dm / 32, ng = a.dm / 4, nr = 2 * np;
  __syncthreads();
  PHASE(9);
  const bool walk = 256 % ns == 0;  // fixed span column a thread: x read once for its rows
  for (u32 it = threadIdx.x; it < (walk ? ns * (256 / ns) : nr * ns); it += 256) {
    const u32 c = it % ns;
    float4 xv[8];
#pragma unroll
    for (u32 g = 0; g < 8; g++) xv[g] = ((const float4*)(xs + 32 * c))[g];
    for (u32 rr = it / ns; rr < nr; rr += walk ? 256 / ns : nr) {
      const u32 row = r0 + (rr >> 1);
      float w[32], l[8];
      if ((rr & 1) == 0) Span<FG>::w(a.G + e * a.es + row * a.rbg, 32 * c, w);
      else Span<FU>::w(a.U + e * a.es + row * a.rbu, 32 * c, w);
#pragma unroll
      for (u32 g = 0; g < 8; g++) l[g] = leaf4(w + 4 * g, xv[g]);
      store_leaves(lv + rr * ng + 8 * c, l);
    }
  }
  PHASE(10);
  __syncthreads();
  PHASE(11);
  const u32 rr = threadIdx.x >> 5, v = threadIdx.x & 31;
  for (u32 rb = 0; rb < nr; rb += 8) {
    const u32 r = rb + rr;
    float s = 0.0f;
    if (r < nr) s = stride_sum(lv + r * ng, ng, v);
    const float u = xpeer32(s);  // the up row sits in the other half of the wave
    if (r < nr && (r & 1) == 0 && v == 0) a.act[(u64)slot * a.ef + r0 + (r >> 1)] = silu_mul(s, u);
  }
  PHASE(12);
}
template <u32 FG, u32 FU>
__global__ void __launch_bounds__(256) k_gu_exact(GuArgs a, u32 np) {
  extern __shared__ float sm[];
  gu_body<FG, FU>(a, np, blockIdx.x, sm);
}

// ---- 8 lanes a row: llb_gemv_any's stride order with the partial sums in registers.
// Lane q of a row's 8 (c0 = q & 3, jh = q >> 2) holds virtual lanes v = 8 c0 + 4 jh + i (i < 4) of
// the 32-lane order: v sums leaves v, v + 32, v + 64, ... in turn, and leaf v + 32 m is leaf
// 4 jh + i of span c0 + 4 m. The xor tree's level 16 pairs lanes q ^ 2, level 8 q ^ 1, level 4 q
// and q + 4; levels 2 and 1 are inside the lane. The row's dot ends on lane q = 0.
DEV float fin8(float* acc) {
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = xadd2(acc[i]);
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = xadd1(acc[i]);
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = xadd4(acc[i]);
  return (acc[0] + acc[2]) + (acc[1] + acc[3]);
}
template <u32 F> DEV void acc16(const Half<F>& h, u32 c, u32 jh, const float* xs, float* acc) {
  float w[16];
  h.dec(32 * c, jh, w);
  const float4* xp = (const float4*)(xs + 32 * c + 16 * jh);
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = acc[i] + leaf4(w + 4 * i, xp[i]);
}
// NM spans a lane (cols = 128 NM), every raw load in flight before the caller waits for x
template <u32 F, u32 NM> struct Row8 {
  Half<F> h[NM];
  MDEV void ld(const u8* row, u32 q) {
#pragma unroll
    for (u32 m = 0; m < NM; m++) h[m].ld(row, 32 * ((q & 3) + 4 * m), q >> 2);
  }
  MDEV float dot(const float* xs, u32 q) const {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (u32 m = 0; m < NM; m++) acc16<F>(h[m], (q & 3) + 4 * m, q >> 2, xs, acc);
    return fin8(acc);
  }
};
// any cols (a multiple of 128): loads in the loop
template <u32 F> DEV float row8_dot(const u8* row, const float* xs, u32 cols, u32 q) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
  for (u32 m = 0; m < cols / 128; m++) {
    Half<F> h;
    h.ld(row, 32 * ((q & 3) + 4 * m), q >> 2);
    acc16<F>(h, (q & 3) + 4 * m, q >> 2, xs, acc);
  }
  return fin8(acc);
}

// gate + up + SwiGLU, 8 lanes a row: a block is 16 act rows of one slot (32 groups of 8 lanes, gate
// row on even groups, up row on odd ones, so lane 16 k + 8 holds the up dot of lane 16 k's gate row).
// Gate and up in one format.
template <u32 F, u32 NM>
__global__ void __launch_bounds__(256) k_gu_lane(GuArgs a) {
  extern __shared__ float xs[];  // [dm]
  PHASE(8);
  BSTAMP(2, 0);
  const u32 tid = threadIdx.x, gi = tid >> 3, q = tid & 7;
  const u32 task0 = blockIdx.x * 16, slot = task0 / a.ef, r = task0 % a.ef + (gi >> 1);
  const float* x = a.h2 + (u64)(slot / a.nk) * a.dm;
  const u64 e = a.ids[slot];
  const u8* row = (gi & 1) ? a.U + e * a.es + (u64)r * a.rbu : a.G + e * a.es + (u64)r * a.rbg;
  float s;
  if constexpr (NM != 0) {
    // issue order matters (vmcnt retires in order): x first, then the weights, so x reaches LDS
    // while the weights are still in flight
    static_assert(NM == 16, "x staging is written for dm = 2048: two float4 a thread");
    const float4 xv0 = ((const float4*)x)[tid], xv1 = ((const float4*)x)[tid + 256];
    __asm__ volatile("" ::: "memory");
    Row8<F, NM> w;
    w.ld(row, q);
    __asm__ volatile("" ::: "memory");
    PHASE(9);
    ((float4*)xs)[tid] = xv0;
    ((float4*)xs)[tid + 256] = xv1;
    __syncthreads();
    PHASE(10);
    s = w.dot(xs, q);
    PHASE(11);
  } else {
    for (u32 i = tid; i < a.dm / 4; i += 256) ((float4*)xs)[i] = ((const float4*)x)[i];
    __syncthreads();
    s = row8_dot<F>(row, xs, a.dm, q);
  }
  const float u = dppf<DPP_XOR8>(s);
  if ((tid & 15) == 0) a.act[(u64)slot * a.ef + r] = silu_mul(s, u);
  PHASE(12);
  BSTAMP(2, 1);
}

// down + rank-order combine + gated shared expert + residual (llb_moe_dn): rw rows of one token a
// block; task j < nk is routed expert ids[j]'s row against act_j, j = nk the shared expert's down
// row against sa (computed here from the shared gate / up logits)
template <u32 FD, u32 FS>
DEV void dn_body(const DnArgs& a, u32 bx, u32 t, float* sm) {
  const u32 nt = a.nk + (FS ? 1u : 0u);
  const u32 nge = a.ef / 4, ngs = a.sf / 4, per_row = a.nk * nge + (FS ? ngs : 0u);
  float* lv = sm;                                  // [rw][nk ef / 4 + sf / 4]
  float* sa = sm + a.rw * per_row;                 // [sf]
  float* part = sa + (FS ? a.sf : 0u);             // [rw][nt]
  PHASE(16);
  if (FS) {
    const float* g = a.gsu + (u64)t * 2 * a.sf;
    for (u32 i = threadIdx.x; i < a.sf; i += 256) sa[i] = silu_mul(g[i], g[a.sf + i]);
    __syncthreads();
  }
  PHASE(17);
  const float* act = a.act + (u64)t * a.nk * a.ef;
  // column q = one 32-column span of one task: q < nk ef / 32 routed (task q / (ef / 32)), then
  // the shared expert's; a thread loads its x slice once and walks the block's rw rows
  const u32 nse = a.ef / 32, nss = a.sf / 32, ncol = a.nk * nse + (FS ? nss : 0u);
  for (u32 q = threadIdx.x; q < ncol; q += 256) {
    const bool routed = q < a.nk * nse;
    const u32 j = routed ? q / nse : a.nk, sp = routed ? q % nse : q - a.nk * nse;
    const float* xsrc = routed ? act + (u64)j * a.ef + 32 * sp : sa + 32 * sp;
    float4 xv[8];
#pragma unroll
    for (u32 g = 0; g < 8; g++) xv[g] = ((const float4*)xsrc)[g];
    const u64 e = routed ? a.ids[(u64)t * a.nk + j] : 0;
    for (u32 rl = 0; rl < a.rw; rl++) {
      const u32 r = min(bx * a.rw + rl, a.dm - 1);
      float w[32], l[8];
      if (routed) Span<FD>::w(a.D + (e * a.dm + r) * a.rbd, 32 * sp, w);
      else Span<FS ? FS : FM_Q4_K>::w(a.SD + (u64)r * a.rbs, 32 * sp, w);
#pragma unroll
      for (u32 g = 0; g < 8; g++) l[g] = leaf4(w + 4 * g, xv[g]);
      store_leaves(lv + rl * per_row + j * nge + 8 * sp, l);
    }
  }
  PHASE(18);
  __syncthreads();
  PHASE(19);
  const u32 sums = a.rw * nt * 32;
  for (u32 q = threadIdx.x; q < ((sums + 63) & ~63u); q += 256) {
    const u32 k = q >> 5, v = q & 31;  // k = rl nt + j
    float s = 0.0f;
    if (q < sums) {
      const u32 rl = k / nt, j = k % nt;
      s = stride_sum(lv + rl * per_row + j * nge, j < a.nk ? nge : ngs, v);
    } else {
      s = stride_sum(lv, 0, v);  // keeps a partial wave's cross-lane steps uniform
    }
    if (q < sums && v == 0) part[k] = s;
  }
  __syncthreads();
  if (threadIdx.x < a.rw) {
    const u32 r = bx * a.rw + threadIdx.x;
    if (r < a.dm) {
      const float* wt = a.wt + (u64)t * a.nk;
      const float* pr = part + threadIdx.x * nt;
      float mo = 0.0f;
      for (u32 j = 0; j < a.nk; j++) mo = j == 0 ? pr[0] * wt[0] : mo + pr[j] * wt[j];
      const float res = a.x1 ? a.x1[(u64)t * a.dm + r] : 0.0f;
      a.y[(u64)t * a.dm + r] = FS ? (mo + pr[a.nk] * a.sgo[t]) + res : mo + res;
    }
  }
  PHASE(20);
}
template <u32 FD, u32 FS>
__global__ void __launch_bounds__(256) k_dn_exact(DnArgs a) {
  extern __shared__ float sm[];
  dn_body<FD, FS>(a, blockIdx.x, blockIdx.y, sm);
}

// top-k + gate + up + SwiGLU in one launch: each block recomputes its token's routing (the same
// topk_body256 as k_topk, so the same ids and weights) instead of reading ids written by a previous
// launch; the first block of each token writes ids / wt / sgo for the down kernel. Rows as k_gu_lane.
template <u32 F, u32 NM>
__global__ void __launch_bounds__(256) k_gu_topk(GuArgs a, TopkArgs k) {
  extern __shared__ float sm[];  // [TOPK_LDS] routing, then [dm] x
  float* xs = sm + TOPK_LDS;
  PHASE(8);
  BSTAMP(2, 0);
  const u32 tid = threadIdx.x, gi = tid >> 3, q = tid & 7;
  const u32 task0 = blockIdx.x * 16, slot = task0 / a.ef, r = task0 % a.ef + (gi >> 1);
  const u32 t = slot / a.nk, jr = slot % a.nk;
  const float* x = a.h2 + (u64)t * a.dm;
  float s;
  if constexpr (NM != 0) {
    static_assert(NM == 16, "x staging is written for dm = 2048: two float4 a thread");
    // x is loaded first (vmcnt retires in order) and reaches LDS once the routing is done
    const float4 xv0 = ((const float4*)x)[tid], xv1 = ((const float4*)x)[tid + 256];
    topk_body256(k, t, sm, false);
    const u64 e = ((const u32*)(sm + TOPK_SIDS))[jr];
    const u8* row = (gi & 1) ? a.U + e * a.es + (u64)r * a.rbu : a.G + e * a.es + (u64)r * a.rbg;
    Row8<F, NM> w;
    w.ld(row, q);
    __asm__ volatile("" ::: "memory");
    if (task0 % a.ef == 0 && jr == 0) topk_write(k, t, sm);  // once a token, behind the weight loads
    PHASE(9);
    ((float4*)xs)[tid] = xv0;
    ((float4*)xs)[tid + 256] = xv1;
    __syncthreads();
    PHASE(10);
    s = w.dot(xs, q);
    PHASE(11);
  } else {
    topk_body256(k, t, sm, task0 % a.ef == 0 && jr == 0);
    const u64 e = ((const u32*)(sm + TOPK_SIDS))[jr];
    const u8* row = (gi & 1) ? a.U + e * a.es + (u64)r * a.rbu : a.G + e * a.es + (u64)r * a.rbg;
    for (u32 i = tid; i < a.dm / 4; i += 256) ((float4*)xs)[i] = ((const float4*)x)[i];
    __syncthreads();
    s = row8_dot<F>(row, xs, a.dm, q);
  }
  const float u = dppf<DPP_XOR8>(s);
  if ((tid & 15) == 0) a.act[(u64)slot * a.ef + r] = silu_mul(s, u);
  PHASE(12);
  BSTAMP(2, 1);
}

// the q8 tier's gate + up + SwiGLU (llb_mx_gu): 256 threads = 32 row pairs of one slot, 4 lanes a row
// (row_q8), gate rows on lane groups 0..7 of a half wave and up rows on 8..15, so lane 32 + L holds
// the up dot of lane L's gate row. Tasks past the T nk ef routed rows are the shared expert's gate /
// up rows of token (task - T nk ef) / sf. With lq the block quantizes its token's x to q8_1 in LDS
// (k_q8_1's steps, the same bits); with top-k (one token) a routed block also recomputes the token's
// routing first (topk_body256, as k_gu_topk) and the token's first block writes ids / wt / sgo.
__global__ void __launch_bounds__(256) k_gu_q8(Q8Args a, TopkArgs k, u32 nslot, u32 lq, u32 topk) {
  extern __shared__ float4 gsm4[];  // [TOPK_LDS] routing (with top-k), then xq [dm], xd [dm / 32]
  float* sm = (float*)gsm4;
  const u32 tid = threadIdx.x, L = tid & 63, q = L >> 2, p = L & 3;
  const u32 pr = 8 * (tid >> 6) + (q & 7);
  const u32 task0 = blockIdx.x * 32;
  const bool routed = task0 < nslot * a.ef;
  u32 slot = 0, row, t;
  if (routed) {
    slot = task0 / a.ef;
    row = task0 % a.ef + pr;
    t = slot / a.nk;
  } else {
    const u32 kk = task0 - nslot * a.ef;
    t = kk / a.sf;
    row = kk % a.sf + pr;
  }
  // x in LDS or in memory: two call sites below, so each pointer keeps its address space (a select
  // between the two would make flat loads, whose waits also wait for the weight loads)
  signed char* lxq = (signed char*)(sm + (topk ? TOPK_LDS : 0));
  float2* lxd = (float2*)(lxq + a.dm);
  if (lq) q8_1_block256<16>(a.h2 + (u64)t * a.dm, a.dm, lxq, lxd);
  u64 e = 0;
  if (routed) {
    if (topk) {  // block-uniform
      topk_body256(k, t, sm, false);
      e = ((const u32*)(sm + TOPK_SIDS))[slot % a.nk];
      if (task0 % a.ef == 0 && slot % a.nk == 0) topk_write(k, t, sm);
    } else {
      e = a.ids[slot];
    }
  }
  if (lq) __syncthreads();  // x in LDS (topk_body256 ends on a barrier too)
  const u8* w;
  u32 f;
  float* out;
  if (routed) {
    w = q < 8 ? a.G + e * a.es + row * a.rbg : a.U + e * a.es + row * a.rbu;
    f = q < 8 ? a.fg : a.fu;
    out = a.act + (u64)slot * a.ef + row;
  } else {
    w = q < 8 ? a.SG + (u64)row * a.rbsg : a.SU + (u64)row * a.rbsu;
    f = q < 8 ? a.fsg : a.fsu;
    out = a.sa + (u64)t * a.sf + row;
  }
  const float v = lq ? row_q8_fm<8>(f, w, a.dm, lxq, lxd, p)
                     : row_q8_fm<8>(f, w, a.dm, a.hq + (u64)t * a.dm, a.hd + (u64)t * (a.dm / 32), p);
  const float u = __shfl_xor(v, 32, 64);
  if (q < 8 && p == 0) *out = silu_mul(v, u);
}

int launch_gu_q8(const Q8Args& a, const TopkArgs* tk, u32 nslot, u32 T, bool lq, hipStream_t st) {
  if (a.ef % 32 || a.sf % 32 || a.dm % 32 || (tk && (T != 1 || tk->ne > 1024 || tk->nk > 64))) return -1;
  if (lq && a.dm > 16 * 256) return -1;
  const u32 tasks = (u32)(((u64)nslot * a.ef + (u64)T * a.sf) / 32);
  const size_t sm = (tk ? (size_t)TOPK_LDS * 4 : 0) + (lq ? (size_t)a.dm * 5 / 4 : 0);
  if (sm > 65536) return -1;
  const TopkArgs k = tk ? *tk : TopkArgs{};
  LAUNCH_K(k_gu_q8, dim3(tasks), dim3(256), sm, st, a, k, nslot, (u32)lq, (u32)(tk != nullptr));
  return 0;
}

// down + rank-order combine + gated shared expert + residual, 8 lanes a row. A block takes R
// outputs of one token and their nt = nk (+ 1 shared) row dots: task k = j R + rl (expert-major, so
// a wave's groups share one act row and read neighbouring weight rows), tasks gi + 32 p (p < P) of
// the block's 32 groups (R nt <= 32 P). The shared down row has the routed rows' format and width
// (ef = sf = 128 NM).
//
// Issue order matters (vmcnt retires in order): ids, then act and the shared gate / up logits into
// registers, the combine's wt / sgo / x1, then the weights; act / sa reach LDS while the weights
// are in flight. The code around the loads is straight-line (per-lane branches make the compiler
// wait at the joins): tasks past the end load a valid row and are dropped, and staging steps past
// the end re-copy a word another thread copies too (index min(tid + 256 i, n - 256 + tid), n >= 256).
template <u32 F, u32 HS, u32 NM, u32 P>
__global__ void __launch_bounds__(256) k_dn_lane(DnArgs a, u32 R) {
  extern __shared__ float sm[];
  BSTAMP(3, 0);
  PHASE(16);
  const u32 nt = a.nk + HS, ntask = R * nt;
  float* xa = sm;                        // [nk][ef] act of the token's slots
  float* sa = xa + a.nk * a.ef;          // [sf]
  float* part = sa + (HS ? a.sf : 0u);   // [R][nt]
  float* wts = part + R * nt;            // [nk] wt, then sgo
  const u32 t = blockIdx.y, r0 = blockIdx.x * R;
  const u32 tid = threadIdx.x, gi = tid >> 3, q = tid & 7;
  u32 kind[P], eid[P];  // kind 0 none, 1 routed, 2 shared
#pragma unroll
  for (u32 p = 0; p < P; p++) {
    const u32 k = gi + 32 * p, j = k / R, r = r0 + k % R;
    kind[p] = (k < ntask && r < a.dm) ? (j < a.nk ? 1u : 2u) : 0u;
    eid[p] = a.ids[(u64)t * a.nk + min(j, a.nk - 1)];
  }
  PHASE_AFTER(21, eid[0]);
  const float4* act4 = (const float4*)(a.act + (u64)t * a.nk * a.ef);
  const u32 na4 = a.nk * a.ef / 4;  // 256 .. 2048
  // (separate variables, not arrays: the ordering fences below would keep an array in memory)
#define DN_AI(i) min(tid + 256u * (i), na4 - 256u + tid)
  const float4 av0 = act4[DN_AI(0)], av1 = act4[DN_AI(1)], av2 = act4[DN_AI(2)], av3 = act4[DN_AI(3)];
  const float4 av4 = act4[DN_AI(4)], av5 = act4[DN_AI(5)], av6 = act4[DN_AI(6)], av7 = act4[DN_AI(7)];
  float gg0 = 0.0f, gg1 = 0.0f, gu0 = 0.0f, gu1 = 0.0f;  // sf 256 or 512
  const u32 sc0 = min(tid, a.sf - 256u + tid), sc1 = min(tid + 256u, a.sf - 256u + tid);
  if (HS) {
    const float* g = a.gsu + (u64)t * 2 * a.sf;
    gg0 = g[sc0]; gg1 = g[sc1]; gu0 = g[a.sf + sc0]; gu1 = g[a.sf + sc1];
  }
  const float wtv = a.wt[(u64)t * a.nk + min(tid, a.nk - 1)];
  const float sgv = HS ? a.sgo[t] : 0.0f;
  const float x1v = a.x1 ? a.x1[(u64)t * a.dm + min(r0 + tid, a.dm - 1)] : 0.0f;
  PHASE_AFTER(22, x1v);
  // the scheduler may not move the weight loads above the staging loads, nor the LDS stores above them
  __asm__ volatile("" ::: "memory");
  // a pass whose tasks are all past the end for this wave (the third one, for most waves) loads
  // nothing: a wave-uniform test
  const u32 wv0 = 8 * (tid >> 6);  // the wave's first group
  Row8<F, NM> w[P];
#pragma unroll
  for (u32 p = 0; p < P; p++) {
    if (p < 2 || wv0 + 32 * p < ntask) {
      const u32 k = gi + 32 * p, r = min(r0 + k % R, a.dm - 1);
      const u8* drow = a.D + ((u64)eid[p] * a.dm + r) * a.rbd;
      w[p].ld(HS && kind[p] == 2 ? a.SD + (u64)r * a.rbs : drow, q);
    }
  }
  __asm__ volatile("" ::: "memory");
  PHASE(17);
  float4* xa4 = (float4*)xa;
  xa4[DN_AI(0)] = av0; xa4[DN_AI(1)] = av1; xa4[DN_AI(2)] = av2; xa4[DN_AI(3)] = av3;
  xa4[DN_AI(4)] = av4; xa4[DN_AI(5)] = av5; xa4[DN_AI(6)] = av6; xa4[DN_AI(7)] = av7;
#undef DN_AI
  if (HS) {
    sa[sc0] = silu_mul(gg0, gu0);
    sa[sc1] = silu_mul(gg1, gu1);
  }
  if (tid < a.nk) wts[tid] = wtv;
  __syncthreads();
  PHASE(18);
#pragma unroll
  for (u32 p = 0; p < P; p++) {
    if (p < 2 || wv0 + 32 * p < ntask) {
      const u32 k = gi + 32 * p, j = k / R, rl = k % R;
      const float s = w[p].dot(kind[p] == 2 ? sa : xa + min(j, a.nk - 1) * a.ef, q);
      if (kind[p] && q == 0) part[rl * nt + j] = s;
    }
  }
  __syncthreads();
  PHASE(19);
  if (tid < R && r0 + tid < a.dm) {
    const float* pr = part + tid * nt;
    float mo = 0.0f;
    for (u32 j = 0; j < a.nk; j++) mo = j == 0 ? pr[0] * wts[0] : mo + pr[j] * wts[j];
    a.y[(u64)t * a.dm + r0 + tid] = HS ? (mo + pr[a.nk] * sgv) + x1v : mo + x1v;
  }
  PHASE(20);
  BSTAMP(3, 1);
}

// ---------------------------------------------------------------- the fused decode layer
//
// One persistent launch runs a whole layer. Blocks take work items from a ticket counter in a
// fixed order -- tree rows (router, shared gate logit, shared gate / up), then one top-k item a
// token, then gate / up items, then down items -- and an item waits, where it must, for every item
// of the phase before it (a completion counter). Tickets are handed out in order, so an item only
// ever waits for items that running blocks already hold: no deadlock whatever the grid size. A
// wait is bounded (a wall-clock limit); past it the block records an error and carries on, so the
// grid always drains. The last block out zeroes the counters for the next launch.
//
// Cross-block visibility: a finished item's stores are released (agent-scope fence in every wave,
// then the block barrier) before its counter increment; a waiting block acquires (agent-scope
// fence in every wave) after it sees the count.

// A counter is read with a read-modify-write atomic, like the increments (L2 atomics), not with a
// cache-bypassing load, which on another XCD need not see them. The compiler turns an idempotent
// RMW (add 0) back into a load, so the read is a compare-exchange against a value the counter
// never holds: it fails and returns the current count, writing nothing.
DEV u32 ctr_read(u32* p) {
  u32 v = 0xFFFFFFFFu;
  __hip_atomic_compare_exchange_strong(p, &v, 0xFFFFFFFFu, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return v;
}

// wait until *ctr >= target, at most `limit` ticks of the 100 MHz wall clock
DEV void phase_wait(u32* ctr, u32 target, u32* err, u32 limit) {
  if (threadIdx.x == 0) {
    const u64 t0 = __builtin_amdgcn_s_memrealtime();
    while (ctr_read(ctr) < target) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > limit) {
        __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
  __threadfence();
}
DEV void item_done(u32* ctr) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <u32 FG, u32 FD, u32 FS, u32 NSP>
__global__ void __launch_bounds__(256) k_fused(FusedArgs f) {
  extern __shared__ float sm[];
  __shared__ u32 ticket;
  u32* c = f.ctr;  // [0] tickets, [1] tree done, [2] top-k done, [3] gate/up done, [4] blocks out, [5] error
  const u32 w = threadIdx.x >> 6, L = threadIdx.x & 63;
  const u32 nK = f.T, e1 = f.nR, e2 = e1 + nK, e3 = e2 + f.nG, total = e3 + f.nD;
  for (;;) {
    if (threadIdx.x == 0) ticket = __hip_atomic_fetch_add(&c[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const u32 it = ticket;
    __syncthreads();
    if (it >= total) break;
    if (it < e1) {
      const u32 t = it / f.rpt, sub = it % f.rpt;
      tree_body<NSP>(f.tr, 4 * sub + w, t, L, sm + w * tree_lds<NSP>());
      item_done(&c[1]);
    } else if (it < e2) {
      phase_wait(&c[1], f.nR, &c[5], f.spin);
      topk_body256(f.tk, it - e1, sm, true);
      item_done(&c[2]);
    } else if (it < e3) {
      phase_wait(&c[2], nK, &c[5], f.spin);
      gu_body<FG, FG>(f.gu, f.np, it - e2, sm);
      item_done(&c[3]);
    } else {
      phase_wait(&c[3], f.nG, &c[5], f.spin);
      const u32 k = it - e3;
      dn_body<FD, FS>(f.dn, k % f.dpt, k / f.dpt, sm);
    }
  }
  if (threadIdx.x == 0 && __hip_atomic_fetch_add(&c[4], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
    for (u32 i = 0; i < 5; i++) __hip_atomic_exchange(&c[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// ---------------------------------------------------------------- llb_rmsnorm_add (the step before the router)

// tools/payload-fuse.patch:106-127 and its other widths (tools/payload-w1024.patch:130-150,
// tools/payload-anyshape.patch:300-340): x1 = x + z; the squares of x1 summed by one balanced pairwise
// tree in column order over a power of two >= n (the reference's 1024 threads x 4, 8 or L leaves with
// +0 past n, then rms_tree's lane pairs t, t + 1, then t, t + 2 ...); s = 1 / sqrt(sum / n + eps), each op
// rounded once; h2 = (x1 s) w. One block of 256 a row: thread t holds leaves Q t .. Q t + Q - 1 of the
// tree over 256 Q >= n (the same sums: the extra leaves are +0), the in-lane levels, then tree64_asc
// across the wave (exact on lane 0), then the four waves as (w0 + w1) + (w2 + w3).
template <u32 Q>
__global__ void __launch_bounds__(256) k_rmsnorm_add(const float* __restrict__ x, const float* __restrict__ z,
                                                     const float* __restrict__ w, float eps, u32 n,
                                                     float* __restrict__ x1, float* __restrict__ h2) {
  __shared__ float ws[4];
  const u32 t = threadIdx.x, r = blockIdx.x;
  const float* xr = x + (u64)r * n;
  const float* zr = z + (u64)r * n;
  // the thread's leaves stay in registers for the output pass: one read of x and z
  float v[Q], b[Q];
  if constexpr (Q % 4 == 0) {  // n % 4 == 0 here (launcher): whole float4s, all in or all out
#pragma unroll
    for (u32 k = 0; k < Q; k += 4) {
      const u32 i = t * Q + k;
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f), c = a;
      if (i < n) {
        a = *(const float4*)(xr + i);
        c = *(const float4*)(zr + i);
      }
      v[k] = a.x + c.x; v[k + 1] = a.y + c.y; v[k + 2] = a.z + c.z; v[k + 3] = a.w + c.w;
    }
  } else {
#pragma unroll
    for (u32 k = 0; k < Q; k++) {
      const u32 i = t * Q + k;
      v[k] = i < n ? xr[i] + zr[i] : 0.0f;
    }
  }
#pragma unroll
  for (u32 k = 0; k < Q; k++) b[k] = t * Q + k < n ? v[k] * v[k] : 0.0f;
#pragma unroll
  for (u32 st = 1; st < Q; st <<= 1)
#pragma unroll
    for (u32 k = 0; k < Q; k += 2 * st) b[k] = b[k] + b[k + st];
  const float sw = tree64_asc(b[0]);
  if ((t & 63) == 0) ws[t >> 6] = sw;
  __syncthreads();
  const float sum = (ws[0] + ws[1]) + (ws[2] + ws[3]);
  // correctly rounded division and square root (HIP's / and __builtin_sqrtf; its __fsqrt_rn is the
  // native approximation unless OCML_BASIC_ROUNDED_OPERATIONS is set)
  const float s = 1.0f / __builtin_sqrtf(sum / (float)n + eps);
  if constexpr (Q % 4 == 0) {
#pragma unroll
    for (u32 k = 0; k < Q; k += 4) {
      const u32 i = t * Q + k;
      if (i < n) {
        const float4 wv = *(const float4*)(w + i);
        if (x1) *(float4*)(x1 + (u64)r * n + i) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
        *(float4*)(h2 + (u64)r * n + i) = make_float4((v[k] * s) * wv.x, (v[k + 1] * s) * wv.y, (v[k + 2] * s) * wv.z,
                                                      (v[k + 3] * s) * wv.w);
      }
    }
  } else {
#pragma unroll
    for (u32 k = 0; k < Q; k++) {
      const u32 i = t * Q + k;
      if (i < n) {
        if (x1) x1[(u64)r * n + i] = v[k];
        h2[(u64)r * n + i] = (v[k] * s) * w[i];
      }
    }
  }
}

int launch_rmsnorm_add(const float* x, const float* z, const float* w, float eps, u32 T, u32 n, float* x1, float* h2,
                       hipStream_t st) {
  if (n == 0 || n > 16384 || T == 0) return -1;
  u32 P = 256;
  while (P < n) P <<= 1;
  if (P >= 1024 && n % 4) return -1;  // the float4 path takes whole quads
  const dim3 grid(T);
#define RN_L(Qv) \
  if (P == 256 * Qv) { LAUNCH_K((k_rmsnorm_add<Qv>), grid, dim3(256), 0, st, x, z, w, eps, n, x1, h2); return 0; }
  RN_L(1) RN_L(2) RN_L(4) RN_L(8) RN_L(16) RN_L(32) RN_L(64)
#undef RN_L
  return -1;
}

// ---------------------------------------------------------------- launchers

#define FM_CASES(X) X(FM_Q8_0) X(FM_Q4_K) X(FM_Q6_K) X(FM_Q5_K)

// compute units of the current device (queried once)
static u32 cu_count() {
  static u32 n = 0;
  if (!n) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = (u32)v;
    else
      n = 256;
  }
  return n;
}

int launch_tree_rows(const TreeArgs& a, u32 nsp, hipStream_t st) {
  u32 rows = 0;
  for (u32 i = 0; i < a.nseg; i++) rows += a.seg[i].rows;
  if (rows == 0) return 0;
  if (a.nz && (a.T >= 16 || a.cols % 4)) return -1;  // the input step rides on the one-token-a-block kernel only
  if (a.T >= 16 && nsp <= 2) {  // token tiles: weights read once a tile
    const u32 tt = 4, nt = (a.T + tt - 1) / tt, slots = 2 * cu_count();
    const size_t sm = (size_t)tt * 64 * (32 * nsp + 4) * 4;
    // rows a wave: 4 (2 for two-span rows), which reads a token's x from LDS once per 4 rows, unless
    // the grid would then not fill one round of resident blocks (few tokens: batched decode); then 1
    u32 rw = nsp == 1 ? 4u : 2u;
    if ((u64)((rows + 4 * rw - 1) / (4 * rw)) * nt < slots) rw = 1;
    // tiles a block: the count that minimises (rounds of resident blocks) x (tiles a block + 2, a
    // block's own cost of loading its rows and filling its pipeline), two blocks resident a CU -- a
    // grid just past one round of blocks would otherwise take two
    const u32 rb = (rows + 4 * rw - 1) / (4 * rw);
    u32 ntb = 1;
    u64 best = ~0ull;
    for (u32 n = 1; n <= nt; n++) {
      const u64 blocks = (u64)rb * ((nt + n - 1) / n), cost = (blocks + slots - 1) / slots * (n + 2);
      if (cost < best) { best = cost; ntb = n; }
    }
    const dim3 grid(rb, (nt + ntb - 1) / ntb);
    static std::atomic<uint64_t> set{0};
    const uint64_t bit = dev_bit();
    if (dev_needs_setup(set, bit)) {
      (void)hipFuncSetAttribute((const void*)k_tree_rows_mt<1, 4, 4>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(4 * 64 * 36 * 4));
      (void)hipFuncSetAttribute((const void*)k_tree_rows_mt<1, 4, 1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(4 * 64 * 36 * 4));
      (void)hipFuncSetAttribute((const void*)k_tree_rows_mt<2, 4, 2>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(4 * 64 * 68 * 4));
      (void)hipFuncSetAttribute((const void*)k_tree_rows_mt<2, 4, 1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(4 * 64 * 68 * 4));
      set.fetch_or(bit);
    }
    if (nsp == 1 && rw == 4) LAUNCH_K((k_tree_rows_mt<1, 4, 4>), grid, dim3(256), sm, st, a, ntb);
    else if (nsp == 1) LAUNCH_K((k_tree_rows_mt<1, 4, 1>), grid, dim3(256), sm, st, a, ntb);
    else if (rw == 2) LAUNCH_K((k_tree_rows_mt<2, 4, 2>), grid, dim3(256), sm, st, a, ntb);
    else LAUNCH_K((k_tree_rows_mt<2, 4, 1>), grid, dim3(256), sm, st, a, ntb);
    return 0;
  }
  const u32 rpw = tree_rows_per_wave(nsp);
  dim3 grid((rows + rpw - 1) / rpw, a.T);
  if (nsp == 1) { LAUNCH_K((k_tree_rows<1>), grid, dim3(64), 0, st, a); return 0; }
  if (nsp == 2) { LAUNCH_K((k_tree_rows<2>), grid, dim3(64), 0, st, a); return 0; }
  if (nsp == 4) { LAUNCH_K((k_tree_rows<4>), grid, dim3(64), 0, st, a); return 0; }
  return -1;
}

int launch_topk(const TopkArgs& a, u32 T, hipStream_t st) {
  LAUNCH_K(k_topk, dim3(T), dim3(256), 0, st, a);
  return 0;
}

int launch_gu_exact(const GuArgs& a, u32 fg, u32 fu, u32 nslots, hipStream_t st) {
  if (fg != fu || a.ef % 16 || a.dm % 128) return -1;
  const dim3 grid(nslots * a.ef / 16);
  const size_t sm = (size_t)a.dm * 4;
#define GU_L(F) \
  if (fg == F) { \
    if (a.dm == 2048) LAUNCH_K((k_gu_lane<F, 16>), grid, dim3(256), sm, st, a); \
    else LAUNCH_K((k_gu_lane<F, 0>), grid, dim3(256), sm, st, a); \
    return 0; \
  }
  FM_CASES(GU_L)
#undef GU_L
  return -1;
}

int launch_gu_topk(const GuArgs& a, const TopkArgs& k, u32 fg, u32 fu, u32 nslots, hipStream_t st) {
  if (fg != fu || a.ef % 16 || a.dm % 128 || k.ne > 1024 || k.nk > 64) return -1;
  const dim3 grid(nslots * a.ef / 16);
  const size_t sm = ((size_t)TOPK_LDS + a.dm) * 4;
#define GU_L(F) \
  if (fg == F) { \
    if (a.dm == 2048) LAUNCH_K((k_gu_topk<F, 16>), grid, dim3(256), sm, st, a, k); \
    else LAUNCH_K((k_gu_topk<F, 0>), grid, dim3(256), sm, st, a, k); \
    return 0; \
  }
  FM_CASES(GU_L)
#undef GU_L
  return -1;
}

// rows a down block takes: each thread's x slice serves rw rows
u32 dn_rows(u32 nk, u32 ef, u32 sf) {
  (void)nk; (void)ef; (void)sf;
  return 4;
}

int launch_dn_exact(const DnArgs& a, u32 fd, u32 fs, u32 T, hipStream_t st) {
  const u32 nt = a.nk + (fs ? 1u : 0u);
  const u32 nm = a.ef / 128;
  // outputs a block: enough that one token's blocks fit the 256 CUs once (dm / 256), in two or
  // three passes of the 32 groups; otherwise R nt <= 64 in two passes
  u32 R = (a.dm + 255) / 256, P = 2;
  if (R * nt > 64) {
    if (R * nt <= 96 && nm <= 4) P = 3;
    else R = 64 / nt;
  }
  const bool lane = R >= 1 && (fs == 0 || (fs == fd && a.sf == a.ef)) && a.ef % 128 == 0 &&
                    (nm == 2 || nm == 4 || nm == 6 || nm == 8) && a.nk * a.ef >= 1024 && a.nk * a.ef <= 8192;
  if (lane) {
    const size_t lsm = ((size_t)a.nk * a.ef + (fs ? a.sf : 0) + (size_t)R * nt + a.nk) * 4;
    const dim3 grid((a.dm + R - 1) / R, T);
#define DN_N(F, HS, N) \
  if (nm == N) { \
    if (P == 2) LAUNCH_K((k_dn_lane<F, HS, N, 2>), grid, dim3(256), lsm, st, a, R); \
    else if constexpr (N <= 4) LAUNCH_K((k_dn_lane<F, HS, N, 3>), grid, dim3(256), lsm, st, a, R); \
    return 0; \
  }
#define DN_L(F) \
  if (fd == F) { \
    if (fs) { DN_N(F, 1, 2) DN_N(F, 1, 4) DN_N(F, 1, 6) DN_N(F, 1, 8) } \
    else { DN_N(F, 0, 2) DN_N(F, 0, 4) DN_N(F, 0, 6) DN_N(F, 0, 8) } \
  }
    FM_CASES(DN_L)
#undef DN_L
#undef DN_N
    return -1;
  }
  dim3 grid((a.dm + a.rw - 1) / a.rw, T);
  const size_t sm = ((size_t)a.rw * (a.nk * a.ef / 4 + (fs ? a.sf / 4 : 0)) + (fs ? a.sf : 0) + a.rw * nt) * 4;
#define DN_L(FD, FS) \
  if (fd == FD && fs == FS) { LAUNCH_K((k_dn_exact<FD, FS>), grid, dim3(256), sm, st, a); return 0; }
#define DN_FS(FD) DN_L(FD, 0u) DN_L(FD, FM_Q4_K) DN_L(FD, FM_Q6_K) DN_L(FD, FM_Q5_K)
  FM_CASES(DN_FS)
#undef DN_FS
#undef DN_L
  return -1;
}

// the fused path's format combinations (others take the four-launch path)
#define FUSED_CASES(X) \
  X(FM_Q8_0, FM_Q8_0, 0u) X(FM_Q4_K, FM_Q6_K, FM_Q6_K) X(FM_Q4_K, FM_Q6_K, 0u) X(FM_Q4_K, FM_Q4_K, 0u) \
  X(FM_Q4_K, FM_Q4_K, FM_Q6_K) X(FM_Q6_K, FM_Q6_K, FM_Q6_K) X(FM_Q5_K, FM_Q5_K, FM_Q4_K) X(FM_Q6_K, FM_Q8_0, FM_Q6_K)

size_t fused_lds(const FusedArgs& f) {
  const size_t gu = ((size_t)f.gu.dm + (size_t)2 * f.np * (f.gu.dm / 4)) * 4;
  const u32 nt = f.dn.nk + (f.dn.sf ? 1u : 0u);
  const size_t dn = ((size_t)f.dn.rw * (f.dn.nk * f.dn.ef / 4 + f.dn.sf / 4) + f.dn.sf + f.dn.rw * nt) * 4;
  const size_t tk = (size_t)TOPK_LDS * 4;  // topk_body256's LDS
  const size_t m = gu > dn ? gu : dn;
  const size_t tr = (size_t)4 * tree_lds<1>() * 4;  // four waves' tree x (one span a lane)
  const size_t m2 = m > tk ? m : tk;
  return m2 > tr ? m2 : tr;
}

// the fused layer's six counters to zero, by a kernel in the same stream (not a memset: the launch pair may
// be captured into a graph, where memset nodes have given wrong results on replay)
__global__ void __launch_bounds__(64) k_fused_clear(u32* c) {
  if (threadIdx.x < 6) c[threadIdx.x] = 0u;
}

int launch_fused(const FusedArgs& f, u32 fg, u32 fd, u32 fs, u32 nsp, u32 grid, hipStream_t st) {
  if (nsp != 1) return -1;  // its LDS holds four waves' tree x of one span a lane
  const size_t sm = fused_lds(f);
  // the counters start at zero at every launch, whatever an earlier call at another T or tier left in
  // the scratch (the last block out still resets them, which keeps a launch's own end state clean)
  if (!fused_supported(fg, fd, fs, nsp)) return -1;
  LAUNCH_K(k_fused_clear, dim3(1), dim3(64), 0, st, f.ctr);
#define FU_L(FG, FD, FS) \
  if (fg == FG && fd == FD && fs == FS) { \
    if (nsp == 1) { LAUNCH_K((k_fused<FG, FD, FS, 1>), dim3(grid), dim3(256), sm, st, f); return 0; } \
    if (nsp == 2) { LAUNCH_K((k_fused<FG, FD, FS, 2>), dim3(grid), dim3(256), sm, st, f); return 0; } \
  }
  FUSED_CASES(FU_L)
#undef FU_L
  return -1;
}
bool fused_supported(u32 fg, u32 fd, u32 fs, u32 nsp) {
#define FU_S(FG, FD, FS) if (fg == FG && fd == FD && fs == FS && (nsp == 1 || nsp == 2)) return true;
  FUSED_CASES(FU_S)
#undef FU_S
  return false;
}

// the path's exp (the float of the double exp, as every softmax, SwiGLU and sigmoid here uses it)
__global__ void __launch_bounds__(256) k_exp_f(const float* __restrict__ x, float* __restrict__ y, u64 n) {
  const u64 i = (u64)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = exp_f(x[i]);
}
int launch_exp(const float* x, float* y, u64 n, hipStream_t st) {
  if (n == 0) return 0;
  if ((n + 255) / 256 > 0x7fffffffull) return -1;
  hipLaunchKernelGGL(k_exp_f, dim3((u32)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
  return 0;
}

int launch_dequant(u32 fm, const u8* W, u64 rb, u32 rows, u32 cols, float* out, hipStream_t st) {
  const u64 n = (u64)rows * (cols / 32);
  dim3 grid((u32)((n + 255) / 256));
#define DQ_L(F) \
  if (fm == F) { LAUNCH_K((k_dequant<F>), grid, dim3(256), 0, st, W, rb, rows, cols, out); return 0; }
  FM_CASES(DQ_L) DQ_L(FM_F32)
#undef DQ_L
  return -1;
}
