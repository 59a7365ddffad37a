// moe_decode.hip -- the exact tier's one-token decode layer on gfx950, three launches:
//
//   k_router   router logits (+ the shared expert's gate logit): F32 rows in the engine tree order
//              (llb_warp / kp_pair, tools/remap.patch:116-171), one row a block of four waves
//   k_gu_dec   top-k (llb_moe_topk, tools/payload-moeany.patch:311-470) recomputed by every routed
//              block, then the chosen experts' gate / up rows and SwiGLU (llb_moe_gu, :477-525, the
//              moe_dot stride order); blocks past the routed ones take the shared expert's gate / up
//              rows in the tree order (llb_kgemv's tuned bodies)
//   k_dn_dec   the chosen experts' down rows, the shared expert's down row, the rank-order combine
//              and the residual (llb_moe_dn, :527-594)
//
// Every float op is the reference's, in its order (the library is built with -ffp-contract=off), so
// the outputs are bit for bit those of the reference's exact kernels and of the CPU oracle.
//
// Memory: a wave copies its weight rows into LDS with the CDNA4 LDS DMA (global_load_lds_dwordx4:
// 64 lanes x 16 consecutive bytes an instruction, every HBM byte fetched once in whole cache lines),
// then its lanes read the fields they decode from LDS. A lane decodes one 64-column group of a row
// (a K-quant sub-block pair: the 32 bytes that carry both nibbles, and its scales), so no byte is
// requested twice from the cache and each scale is decoded once for 32 weights. The group's 16
// leaves ((w0 x0 + w1 x1) + (w2 x2 + w3 x3), 4 columns each) are independent values; the reduction
// order is imposed afterwards:
//   stride order (moe_dot): leaves go to LDS at their leaf index; lane v of 32 then sums leaves
//       v, v + 32, ... in turn and the xor tree 16 .. 1 finishes (tree32_desc);
//   tree order: a lane's leaves are a subtree (in-lane levels), the upper levels pair lanes.
// The activations a lane multiplies (its group's 64 columns) stay in registers for all its rows.
#include "moe_dev.h"
#include "moe_kernels.h"
#include "moe_q8dot.h"

// per-block clock stamps for latency studies: a build that defines MOE_DEC_STAMPS records them; the
// library build compiles them away
#ifdef MOE_DEC_STAMPS
// stamp i of block b (thread 0; stamps 8..15 of k_gu_dec from thread 960, its last wave) in shader clocks
// (s_memtime), into the buffer the arguments carry (dec_stamps: [32][1024] u64, set by the host)
#define DSTAMP(i) do { if ((threadIdx.x == 0 || ((i) >= 8 && (i) < 16 && threadIdx.x == 960)) && blockIdx.x < 1024 && a.stamps) { \
    __builtin_amdgcn_sched_barrier(0); a.stamps[(i) * 1024 + blockIdx.x] = __builtin_readcyclecounter(); __builtin_amdgcn_sched_barrier(0); } } while (0)
// the host side: the decode launches pass this buffer
unsigned long long* g_dec_stamps = nullptr;
extern "C" void moe_dec_set_stamps(unsigned long long* p) { g_dec_stamps = p; }
#else
#define DSTAMP(i) do {} while (0)
#endif

typedef __attribute__((address_space(3))) void lds_void;
typedef u32 v4u __attribute__((ext_vector_type(4)));  // a 16-byte chunk in registers (uint4 copies lower to memcpy)

// 16 bytes a lane from g into LDS at lds + 16 * lane (lds wave-uniform): global_load_lds_dwordx4.
// Completion is tracked by vmcnt only; the compiler inserts no wait before the LDS reads of that
// data, so every reader waits with wait_vm first.
DEV void dma16(const void* g, void* lds) { __builtin_amdgcn_global_load_lds(g, (lds_void*)lds, 16, 0, 0); }

// s_waitcnt vmcnt(N) (lgkmcnt, expcnt untouched), and a compiler fence so no LDS read moves above it
template <u32 N> DEV void wait_vm() {
  static_assert(N < 64, "vmcnt has six bits");
  __builtin_amdgcn_s_waitcnt((int)((N & 15u) | ((N >> 4) << 14) | (7u << 4) | (15u << 8)));
  __asm__ volatile("" ::: "memory");
}
DEV void wait_vm0() { wait_vm<0>(); }
#define WAVE_FENCE() do { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); __builtin_amdgcn_wave_barrier(); } while (0)

DEV uint4 lds16(const u8* p) {  // 16 bytes from LDS at any 2-aligned address (ds_read_b128)
  uint4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}
DEV u32 lds_u16(const u8* p) { unsigned short v; __builtin_memcpy(&v, p, 2); return v; }

// x of column c in the padded LDS copy: 64-column groups 68 floats apart (conflict-free b128 reads)
DEV u32 xpad(u32 c) { return c + 4u * (c >> 6); }

// ---------------------------------------------------------------- a lane's 64-column group

// column of leaf i (0..15) of group q: K-quants with nibble-paired sub-blocks and Q8_0 hold columns
// 64 q .. 64 q + 63; Q6_K's group is the ql / qh bytes of quads a and a + 2 of half n of super-block
// s (q = 4 s + 2 n + a): columns 256 s + 128 n + 32 a + l and + 64
template <u32 F> DEV u32 leaf_col(u32 q, u32 i) {
  if constexpr (F == FM_Q6_K)
    return 256u * (q >> 2) + 128u * ((q >> 1) & 1u) + 32u * (q & 1u) + (i < 8 ? 4u * i : 64u + 4u * (i - 8));
  else
    return 64u * q + 4u * i;
}

// the 16 leaves of group q of a row whose bytes are at rp (LDS); x[i]: the lane's activations of leaf i.
// The weights are the reference's dequant values (q8g_w / q4k_w / q5k_w / q6k_w), as Span / Half give them.
template <u32 F> DEV void leaves64(const u8* rp, u32 q, const float* xs, float* lf);
// the activations of leaf i of group q, from the padded LDS copy
template <u32 F> DEV float4 xleaf(const float* xs, u32 q, u32 i);

template <> DEV void leaves64<FM_Q4_K>(const u8* rp, u32 q, const float* xs, float* lf) {
  constexpr u32 F_ = FM_Q4_K;
  const u8* B = rp + 144u * (q >> 2);
  const u32 g = q & 3u;
  const uint4 h = lds16(B), qa = lds16(B + 16 + 32 * g), qb = lds16(B + 32 + 32 * g);
  u32 sc0, mn0, sc1, mn1;
  k4_scmin(h, 2 * g, sc0, mn0);
  k4_scmin(h, 2 * g + 1, sc1, mn1);
  const float d = f16v(h.x & 0xffffu), dn = f16v(h.x >> 16);
  // sub-block 2 g: the low nibbles; 2 g + 1: the high nibbles masked in place (16 q), scaled by d sc / 16
  const float d0 = d * (float)sc0, m0 = dn * (float)mn0;
  const float d1 = d * (float)sc1 * 0.0625f, m1 = dn * (float)mn1;
  const u32 qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
  for (int k = 0; k < 8; k++) {
    float w[4];
    const u32 lo = opq(qw[k] & 0x0F0F0F0Fu), hi = opq(qw[k] & 0xF0F0F0F0u);
#pragma unroll
    for (int t = 0; t < 4; t++) w[t] = __builtin_fmaf(d0, ubyte(lo, t), -m0);
    lf[k] = leaf4(w, xleaf<F_>(xs, q, k));
#pragma unroll
    for (int t = 0; t < 4; t++) w[t] = __builtin_fmaf(d1, ubyte(hi, t), -m1);
    lf[8 + k] = leaf4(w, xleaf<F_>(xs, q, 8 + k));
  }
}

template <> DEV void leaves64<FM_Q5_K>(const u8* rp, u32 q, const float* xs, float* lf) {
  constexpr u32 F_ = FM_Q5_K;
  const u8* B = rp + 176u * (q >> 2);
  const u32 g = q & 3u, j0 = 2 * g, j1 = 2 * g + 1;
  const uint4 h = lds16(B), ha = lds16(B + 16), hb = lds16(B + 32);
  const uint4 qa = lds16(B + 48 + 32 * g), qb = lds16(B + 64 + 32 * g);
  u32 sc0, mn0, sc1, mn1;
  k4_scmin(h, j0, sc0, mn0);
  k4_scmin(h, j1, sc1, mn1);
  const float d = f16v(h.x & 0xffffu), dn = f16v(h.x >> 16);
  const float d0 = d * (float)sc0, m0 = dn * (float)mn0, d1 = d * (float)sc1, m1 = dn * (float)mn1;
  const u32 qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  const u32 hw[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
#pragma unroll
  for (int k = 0; k < 8; k++) {
    float w[4];
    const u32 lo = opq((qw[k] & 0x0F0F0F0Fu) | (((hw[k] >> j0) & 0x01010101u) << 4));
    const u32 hi = opq(((qw[k] >> 4) & 0x0F0F0F0Fu) | (((hw[k] >> j1) & 0x01010101u) << 4));
#pragma unroll
    for (int t = 0; t < 4; t++) w[t] = __builtin_fmaf(d0, ubyte(lo, t), -m0);
    lf[k] = leaf4(w, xleaf<F_>(xs, q, k));
#pragma unroll
    for (int t = 0; t < 4; t++) w[t] = __builtin_fmaf(d1, ubyte(hi, t), -m1);
    lf[8 + k] = leaf4(w, xleaf<F_>(xs, q, 8 + k));
  }
}

// Q6_K: each byte built as (q ^ 32) << 2, read as a signed byte (4 (q - 32)), times d sc / 4: the same
// exact product (d sc) (q - 32), with the same sign of zero (Half<FM_Q6_K>)
template <> DEV void leaves64<FM_Q6_K>(const u8* rp, u32 q, const float* xs, float* lf) {
  constexpr u32 F_ = FM_Q6_K;
  const u8* B = rp + 210u * (q >> 2);
  const u32 n = (q >> 1) & 1u, a = q & 1u;
  const uint4 la = lds16(B + 64 * n + 32 * a), lb = lds16(B + 64 * n + 32 * a + 16);
  const uint4 ha = lds16(B + 128 + 32 * n), hb = lds16(B + 128 + 32 * n + 16);
  const u32 s01 = lds_u16(B + 192 + 8 * n + 2 * a), s45 = lds_u16(B + 196 + 8 * n + 2 * a);
  const float d = f16v(lds_u16(B + 208));
  // scales: quad a's columns 0..15, 16..31 (s01), quad a + 2's (s45)
  const float ds[4] = {d * (float)(int)(signed char)(s01 & 255u) * 0.25f, d * (float)(int)(signed char)(s01 >> 8) * 0.25f,
                       d * (float)(int)(signed char)(s45 & 255u) * 0.25f, d * (float)(int)(signed char)(s45 >> 8) * 0.25f};
  const u32 lw[8] = {la.x, la.y, la.z, la.w, lb.x, lb.y, lb.z, lb.w};
  const u32 hw[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
  // quad a: the low nibble rotated into bits 2..5 (rotate left 2), high bits 2 a, 2 a + 1 into 6, 7;
  // quad a + 2: the high nibble (rotate right 2), high bits 2 a + 4, 2 a + 5
  const u32 hs0 = 6u - 2u * a, hs1 = 2u - 2u * a;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    float w[4];
    const u32 lo = opq(((__builtin_amdgcn_alignbit(lw[k], lw[k], 30) & 0x3C3C3C3Cu) | ((hw[k] << hs0) & 0xC0C0C0C0u)) ^ 0x80808080u);
    const u32 hi = opq(((__builtin_amdgcn_alignbit(lw[k], lw[k], 2) & 0x3C3C3C3Cu) | ((hw[k] << hs1) & 0xC0C0C0C0u)) ^ 0x80808080u);
    const float s0 = ds[k >> 2], s1 = ds[2 + (k >> 2)];
#pragma unroll
    for (int t = 0; t < 4; t++) w[t] = s0 * (float)(int)(signed char)((lo >> (8 * t)) & 255u);
    lf[k] = leaf4(w, xleaf<F_>(xs, q, k));
#pragma unroll
    for (int t = 0; t < 4; t++) w[t] = s1 * (float)(int)(signed char)((hi >> (8 * t)) & 255u);
    lf[8 + k] = leaf4(w, xleaf<F_>(xs, q, 8 + k));
  }
}

// Q8_0: blocks 2 q and 2 q + 1 (34 bytes each: f16 d, 32 signed codes); w = (q' - 128) d with q' the
// unsigned byte of q ^ 0x80 (exact products, the reference's sign of zero)
template <> DEV void leaves64<FM_Q8_0>(const u8* rp, u32 q, const float* xs, float* lf) {
  constexpr u32 F_ = FM_Q8_0;
  const u8* B = rp + 68u * q;
#pragma unroll
  for (int b = 0; b < 2; b++) {
    const u8* K = B + 34 * b;
    const float d = f16v(lds_u16(K));
    const uint4 qa = lds16(K + 2), qb = lds16(K + 18);
    const u32 qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float w[4];
      const u32 v = opq(qw[k] ^ 0x80808080u);
#pragma unroll
      for (int t = 0; t < 4; t++) w[t] = (ubyte(v, t) - 128.0f) * d;
      lf[8 * b + k] = leaf4(w, xleaf<F_>(xs, q, 8 * b + k));
    }
  }
}

template <u32 F> DEV float4 xleaf(const float* xs, u32 q, u32 i) {
  return *(const float4*)(xs + xpad(leaf_col<F>(q, i)));
}

// leaves to LDS at their leaf index (lv: the row's [cols / 4])
template <u32 F> DEV void put_leaves(float* lv, u32 q, const float* lf) {
#pragma unroll
  for (u32 i = 0; i < 16; i += 4)
    *(float4*)(lv + leaf_col<F>(q, i) / 4) = make_float4(lf[i], lf[i + 1], lf[i + 2], lf[i + 3]);
}

// moe_dot's order for vlane v (0..31) of a row whose nm = cols / 128 leaf columns are at lv: the
// sequential sums, then the xor tree 16 .. 1 (exact at lanes 0 and 32)
DEV float chain32(const float* lv, u32 nm, u32 v) {
  float acc = 0.0f;
  for (u32 m = 0; m < nm; m++) acc = acc + lv[32 * m + v];
  return tree32_desc(acc);
}
template <u32 NM> DEV float chain32c(const float* lv, u32 v) {
  float acc = 0.0f;
#pragma unroll
  for (u32 m = 0; m < NM; m++) acc = acc + lv[32 * m + v];
  return tree32_desc(acc);
}

// the engine tree over a row's 512 leaves (dm 2048: 32 lanes a row, exact on lanes 0 and 32): the lane's
// leaves are subtrees; the upper levels pair lanes
template <u32 F> DEV float tree_row(float* lf) {
  if constexpr (F == FM_Q6_K) {
    // two runs of 8 leaves (blocks 8 a and 16 + 8 a of the lane's 32-leaf group): in-lane, then the
    // blocks of the two lanes of the group, then the group's two halves, then the groups
#pragma unroll
    for (u32 st = 1; st < 8; st <<= 1)
#pragma unroll
      for (u32 i = 0; i < 8; i += 2 * st) { lf[i] = lf[i] + lf[i + st]; lf[8 + i] = lf[8 + i] + lf[8 + i + st]; }
    const float r0 = xadd1(lf[0]), r1 = xadd1(lf[8]);
    return xadd16(xadd8(xadd4(xadd2(r0 + r1))));
  } else {
#pragma unroll
    for (u32 st = 1; st < 16; st <<= 1)
#pragma unroll
      for (u32 i = 0; i < 16; i += 2 * st) lf[i] = lf[i] + lf[i + st];
    return xadd16(xadd8(xadd4(xadd2(xadd1(lf[0])))));
  }
}

// ---------------------------------------------------------------- top-k in one wave

// llb_moe_topk block 0 for one token, in one wave (ne <= 1024, nk <= 64): lane L holds experts
// L + 64 i (i < NI). mx = max lg; v = exp(lg - mx) (through double); the sum in the 1024-thread block's
// order (each 32-expert group by the xor tree 16 .. 1, then the group sums in order from group 0);
// p = v (1 / sum).
// Selection: a p >= 0 maps to the key kb = bits(p) + 1, which orders like p (0: no expert -- past ne,
// or a NaN p). Each lane sorts its NI (key, expert) pairs, larger key first and the lower expert first
// among equal keys; then nk rounds each take the wave's largest head (a DPP max over the lane heads),
// the lowest expert among the lanes holding it, and pop that lane's head. Round r's pick is rank r of
// the reference's order (p descending, ties to the lower index), so lane r keeps it. Rounds without a
// real p left keep expert 0 with p 0, so every id addresses a valid expert.
struct TopkLane {
  u32 id;
  float p;
};
DEV float wave_fmax(float v) {
  v = fmaxf(v, dppf<DPP_XOR1>(v));
  v = fmaxf(v, dppf<DPP_XOR2>(v));
  v = fmaxf(v, dppf<DPP_UP4>(v));
  v = fmaxf(v, dppf<DPP_XOR8>(v));
  v = fmaxf(v, xpeer32(v));  // rows r and r ^ 2, then below r ^ 1
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
DEV u32 umax_(u32 a, u32 b) { return a > b ? a : b; }
DEV u32 wave_umax(u32 v) {
  v = umax_(v, dppu<DPP_XOR1>(v));
  v = umax_(v, dppu<DPP_XOR2>(v));
  v = umax_(v, dppu<DPP_UP4>(v));
  v = umax_(v, dppu<DPP_XOR8>(v));
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  v = umax_(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return umax_(b[0], b[1]);
}
DEV float rlane(float v, u32 l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)l)); }
// (key, expert) pairs: a before b when a's key is larger, or equal with the lower expert
DEV void cx(u32& ka, u32& ea, u32& kb, u32& eb) {
  const bool sw = kb > ka || (kb == ka && eb < ea);
  const u32 tk = sw ? kb : ka, te = sw ? eb : ea;
  kb = sw ? ka : kb;
  eb = sw ? ea : eb;
  ka = tk;
  ea = te;
}
template <u32 NI>
DEV TopkLane topk_wave(const float* lg, u32 ne, u32 nk) {
  const u32 L = __lane_id();
  float v[NI];
  float mx = bits_f(0xFF800000u);
#pragma unroll
  for (u32 i = 0; i < NI; i++) {
    const u32 e = L + 64 * i;
    v[i] = e < ne ? lg[e] : 0.0f;
    if (e < ne) mx = fmaxf(mx, v[i]);
  }
  mx = wave_fmax(mx);
  // group sums in order; groups past ne sum to +0, which leaves a sum of non-negative terms unchanged
  float tot = 0.0f;
#pragma unroll
  for (u32 i = 0; i < NI; i++) {
    v[i] = L + 64 * i < ne ? exp_f(v[i] - mx) : 0.0f;
    const float s = tree32_desc(v[i]);
    tot = tot + rlane(s, 0);
    tot = tot + rlane(s, 32);
  }
  const float inv = 1.0f / tot;
  u32 k[NI], ex[NI];
#pragma unroll
  for (u32 i = 0; i < NI; i++) {
    const float p = v[i] * inv;
    k[i] = (L + 64 * i < ne && p >= 0.0f) ? __float_as_uint(p) + 1u : 0u;
    ex[i] = L + 64 * i;
  }
  // the lane's pairs sorted (odd-even transposition: NI rounds of neighbour exchanges)
#pragma unroll
  for (u32 r = 0; r < NI; r++)
#pragma unroll
    for (u32 i = r & 1; i + 1 < NI; i += 2) cx(k[i], ex[i], k[i + 1], ex[i + 1]);
  TopkLane out{0u, 0.0f};
  for (u32 r = 0; r < nk; r++) {  // branch-free: two DPP maxima, selects
    const u32 m = wave_umax(k[0]);
    // the lowest expert among the heads equal to m (experts < 1024, so 1023 - e orders them)
    const u32 e = 1023u - wave_umax(k[0] == m && m != 0u ? 1023u - ex[0] : 0u);
    if (L == r) { out.id = m ? e : 0u; out.p = m ? __uint_as_float(m - 1u) : 0.0f; }
    const bool pop = m != 0u && ex[0] == e;
#pragma unroll
    for (u32 i = 0; i + 1 < NI; i++) { k[i] = pop ? k[i + 1] : k[i]; ex[i] = pop ? ex[i + 1] : ex[i]; }
    k[NI - 1] = pop ? 0u : k[NI - 1];
  }
  return out;
}
// The same routing by a block of 1024 threads (ne <= 512, nk <= 16; the gate / up block's waves are
// idle until it is known). Expert e on thread e for the softmax (group sums in order, as above). The
// 64-bit keys kb << 32 | ~e (a larger key is a larger p, then a lower index; all distinct) go to LDS.
// A key's place in its 64-expert group is the count of the group's larger keys, four threads a key
// (16 compares each); only a group's first nk can be in the top nk, so places below nk become
// candidates, in place order. A candidate's rank is its place plus the count of larger candidates of
// the other groups, again spread over threads (one (candidate, group) pair a thread). Ranks below nk
// name the slots. A key without a real p (past ne, or NaN) fills no slot; unfilled slots keep
// expert 0, p 0.
// LDS: keys [512] u64, candidates [8 x 16] u64, counts [1024] u8 (as u32 words), red [64] f32,
// slots [64] u32 + [64] f32 (slot j's expert at sid[j] when it returns). Every thread calls it; thread
// j < nk returns slot j.
constexpr u32 TKB_LDS = 512 * 8 + 128 * 8 + 1024 + 64 * 4 + 64 * 8;
#ifdef MOE_DEC_STAMPS
#define TSTAMP(i) do { if (threadIdx.x == 0 && stamps) { __builtin_amdgcn_sched_barrier(0); stamps[(i) * 1024 + blockIdx.x] = __builtin_readcyclecounter(); __builtin_amdgcn_sched_barrier(0); } } while (0)
#else
#define TSTAMP(i) do {} while (0)
#endif
template <u32 NP>
DEV TopkLane topk_block(const float* lg, u32 ne, u32 nk, u8* tl, float* xs, float4 xv,
                        unsigned long long* stamps = nullptr) {
  static_assert(NP == 256 || NP == 512, "64-expert groups, 1024 threads");
  unsigned long long* key = (unsigned long long*)tl;             // [NP]
  unsigned long long* cand = key + 512;                          // [NW][16]
  u8* cnt = (u8*)(cand + 128);                                   // [1024]
  float* red = (float*)(cnt + 1024);
  u32* sid = (u32*)(red + 64);
  float* sp = (float*)(sid + 64);
  const u32 t = threadIdx.x, L = t & 63, w = t >> 6;
  constexpr u32 NW = NP / 64;       // expert groups (waves that hold experts)
  constexpr u32 PK = 1024 / NP;     // threads a key for its place (4 or 2)
  constexpr u32 PZ = 64 / PK;       // keys each of them compares (16 or 32)
  float v = 0.0f;
  if (t < NP) {
    v = t < ne ? lg[t] : 0.0f;
    __asm__ volatile("" :: "v"(v));
    TSTAMP(11);
    const float mw = wave_fmax(t < ne ? v : bits_f(0xFF800000u));
    if (L == 0) red[w] = mw;
  }
  if (t < 64) { sid[t] = 0u; sp[t] = 0.0f; }
  __syncthreads();
  TSTAMP(12);
  if (t < 512) *(float4*)(xs + xpad(4 * t)) = xv;
  float mx = red[0];
#pragma unroll
  for (u32 i = 1; i < NW; i++) mx = fmaxf(mx, red[i]);
  if (t < NP) {
    v = t < ne ? exp_f(v - mx) : 0.0f;
    const float sg = tree32_desc(v);
    if ((L & 31) == 0) red[16 + (t >> 5)] = sg;  // group t / 32
  }
  __syncthreads();
  if (t < NP) {
    float tot = 0.0f;
#pragma unroll
    for (u32 g = 0; g < 2 * NW; g++) tot = tot + red[16 + g];  // groups past ne sum to +0
    const float p = v * (1.0f / tot);
    const u32 kb = (t < ne && p >= 0.0f) ? __float_as_uint(p) + 1u : 0u;
    key[t] = ((u64)kb << 32) | (0xFFFFFFFFu - t);
  }
  __syncthreads();
  TSTAMP(13);
  {  // key j's larger keys among part s of its group
    const u32 j = t % NP, sg = t / NP;
    const u64 mine = key[j];
    const u64* kp = (const u64*)key + (j & ~63u) + sg * PZ;
    u32 c = 0;
#pragma unroll
    for (u32 i = 0; i < PZ; i++) c += kp[i] > mine ? 1u : 0u;
    cnt[sg * NP + j] = (u8)c;
  }
  __syncthreads();
  const u32 nc = min(nk, 16u);  // candidates a group
  if (t < NP) {
    u32 r = 0;
#pragma unroll
    for (u32 s2 = 0; s2 < PK; s2++) r += cnt[s2 * NP + t];
    if (r < nc) cand[w * 16 + r] = key[t];
  }
  __syncthreads();
  TSTAMP(14);
  // candidate c = (group g, place q) against group o: thread (g, q, o), 16 x NW x NW <= 1024 threads
  {
    const u32 g = t / (16 * NW), q = (t / NW) % 16, o = t % NW;
    u32 c = 0;
    if (g < NW && q < nc && o != g) {
      const u64 mine = cand[g * 16 + q];
#pragma unroll
      for (u32 i = 0; i < 16; i++) c += (i < nc && cand[o * 16 + i] > mine) ? 1u : 0u;
    }
    if (t < 16 * NW * NW) cnt[t] = (u8)c;
  }
  __syncthreads();
  if (t < 16 * NW) {
    const u32 g = t / 16, q = t % 16;
    if (q < nc) {
      u32 rk = q;
#pragma unroll
      for (u32 o = 0; o < NW; o++) rk += cnt[t * NW + o];
      const u64 mine = cand[g * 16 + q];
      if (rk < nk && (mine >> 32) != 0ull) {
        sid[rk] = 0xFFFFFFFFu - (u32)mine;
        sp[rk] = __uint_as_float((u32)(mine >> 32) - 1u);
      }
    }
  }
  __syncthreads();
  TopkLane out{0u, 0.0f};
  if (t < 64) { out.id = sid[t]; out.p = sp[t]; }
  return out;
}

// The same routing for ne <= 256 with four barriers instead of seven (selected by DecGuArgs::lean).
// Expert e on thread e (waves 0..3 hold the four 64-expert groups); max and group sums as topk_block.
// A key's place in its group is counted in registers: lane L compares its key with the 64 keys of its
// wave read one lane at a time (readlane), no LDS and no barrier. Places below nc = min(nk, 16) go to
// LDS as candidates (other places: key 0, below every real key). Wave 0 then ranks the 64 candidate
// slots (lane g 16 + q: group g's place q) by counting larger candidates among all 64, again by
// readlane; ranks below nk with a real p name the slots. Same keys, same order, same results as
// topk_block. LDS: the candidates at topk_block's candidate offset, red and the slots at its offsets.
DEV TopkLane topk_block4(const float* lg, u32 ne, u32 nk, u8* tl, float* xs, float4 xv) {
  unsigned long long* cand = (unsigned long long*)tl + 512;  // [4][16]
  float* red = (float*)(tl + 512 * 8 + 128 * 8 + 1024);
  u32* sid = (u32*)(red + 64);
  float* sp = (float*)(sid + 64);
  const u32 t = threadIdx.x, L = t & 63, w = t >> 6;
  const u32 nc = min(nk, 16u);
  float v = 0.0f;
  if (t < 256) {
    v = t < ne ? lg[t] : 0.0f;
    const float mw = wave_fmax(t < ne ? v : bits_f(0xFF800000u));
    if (L == 0) red[w] = mw;
  }
  if (t < 64) { sid[t] = 0u; sp[t] = 0.0f; }
  __syncthreads();
  if (t < 512) *(float4*)(xs + xpad(4 * t)) = xv;
  float mx = red[0];
#pragma unroll
  for (u32 i = 1; i < 4; i++) mx = fmaxf(mx, red[i]);
  if (t < 256) {
    v = t < ne ? exp_f(v - mx) : 0.0f;
    const float sg = tree32_desc(v);
    if ((L & 31) == 0) red[16 + (t >> 5)] = sg;
  }
  __syncthreads();
  if (t < 256) {
    float tot = 0.0f;
#pragma unroll
    for (u32 g = 0; g < 8; g++) tot = tot + red[16 + g];
    const float p = v * (1.0f / tot);
    const u32 kb = (t < ne && p >= 0.0f) ? __float_as_uint(p) + 1u : 0u;
    const u32 klo = 0xFFFFFFFFu - t;
    u32 place = 0;
#pragma unroll
    for (u32 i = 0; i < 64; i++) {
      const u32 hi = (u32)__builtin_amdgcn_readlane((int)kb, (int)i), lo = (u32)__builtin_amdgcn_readlane((int)klo, (int)i);
      place += (hi > kb || (hi == kb && lo > klo)) ? 1u : 0u;
    }
    if (place < nc) cand[w * 16 + place] = ((u64)kb << 32) | klo;
    if (L < 16 && L >= nc) cand[w * 16 + L] = 0ull;
  }
  __syncthreads();
  if (t < 64) {
    const u64 mine = cand[t];
    const u32 mh = (u32)(mine >> 32), ml = (u32)mine;
    u32 rk = 0;
#pragma unroll
    for (u32 i = 0; i < 64; i++) {
      const u32 hi = (u32)__builtin_amdgcn_readlane((int)mh, (int)i), lo = (u32)__builtin_amdgcn_readlane((int)ml, (int)i);
      rk += (hi > mh || (hi == mh && lo > ml)) ? 1u : 0u;
    }
    if ((t & 15) < nc && rk < nk && mh != 0u) {
      sid[rk] = 0xFFFFFFFFu - ml;
      sp[rk] = __uint_as_float(mh - 1u);
    }
  }
  __syncthreads();
  TopkLane out{0u, 0.0f};
  if (t < 64) { out.id = sid[t]; out.p = sp[t]; }
  return out;
}

// wt_j = p_j / max(sum of the nk p in rank order, 2^-14) on lane j
DEV float topk_renorm(const TopkLane& t, u32 nk) {
  float s = 0.0f;
  for (u32 j = 0; j < nk; j++) s = s + rlane(t.p, j);
  s = s < 6.103515625e-5f ? 6.103515625e-5f : s;
  return t.p / s;
}

// ---------------------------------------------------------------- the router launch

// F32 rows, the engine tree over 2^cdepth leaves (leaf = 4 columns, +0 past cols): lane L holds the
// leaves 64 q + L, q < NQ; a block of four waves takes one row, wave w the q in [QW w, QW w + QW).
// Per q the six lane levels (tree64_asc, exact on lane 0), then the wave's in-lane levels over its q,
// then the four wave sums as the tree's top two levels. Rows: ne router rows, then the shared gate row.
// With the input step (nz set) each wave recomputes the token's norm over the whole row, as
// k_rmsnorm_add sums it, and block 0 stores x1 and h2.
template <u32 NQ>
__global__ void __launch_bounds__(256) k_router(TreeArgs a) {
  constexpr u32 QW = NQ / 4;
  __shared__ float part[4];
  DSTAMP(24);
  const u32 tid = threadIdx.x, L = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const u32 nl4 = a.cols / 4;
  // row r of segment 0 (router) or 1 (the shared gate row); fields picked by selects, not an index
  const bool s1 = blockIdx.x >= a.seg[0].rows;
  const u32 r = s1 ? blockIdx.x - a.seg[0].rows : blockIdx.x;
  const u8* W = s1 ? a.seg[1].W : a.seg[0].W;
  float* out = s1 ? a.seg[1].out : a.seg[0].out;
  const float* bias = s1 ? a.seg[1].bias : a.seg[0].bias;
  const float4* wr = (const float4*)(W + (u64)r * a.cols * 4);
  float4 wv[QW], xv[QW];
#pragma unroll
  for (u32 k = 0; k < QW; k++) {
    const u32 q = QW * w + k;
    wv[k] = 64 * q + L < nl4 ? wr[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (a.nz) {
    const float4* x4 = (const float4*)a.x;
    const float4* z4 = (const float4*)a.nz;
    const float4* n4 = (const float4*)a.nw;
    float4 v[NQ];
#pragma unroll
    for (u32 q = 0; q < NQ; q++) {
      const bool in = 64 * q + L < nl4;
      const float4 xa = in ? x4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 za = in ? z4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
      v[q] = make_float4(xa.x + za.x, xa.y + za.y, xa.z + za.z, xa.w + za.w);
    }
    float4 nwv[QW];
#pragma unroll
    for (u32 k = 0; k < QW; k++) {
      const u32 q = QW * w + k;
      nwv[k] = 64 * q + L < nl4 ? n4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float n[NQ];
#pragma unroll
    for (u32 q = 0; q < NQ; q++)
      n[q] = tree64_asc((v[q].x * v[q].x + v[q].y * v[q].y) + (v[q].z * v[q].z + v[q].w * v[q].w));
#pragma unroll
    for (u32 st = 1; st < NQ; st <<= 1)
#pragma unroll
      for (u32 q = 0; q < NQ; q += 2 * st) n[q] = n[q] + n[q + st];
    const float sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, n[0])));
    const float sc = 1.0f / __builtin_sqrtf(sum / (float)a.cols + a.eps);  // correctly rounded, as k_rmsnorm_add
#pragma unroll
    for (u32 k = 0; k < QW; k++) {
      const u32 q = QW * w + k;
      float4 x1 = v[0];
#pragma unroll
      for (u32 qq = 1; qq < NQ; qq++)
        if (qq == q) x1 = v[qq];
      xv[k] = make_float4((x1.x * sc) * nwv[k].x, (x1.y * sc) * nwv[k].y, (x1.z * sc) * nwv[k].z, (x1.w * sc) * nwv[k].w);
      if (blockIdx.x == 0 && 64 * q + L < nl4) {
        ((float4*)a.x1o)[64 * q + L] = x1;
        ((float4*)a.h2o)[64 * q + L] = xv[k];
      }
    }
  } else {
    const float4* x4 = (const float4*)a.x;
#pragma unroll
    for (u32 k = 0; k < QW; k++) {
      const u32 q = QW * w + k;
      xv[k] = 64 * q + L < nl4 ? x4[64 * q + L] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float n[QW];
#pragma unroll
  for (u32 k = 0; k < QW; k++) n[k] = tree64_asc(leaf4((const float*)&wv[k], xv[k]));
#pragma unroll
  for (u32 st = 1; st < QW; st <<= 1)
#pragma unroll
    for (u32 k = 0; k < QW; k += 2 * st) n[k] = n[k] + n[k + st];
  if (L == 0) part[w] = n[0];
  __syncthreads();
  if (tid == 0) {
    const float v = (part[0] + part[1]) + (part[2] + part[3]);
    out[r] = bias ? v + bias[r] : v;
  }
  DSTAMP(25);
}

int launch_router(const TreeArgs& a, u32 nq, hipStream_t st) {
  u32 rows = 0;
  for (u32 i = 0; i < a.nseg; i++) {
    if (a.seg[i].fm != FM_F32) return -1;
    rows += a.seg[i].rows;
  }
  if (a.T != 1 || rows == 0 || a.nseg > 2) return -1;
  if (nq == 8) { LAUNCH_K((k_router<8>), dim3(rows), dim3(256), 0, st, a); return 0; }
  if (nq == 16) { LAUNCH_K((k_router<16>), dim3(rows), dim3(256), 0, st, a); return 0; }
  if (nq == 32) { LAUNCH_K((k_router<32>), dim3(rows), dim3(256), 0, st, a); return 0; }
  return -1;
}

// ---------------------------------------------------------------- the q8 tier's activations and dots

// q8_1 (pf_q8x's quantizer) of 4 consecutive values a lane, eight lanes a 32-block (lanes 8 m .. 8 m + 7
// hold block m's float4s in column order): d = amax / 127, q = roundf(x / d) in [-127, 127], s = the
// block's sum (in lane-group order: the q8 tier's sums are checked to a tolerance, not to an order).
// Returns the four codes packed; d and s come back on every lane of the group.
DEV u32 q8_quad(float4 x, float& d_out, float& s_out) {
  float a = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
  float s = (x.x + x.y) + (x.z + x.w);
#pragma unroll
  for (u32 m = 1; m < 8; m <<= 1) {
    a = fmaxf(a, __shfl_xor(a, m, 64));
    s = s + __shfl_xor(s, m, 64);
  }
  const float d = a / 127.0f;
  auto code = [&](float v) -> u32 {
    return a == 0.0f ? 0u : (u32)(u8)(signed char)max(-127, min(127, (int)roundf(v / d)));
  };
  d_out = d;
  s_out = s;
  return code(x.x) | code(x.y) << 8 | code(x.z) << 16 | code(x.w) << 24;
}

// blocks 2 q and 2 q + 1 of a row (its bytes at rp, in LDS) against the q8_1 activations xq / xd (LDS)
template <u32 F> DEV float pair_blocks_q8(const u8* rp, u32 q, const u32* xq, const float2* xd) {
  float v = 0.0f;
#pragma unroll
  for (u32 bb = 0; bb < 2; bb++) {
    const u32 b = 2 * q + bb;
    const uint4 x0 = lds16((const u8*)(xq + 8 * b)), x1 = lds16((const u8*)(xq + 8 * b + 4));
    const u32 x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    v += blk_q8<F>(rp, b, x, xd[b]);
  }
  return v;
}

// ---------------------------------------------------------------- gate / up (+ SwiGLU), one token

// LDS of k_gu_dec (bytes): x (dm = 2048, padded) | routing: ids [64], candidates [64] u64 | the pairs'
// gate / up dots [32][2] | per wave: one staged pair (gate row | up row), the pair's leaves [2][512]
constexpr u32 DEC_DM = 2048;
constexpr u32 DN_RB_G = 8;  // outputs a down block takes (DN_RB below)
// row bytes of 2048 columns
static constexpr u32 rb2048(u32 f) {
  return f == FM_Q8_0 ? 2176u : f == FM_Q4_K ? 1152u : f == FM_Q5_K ? 1408u : f == FM_Q6_K ? 1680u : 0u;
}
constexpr u32 DEC_XS = (DEC_DM + DEC_DM / 16) * 4;  // 8704
constexpr u32 DEC_TK = 64 * 4 + 64 * 8;              // 768
constexpr u32 DEC_GU = 32 * 2 * 4;                   // 256
constexpr u32 DEC_LV = 2 * (DEC_DM / 4) * 4;         // 4096
constexpr u32 GU_WAVES = 16;
constexpr u32 gu_wave_lds(u32 rb) { return 2 * rb + DEC_LV; }
constexpr u32 DEC_TKB = TKB_LDS;  // topk_block's LDS
constexpr u32 gu_lds(u32 rb) { return DEC_XS + DEC_TK + DEC_GU + DEC_TKB + GU_WAVES * gu_wave_lds(rb); }

// one row pair, staged by the wave: the 16-byte chunks of [gate row | up row] (RB bytes each, 16-aligned),
// chunk c = 64 k + L, loaded coalesced into registers (lanes past the end re-load the last chunk)
template <u32 RB> struct PairChunks {
  static constexpr u32 CP = 2 * (RB / 16), NR = (CP + 63) / 64;
  v4u ch[NR];
  MDEV void load(const u8* g, const u8* u, u32 L) {
#pragma unroll
    for (u32 k = 0; k < NR; k++) {
      const u32 c = min(L + 64 * k, CP - 1);
      ch[k] = *(const v4u*)(c < RB / 16 ? g + 16 * c : u + 16 * (c - RB / 16));
    }
  }
  MDEV void store(u8* stage, u32 L) const {
#pragma unroll
    for (u32 k = 0; k < NR; k++)
      if (L + 64 * k < CP) *(v4u*)(stage + 16 * (L + 64 * k)) = ch[k];
  }
};

// the pair's dots on lane 0 (gate) and lane 32 (up): moe_dot's stride order (routed rows), or the
// engine tree (the shared expert's rows)
template <u32 F, u32 RB, bool TREE>
DEV float pair_compute(u8* stage, float* lv, const float* xs, u32 L) {
  const u32 h = L >> 5, q = L & 31;
  float lf[16];
  leaves64<F>(stage + h * RB, q, xs, lf);
  if constexpr (TREE) {
    return tree_row<F>(lf);
  } else {
    put_leaves<F>(lv + h * (DEC_DM / 4), q, lf);
    WAVE_FENCE();
    return chain32c<DEC_DM / 128>(lv + h * (DEC_DM / 4), q);
  }
}
template <u32 F, u32 RB, bool TREE>
DEV float pair_dots(const PairChunks<RB>& pc, u8* stage, float* lv, const float* xs, u32 L) {
  pc.store(stage, L);
  WAVE_FENCE();
  return pair_compute<F, RB, TREE>(stage, lv, xs, L);
}
// the q8 tier's pair: lane q of each half takes blocks 2 q, 2 q + 1 of its row; the 32 partial sums meet
// in an xor tree (lane 0: the gate dot, lane 32: the up dot)
template <u32 F, u32 RB>
DEV float pair_compute_q8(const u8* stage, const u32* xq, const float2* xd, u32 L) {
  float v = pair_blocks_q8<F>(stage + (L >> 5) * RB, L & 31, xq, xd);
#pragma unroll
  for (u32 m = 16; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// A block of 16 waves takes 16 consecutive features of one slot, one a wave: the feature's gate row on
// lanes 0..31 and its up row on lanes 32..63, each lane one 64-column group. Wave 0 routes the token
// first (every block recomputes it; block 0 writes ids / wt / sgo). The shared expert's gate / up rows
// (tree order) are spread over the blocks, waves 1, 2, ... taking shared feature b, b + nblocks, ...
// (their loads go out before the routing is known). SwiGLU is applied once a block, a lane a feature.
template <u32 F, u32 FS, u32 NI, bool Q8>
__global__ void __launch_bounds__(1024) k_gu_dec(DecGuArgs a) {
  extern __shared__ uint4 dsm[];
  DSTAMP(0);
  constexpr u32 RB = rb2048(F), RBS = rb2048(FS), RBX = RB > RBS ? RB : RBS;
  u8* sm = (u8*)dsm;
  float* xs = (float*)sm;
  u32* tk_id = (u32*)(sm + DEC_XS);
  float* gus = (float*)(sm + DEC_XS + DEC_TK);
  const u32 tid = threadIdx.x, L = tid & 63;
  const u32 w = __builtin_amdgcn_readfirstlane(tid >> 6);
  u8* tkb = sm + DEC_XS + DEC_TK + DEC_GU;
  u8* stage = tkb + DEC_TKB + w * gu_wave_lds(RBX);
  float* lv = (float*)(stage + 2 * RBX);
  const u32 bps = a.ef / GU_WAVES, slot = blockIdx.x / bps, f = (blockIdx.x % bps) * GU_WAVES + w;
  // the shared feature this wave takes (waves 1 ..), or none
  const u32 sfeat = blockIdx.x + gridDim.x * (w - 1);
  const bool has_s = FS != 0 && w >= 1 && sfeat < a.sf;
  PairChunks<RBS> sc;
  if constexpr (FS != 0)
    if (has_s) sc.load(a.SG + (u64)sfeat * RBS, a.SU + (u64)sfeat * RBS, L);
  // x, loaded now (its latency overlaps the routing's) and stored to LDS, padded, once routed
  const float4 xv = tid < 512 ? ((const float4*)a.h2)[tid] : make_float4(0.f, 0.f, 0.f, 0.f);
  TopkLane tl{0u, 0.0f};
  const u32* ids_s = tk_id;  // the token's experts by rank, in LDS
  bool routed_ok = false;
  if constexpr (NI <= 8) {
    if (a.tk.nk <= 16) {  // the routing by the whole block; x goes to LDS on the way; its last barrier
                          // publishes the slots
      if (NI == 4 && a.lean) {
        tl = topk_block4(a.tk.lg, a.tk.ne, a.tk.nk, tkb, xs, xv);
      } else {
#ifdef MOE_DEC_STAMPS
        tl = topk_block<64 * NI>(a.tk.lg, a.tk.ne, a.tk.nk, tkb, xs, xv, a.stamps);
#else
        tl = topk_block<64 * NI>(a.tk.lg, a.tk.ne, a.tk.nk, tkb, xs, xv);
#endif
      }
      ids_s = (const u32*)(tkb + 512 * 8 + 128 * 8 + 1024 + 64 * 4);
      routed_ok = true;
    }
  }
  if (!routed_ok) {  // the one-wave routing (more experts, or more than 16 slots)
    if (w == 0) {
      tl = topk_wave<NI>(a.tk.lg, a.tk.ne, a.tk.nk);
      if (L < a.tk.nk) tk_id[L] = tl.id;
    }
    if (tid < 512) *(float4*)(xs + xpad(4 * tid)) = xv;
    __syncthreads();
    ids_s = tk_id;
  }
  // the q8 tier: x as q8_1 over the x copy (whose float values this tier does not read): codes [2048],
  // then {d, s} [64]; waves 0 .. 7 hold x in xv
  u32* xq = (u32*)xs;
  float2* xd = (float2*)(sm + DEC_DM);
  if constexpr (Q8) {
    if (tid < 512) {
      float d, sum;
      xq[tid] = q8_quad(xv, d, sum);
      if ((tid & 7u) == 0) xd[tid >> 3] = make_float2(d, sum);
    }
    __syncthreads();
  }
  DSTAMP(1);
  DSTAMP(2);
  DSTAMP(8);
  const u64 e = ids_s[slot % a.nk];
  PairChunks<RB> pc;
  pc.load(a.G + e * a.es + (u64)f * RB, a.U + e * a.es + (u64)f * RB, L);
  DSTAMP(3);
  const u32 q = L & 31;
  if constexpr (FS != 0) {
    if (has_s) {
      float sv;
      if constexpr (Q8) {
        sc.store(stage, L);
        WAVE_FENCE();
        sv = pair_compute_q8<FS, RBS>(stage, xq, xd, L);
      } else {
        sv = pair_dots<FS, RBS, true>(sc, stage, lv, xs, L);
      }
      if (L == 0) gus[2 * (16 + w - 1)] = sv;
      if (L == 32) gus[2 * (16 + w - 1) + 1] = sv;
      WAVE_FENCE();
    }
  }
  pc.store(stage, L);
  WAVE_FENCE();
  DSTAMP(7);
  DSTAMP(10);
  // the down launch's rows for its block b3 = blockIdx (same XCD, so the same L2): task w's DN_RB rows,
  // one dword a 128-byte line, issued once this wave's own rows have landed. It is a plain load held in
  // place by a scheduling barrier; its value feeds only an empty asm statement at the end, so the wait
  // for it comes last.
  u32 touch = 0;
  {
    // waves past the tasks, and grids where this block has no down block, touch expert 0's first line
    const u32 b3 = blockIdx.x < a.ndb ? blockIdx.x : 0u;
    const bool sh = a.SD && w == a.nk;
    const u64 rb = sh ? a.rbs : a.rbd;
    const u8* base = sh ? a.SD + (u64)(DN_RB_G * b3) * rb
                        : a.D + ((u64)ids_s[min(w, a.nk - 1)] * a.dm + DN_RB_G * b3) * rb;
    // (pointer arithmetic, not integers, so the load stays a global load: a flat one would also count
    // against the LDS wait counter)
    // line L of the rows: its first dword, but never below base (line 0 when base is not 128-aligned,
    // which for expert 0 would read before the stack) and never past the rows' last byte
    const u8* lo = base - ((u32)(uintptr_t)base & 127u);
    const u8* p = L == 0 ? base : lo + 128 * L;
    const bool live = w < a.nk + (a.SD ? 1u : 0u) && p + 4 <= base + DN_RB_G * rb;
    touch = *(const u32*)(live ? p : a.D);
    __builtin_amdgcn_sched_barrier(0);
  }
  float sv;
  if constexpr (Q8) sv = pair_compute_q8<F, RB>(stage, xq, xd, L);
  else sv = pair_compute<F, RB, false>(stage, lv, xs, L);
  if (L == 0) gus[2 * w] = sv;
  if (L == 32) gus[2 * w + 1] = sv;
  DSTAMP(4);
  DSTAMP(9);
  __syncthreads();
  DSTAMP(5);
  if (w == 0) {
    // lanes 0..15: the block's routed features; 16 + k: shared feature blockIdx + gridDim k
    const u32 ns = FS ? min(15u, (a.sf > blockIdx.x ? (a.sf - blockIdx.x + gridDim.x - 1) / gridDim.x : 0u)) : 0u;
    if (L < 16 + ns) {
      const float g = gus[2 * L], u = gus[2 * L + 1];
      const float av = silu_mul(g, u);
      if (L < 16) {
        a.act[(u64)slot * a.ef + (blockIdx.x % bps) * GU_WAVES + L] = av;
      } else {
        const u32 sf_i = blockIdx.x + gridDim.x * (L - 16);
        a.sa[sf_i] = av;
        a.gsu[sf_i] = g;
        a.gsu[a.sf + sf_i] = u;
      }
    }
    if (blockIdx.x == 0) {
      const float wt = topk_renorm(tl, a.tk.nk);
      if (L < a.tk.nk) {
        a.tk.ids[L] = tl.id;
        a.tk.wt[L] = wt;
      }
      if (L == 0) {
        const float sg = a.tk.has_sg ? a.tk.lg[a.tk.ne] : 0.0f;
        a.tk.sgo[0] = 1.0f / (1.0f + exp_f(-sg));
      }
    }
  }
  wait_vm0();
  __asm__ volatile("" :: "v"(touch));
  DSTAMP(6);
}

// ---------------------------------------------------------------- down + combine, one token

// A block of nt = nk (+ 1 shared) waves takes DN_RB consecutive outputs: wave j < nk the rows of expert
// ids[j] against act_j, wave nk the shared down rows against sa. Each wave stages its own rows (LDS DMA)
// and its own activations (a wave-local LDS copy), so nothing waits on another wave until the combine.
// A lane decodes 64-column group q of one row (LPR = cols / 64 lanes a row, 64 / LPR rows a pass);
// part[DN_RB][16] holds the dots; threads < DN_RB combine them: ((v0 wt0 + v1 wt1 + ...) in rank
// order + hv sgo) + x1.
constexpr u32 DN_RB = DN_RB_G;
constexpr u32 DN_PART = DN_RB * 16 * 4;                 // part, bytes
// a wave's LDS: staged rows | its activations (padded) | leaves [<= 1024]
DEV u32 dn_wave_lds(const DecDnArgs& a) { return a.stage_bytes + a.xw_bytes + 4096; }

template <u32 F>
DEV void dn_rows(const u8* rows, u64 rb, u32 cols, u32 nrow, const float* xw, float* lv, float* part, u32 w, u32 L) {
  const u32 lpr = cols / 64, rpp = 64 / lpr, rho = L / lpr, q = L % lpr, nm = cols / 128;
  for (u32 p0 = 0; p0 < nrow; p0 += rpp) {
    const u32 rr = p0 + rho;
    if (rho < rpp && rr < nrow) {
      float lf[16];
      leaves64<F>(rows + rr * rb, q, xw, lf);
      put_leaves<F>(lv + rho * (cols / 4), q, lf);
    }
    WAVE_FENCE();
    const u32 np = min(rpp, nrow - p0);
    for (u32 c = 0; c < np; c += 2) {  // two rows an iteration, 32 vlanes each
      const u32 rl = c + (L >> 5);
      const float sv = chain32(lv + min(rl, np - 1) * (cols / 4), nm, L & 31);
      if ((L & 31) == 0 && rl < np) part[(p0 + rl) * 16 + w] = sv;
    }
    WAVE_FENCE();
  }
}

// the q8 tier's rows: lane (rho, q) takes blocks 2 q, 2 q + 1 of row rho of the pass; the row's lpr
// partial sums go through LDS (lpr need not be a power of two) and its first lane adds them in order
template <u32 F>
DEV void dn_rows_q8(const u8* rows, u64 rb, u32 cols, u32 nrow, const u32* xq, const float2* xd, float* lv,
                    float* part, u32 w, u32 L) {
  const u32 lpr = cols / 64, rpp = 64 / lpr, rho = L / lpr, q = L % lpr;
  for (u32 p0 = 0; p0 < nrow; p0 += rpp) {
    const u32 rr = p0 + rho;
    const bool live = rho < rpp && rr < nrow;
    lv[L] = live ? pair_blocks_q8<F>(rows + rr * rb, q, xq, xd) : 0.0f;
    WAVE_FENCE();
    if (live && q == 0) {
      float v = lv[L];
      for (u32 i = 1; i < lpr; i++) v += lv[L + i];
      part[rr * 16 + w] = v;
    }
    WAVE_FENCE();
  }
}

template <u32 FD, u32 FS, bool Q8>
__global__ void __launch_bounds__(1024) k_dn_dec(DecDnArgs a) {
  extern __shared__ uint4 dsm[];
  u8* sm = (u8*)dsm;
  const u32 tid = threadIdx.x, L = tid & 63;
  const u32 w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const u32 nk = a.nk;
  const u32 r0 = blockIdx.x * DN_RB;
  DSTAMP(16);
  const bool shared = FS && w == nk;
  const u32 cols = shared ? a.sf : a.ef;
  const u64 rb = shared ? a.rbs : a.rbd;
  const u32 nrow = min(DN_RB, a.dm - r0);
  // the wave's rows: one byte window [a16, b16) of the stack, 16-aligned (stacks are 16-aligned and a
  // multiple of 16 bytes long), into its staging area by the LDS DMA
  const u8* base = shared ? a.SD + (u64)r0 * rb : a.D + ((u64)a.ids[w] * a.dm + r0) * rb;
  float* part = (float*)sm;
  u8* wl = sm + DN_PART + w * dn_wave_lds(a);
  u8* stage = wl;
  float* xw = (float*)(wl + a.stage_bytes);
  float* lv = (float*)(wl + a.stage_bytes + a.xw_bytes);
  const uintptr_t a0 = (uintptr_t)base, a16 = a0 & ~(uintptr_t)15, b16 = (a0 + nrow * rb + 15) & ~(uintptr_t)15;
  const u32 nch = (u32)((b16 - a16) / 16);
  for (u32 k = 0; 64 * k < nch; k++) {
    const u32 c = L + 64 * k;
    if (c < nch) dma16((const u8*)a16 + 16 * (u64)c, stage + 1024 * k);
  }
  DSTAMP(17);
  // the wave's activations: act_j or sa, coalesced, to its padded LDS copy
  const float4* xsrc = (const float4*)(shared ? a.sa : a.act + (u64)w * a.ef);
  u32* xq = (u32*)xw;  // the q8 tier: codes [cols], then {d, s} [cols / 32]
  float2* xd = (float2*)(xq + cols / 4);
  if constexpr (Q8) {
    for (u32 i = L; i < cols / 4; i += 64) {  // cols % 256 == 0: every lane takes part in each round
      float d, sum;
      xq[i] = q8_quad(xsrc[i], d, sum);
      if ((i & 7u) == 0) xd[i >> 3] = make_float2(d, sum);
    }
  } else {
    for (u32 i = L; i < cols / 4; i += 64) *(float4*)(xw + xpad(4 * i)) = xsrc[i];
  }
  // the combine's inputs
  const float wtv = tid < nk ? a.wt[tid] : 0.0f;
  const float sgv = FS ? a.sgo[0] : 0.0f;
  const float x1v = (a.x1 && tid < nrow) ? a.x1[r0 + tid] : 0.0f;
  WAVE_FENCE();
  wait_vm0();  // the rows are in LDS
  DSTAMP(19);
  const u8* rows = stage + (a0 - a16);
  if constexpr (Q8) {
    if (shared) {
      if constexpr (FS != 0) dn_rows_q8<FS>(rows, rb, cols, nrow, xq, xd, lv, part, w, L);
    } else {
      dn_rows_q8<FD>(rows, rb, cols, nrow, xq, xd, lv, part, w, L);
    }
  } else if (shared) {
    if constexpr (FS != 0) dn_rows<FS>(rows, rb, cols, nrow, xw, lv, part, w, L);
  } else {
    dn_rows<FD>(rows, rb, cols, nrow, xw, lv, part, w, L);
  }
  DSTAMP(21);
  __shared__ float wsh[16];
  if (tid < nk) wsh[tid] = wtv;
  __syncthreads();
  if (tid < nrow) {
    const float* pr = part + tid * 16;
    float mo = 0.0f;
    for (u32 j = 0; j < nk; j++) mo = j == 0 ? pr[0] * wsh[0] : mo + pr[j] * wsh[j];
    a.y[r0 + tid] = FS ? (mo + pr[nk] * sgv) + x1v : mo + x1v;
  }
  DSTAMP(22);
}

// ---------------------------------------------------------------- launchers

template <u32 F, u32 FS, bool Q8>
static int gu_dec_one(const DecGuArgs& a, hipStream_t st) {
  constexpr u32 RB = rb2048(F), RBS = rb2048(FS);
  constexpr size_t lds = gu_lds(RB > RBS ? RB : RBS);
  static_assert(lds <= 160 * 1024, "LDS of the gate / up block");
  static std::atomic<uint64_t> set{0};
  const uint64_t bit = dev_bit();
  if (dev_needs_setup(set, bit)) {
    if (hipFuncSetAttribute((const void*)k_gu_dec<F, FS, 4, Q8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess ||
        hipFuncSetAttribute((const void*)k_gu_dec<F, FS, 8, Q8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess ||
        hipFuncSetAttribute((const void*)k_gu_dec<F, FS, 16, Q8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess) {
      (void)hipGetLastError();
      return -1;
    }
    set.fetch_or(bit);
  }
  // experts a lane holds in top-k (ne / 64, rounded up to 4, 8 or 16)
  if (a.tk.ne <= 256) LAUNCH_K((k_gu_dec<F, FS, 4, Q8>), dim3(a.nrb), dim3(64 * GU_WAVES), lds, st, a);
  else if (a.tk.ne <= 512) LAUNCH_K((k_gu_dec<F, FS, 8, Q8>), dim3(a.nrb), dim3(64 * GU_WAVES), lds, st, a);
  else LAUNCH_K((k_gu_dec<F, FS, 16, Q8>), dim3(a.nrb), dim3(64 * GU_WAVES), lds, st, a);
  return 0;
}

int launch_gu_dec(DecGuArgs a, u32 f, u32 fs, bool q8, hipStream_t st) {
  if (a.dm != DEC_DM || a.ef % GU_WAVES || a.tk.ne > 1024 || a.tk.nk > 64) return -1;
  a.nrb = a.nk * a.ef / GU_WAVES;
  // the shared features: at most 15 a block (waves 1 .. 15)
  if (fs && a.sf > 15 * a.nrb) return -1;
#define GU_FS(F, FS) \
  if (f == F && fs == FS) return q8 ? gu_dec_one<F, FS, true>(a, st) : gu_dec_one<F, FS, false>(a, st);
#define GU_F(F) GU_FS(F, 0u) GU_FS(F, FM_Q4_K) GU_FS(F, FM_Q5_K) GU_FS(F, FM_Q6_K)
  GU_F(FM_Q8_0) GU_F(FM_Q4_K) GU_F(FM_Q5_K) GU_F(FM_Q6_K)
#undef GU_F
#undef GU_FS
  return -1;
}

template <u32 FD, u32 FS, bool Q8>
static int dn_dec_one(const DecDnArgs& a, u32 nt, size_t lds, hipStream_t st) {
  static std::atomic<size_t> set[64];  // per device: the dynamic LDS the kernel is allowed so far
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    dev = 0;
  }
  if (dev >= 64 || lds > set[dev].load()) {
    if (hipFuncSetAttribute((const void*)k_dn_dec<FD, FS, Q8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
        hipSuccess) {
      (void)hipGetLastError();
      return -1;
    }
    if (dev < 64) set[dev].store(lds);
  }
  LAUNCH_K((k_dn_dec<FD, FS, Q8>), dim3((a.dm + DN_RB - 1) / DN_RB), dim3(64 * nt), lds, st, a);
  return 0;
}

// the down launch's LDS for these shapes, or 0 when it cannot take them
size_t dn_dec_lds(u32 nk, u32 ef, u32 sf, u64 rbd, u64 rbs, u32 dm, bool shared, bool q8, u32* stage_bytes,
                  u32* xw_bytes) {
  const u32 nt = nk + (shared ? 1u : 0u);
  const u32 cm = q8 ? 256u : 128u;  // (the q8 tier quantizes a wave's activations 256 at a time)
  if (nt > 16 || ef % cm || ef > 4096 || (shared && (sf % cm || sf > 4096)) || dm % DN_RB) return 0;
  const u64 rbmax = rbd > rbs ? rbd : rbs;
  const u32 sb = (u32)((DN_RB * rbmax + 32 + 15) & ~(u64)15);
  const u32 cmax = ef > sf ? ef : sf;
  // float activations, padded (exact), or q8_1 codes and {d, s} (q8)
  const u32 xb = q8 ? (cmax + cmax / 32 * 8 + 15) & ~15u : (cmax + cmax / 16) * 4;
  const size_t lds = DN_PART + (size_t)nt * (sb + xb + 4096);
  if (lds > 160 * 1024 - 256) return 0;  // (and 64 bytes of static LDS)
  if (stage_bytes) *stage_bytes = sb;
  if (xw_bytes) *xw_bytes = xb;
  return lds;
}

int launch_dn_dec(DecDnArgs a, u32 fd, u32 fs, bool q8, hipStream_t st) {
  const u32 nt = a.nk + (fs ? 1u : 0u);
  const size_t lds = dn_dec_lds(a.nk, a.ef, a.sf, a.rbd, a.rbs, a.dm, fs != 0, q8, &a.stage_bytes, &a.xw_bytes);
  if (!lds) return -1;
#define DN_FS(FD, FS) \
  if (fd == FD && fs == FS) return q8 ? dn_dec_one<FD, FS, true>(a, nt, lds, st) : dn_dec_one<FD, FS, false>(a, nt, lds, st);
#define DN_F(FD) DN_FS(FD, 0u) DN_FS(FD, FM_Q4_K) DN_FS(FD, FM_Q5_K) DN_FS(FD, FM_Q6_K)
  DN_F(FM_Q8_0) DN_F(FM_Q4_K) DN_F(FM_Q5_K) DN_F(FM_Q6_K)
#undef DN_F
#undef DN_FS
  return -1;
}
