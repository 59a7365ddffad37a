// moe_q8dot.h -- the q8 tier's device arithmetic, shared by its kernels (moe_q8.hip) and the fused
// top-k + gate / up launch (moe_exact.hip): the q8_1 quantizer step (pf_q8x, tools/pf27/pfmm.cuh:39-54)
// and the int8 block dots (mx_blk / mx_dot, host/llb_pf.cuh:468-530).
#pragma once
#include "moe_dev.h"

// q8_1 of a 32-element block, one element a lane (lanes 32 h .. 32 h + 31 of a wave hold one block;
// every lane of the wave takes part): d = amax / 127, q = round(v / d) (0 when amax = 0), sum = the
// block's sum by the xor butterfly 16, 8, 4, 2, 1. Returns q; d and sum on every lane of the block.
DEV signed char q8_1_lane(float v, float& d, float& sum) {
  float a = fabsf(v), s = v;
#pragma unroll
  for (u32 m = 16; m > 0; m >>= 1) {
    a = fmaxf(a, __shfl_xor(a, m, 64));
    s = s + __shfl_xor(s, m, 64);
  }
  d = a / 127.0f;
  sum = s;
  return a == 0.0f ? (signed char)0 : (signed char)max(-127, min(127, (int)roundf(v / d)));
}
// n values (n % 32 == 0, n <= 256 MAXR) from x to q8_1 in q / ds, by the whole block of 256 threads:
// rounds of 256 consecutive values, every thread in every round (the butterfly needs all lanes); all
// rounds' loads are issued before the first is reduced
template <u32 MAXR>
DEV void q8_1_block256(const float* __restrict__ x, u32 n, signed char* q, float2* ds) {
  float v[MAXR];
#pragma unroll
  for (u32 r = 0; r < MAXR; r++) {
    const u32 i = 256 * r + threadIdx.x;
    v[r] = i < n ? x[i] : 0.0f;
  }
#pragma unroll
  for (u32 r = 0; r < MAXR; r++) {
    if (256 * r >= n) break;  // block-uniform
    const u32 i = 256 * r + threadIdx.x;
    float d, sum;
    const signed char c = q8_1_lane(v[r], d, sum);
    if (i < n) q[i] = c;
    if (i < n && (threadIdx.x & 31) == 0) ds[i >> 5] = make_float2(d, sum);
  }
}

// ---------------------------------------------------------------- block dots

DEV int dot4(u32 a, u32 b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// 32-column block b of a row against 32 int8 x (8 dwords) with {d, s}
template <u32 F> DEV float blk_q8(const u8* row, u32 b, const u32* xq, float2 e);

template <> __device__ __forceinline__ float blk_q8<FM_Q4_K>(const u8* row, u32 b, const u32* xq, float2 e) {
  const u8* B = row + (u64)(b >> 3) * 144u;
  const u32 j = b & 7u;
  const uint4 h = *(const uint4*)B;
  const uint4* qp = (const uint4*)(B + 16 + 32 * (j >> 1));
  const uint4 q0 = qp[0], q1 = qp[1];
  const u32 q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const u32 sh = 4u * (j & 1u);
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) acc = dot4((q[k] >> sh) & 0x0F0F0F0Fu, xq[k], acc);
  u32 sc, mn;
  k4_scmin(h, j, sc, mn);
  return f16v(h.x & 0xffffu) * (float)sc * e.x * (float)acc - f16v(h.x >> 16) * (float)mn * e.y;
}
template <> __device__ __forceinline__ float blk_q8<FM_Q5_K>(const u8* row, u32 b, const u32* xq, float2 e) {
  const u8* B = row + (u64)(b >> 3) * 176u;
  const u32 j = b & 7u;
  const uint4 h = *(const uint4*)B;
  const uint4 h0 = *(const uint4*)(B + 16), h1 = *(const uint4*)(B + 32);
  const uint4* qp = (const uint4*)(B + 48 + 32 * (j >> 1));
  const uint4 q0 = qp[0], q1 = qp[1];
  const u32 q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const u32 qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
  const u32 sh = 4u * (j & 1u);
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) acc = dot4(((q[k] >> sh) & 0x0F0F0F0Fu) | (((qh[k] >> j) & 0x01010101u) << 4), xq[k], acc);
  u32 sc, mn;
  k4_scmin(h, j, sc, mn);
  return f16v(h.x & 0xffffu) * (float)sc * e.x * (float)acc - f16v(h.x >> 16) * (float)mn * e.y;
}
template <> __device__ __forceinline__ float blk_q8<FM_Q6_K>(const u8* row, u32 b, const u32* xq, float2 e) {
  const u8* B = row + (u64)(b >> 3) * 210u;
  const u32 bb = b & 7u, n = bb >> 2, quad = bb & 3u;
  u32 ql[8], qh[8];
  ld32_a2(B + 64 * n + 32 * (quad & 1u), ql);
  ld32_a2(B + 128 + 32 * n, qh);
  const u32 nsh = quad >= 2u ? 4u : 0u, hsh = 2u * quad;
  int a0 = 0, a1 = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const u32 v = ((ql[k] >> nsh) & 0x0F0F0F0Fu) | (((qh[k] >> hsh) & 0x03030303u) << 4);
    const u32 c = ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;  // per byte q - 32, signed
    if (k < 4) a0 = dot4(c, xq[k], a0);
    else a1 = dot4(c, xq[k], a1);
  }
  const u32 scw = ld_u16(B + 192 + 8 * n + 2 * quad);
  const float d = f16v(ld_u16(B + 208));
  return d * e.x * ((float)(int)(signed char)(scw & 255u) * (float)a0 + (float)(int)(signed char)(scw >> 8) * (float)a1);
}
template <> __device__ __forceinline__ float blk_q8<FM_Q8_0>(const u8* row, u32 b, const u32* xq, float2 e) {
  const u8* B = row + (u64)b * 34u;
  const u32* a = al4(B);
  const bool odd = ((uintptr_t)B & 2u) != 0;
  u32 v[9];
#pragma unroll
  for (int k = 0; k < 9; k++) v[k] = a[k];
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) acc = dot4(odd ? v[k + 1] : __builtin_amdgcn_alignbit(v[k + 1], v[k], 16), xq[k], acc);
  return f16v(odd ? v[0] >> 16 : v[0] & 0xffffu) * e.x * (float)acc;
}

// a row's q8 dot on the 4 lanes of a lane group: lane p takes blocks p, p + 4, ...; U: the loop's
// unroll (long rows: the loads of U blocks go out together)
template <u32 F, u32 U>
DEV float row_q8(const u8* row, u32 cols, const signed char* xq, const float2* xd, u32 p) {
  float acc = 0.0f;
#pragma unroll U
  for (u32 b = p; b < cols / 32; b += 4) {
    const uint4 a0 = *(const uint4*)(xq + 32 * b), a1 = *(const uint4*)(xq + 32 * b + 16);
    const u32 x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    acc += blk_q8<F>(row, b, x, xd[b]);
  }
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 1, 64);
  return acc;
}
template <u32 U = 1>
DEV float row_q8_fm(u32 f, const u8* row, u32 cols, const signed char* xq, const float2* xd, u32 p) {
  switch (f) {
    case FM_Q8_0: return row_q8<FM_Q8_0, U>(row, cols, xq, xd, p);
    case FM_Q4_K: return row_q8<FM_Q4_K, U>(row, cols, xq, xd, p);
    case FM_Q6_K: return row_q8<FM_Q6_K, U>(row, cols, xq, xd, p);
    default: return row_q8<FM_Q5_K, U>(row, cols, xq, xd, p);
  }
}

