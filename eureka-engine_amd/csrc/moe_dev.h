// moe_dev.h -- device building blocks of the MoE FFN path for gfx950 (wave64).
//
// Weight rows keep the GGUF bytes verbatim (expert stacks [ne][rows][row bytes], cols fastest):
//   Q8_0 34 B / 32 cols (2-aligned), Q4_K 144 B / 256, Q5_K 176 B / 256 (16-aligned),
//   Q6_K 210 B / 256 (2-aligned). Format codes follow host/llb_formats.h:4-14.
//
// The unit of decode is a 32-column span: span_w<F>(row, c0, w) writes the 32 f32 weights of
// columns c0 .. c0 + 31 (c0 % 32 == 0) with exactly the values of the reference's dequant
// (q8g_w / q4k_w / q6k_w / q5k_w, tools/payload-moeany.patch:85-91, tools/quant-doors.patch:34-80,
// tools/payload-anyshape.patch:54-81): every product there is exact, so an FMA that folds the
// final subtract (Q4_K / Q5_K) or a rebias (Q6_K, Q8_0) rounds once, at the same place.
//
// Everything here is compiled with -ffp-contract=off: a float op written is a float op executed.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32;
typedef uint64_t u64;
typedef uint8_t u8;

#define FM_F32 0u
#define FM_Q8_0 1u
#define FM_Q4_K 3u
#define FM_Q6_K 4u
#define FM_Q5_K 9u

#define DEV static __device__ __forceinline__

DEV float bits_f(u32 u) { return __uint_as_float(u); }

// llb_f16 (tools/quant-fix.patch:11-21): (m [+ 1024]) * 2^(e' - 25), exact; exponent 31 keeps
// the mantissa as an f32 inf / NaN payload
DEV float f16v(u32 h) {
  const u32 e = (h >> 10) & 31u, m = h & 1023u, s = (h >> 15) << 31;
  const float mag = (float)(e ? m + 1024u : m) * bits_f(((e ? e : 1u) + 102u) << 23);
  return bits_f(e == 31u ? (s | 0x7f800000u | m << 13) : (__float_as_uint(mag) | s));
}

// byte k of v as an exact float (v_cvt_f32_ubyte{0..3})
DEV float ubyte(u32 v, u32 k) { return (float)((v >> (8 * k)) & 255u); }

DEV u32 ld_u16(const u8* p) { return (u32)*(const unsigned short*)p; }

// 32 bytes from a 2-aligned address: nine aligned dwords, funnel-shifted by 16 when p % 4 == 2.
// Reads at most 4 bytes past p + 32 (every caller's span has them inside its own block).
DEV void ld32_a2(const u8* p, u32 o[8]) {
  const u32* a = (const u32*)((uintptr_t)p & ~(uintptr_t)3);
  const u32 sh = ((u32)(uintptr_t)p & 2u) * 8u;
  u32 w[9];
#pragma unroll
  for (int k = 0; k < 9; k++) w[k] = a[k];
#pragma unroll
  for (int k = 0; k < 8; k++) o[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
}

// ggml get_scale_min_k4 (tools/q4k.py:20-23) from the 12 scale bytes held in h.y, h.z, h.w
DEV void k4_scmin(uint4 h, u32 j, u32& sc, u32& mn) {
  const u32 b[12] = {h.y & 255u, (h.y >> 8) & 255u, (h.y >> 16) & 255u, h.y >> 24,
                     h.z & 255u, (h.z >> 8) & 255u, (h.z >> 16) & 255u, h.z >> 24,
                     h.w & 255u, (h.w >> 8) & 255u, (h.w >> 16) & 255u, h.w >> 24};
  if (j < 4) {
    sc = b[j] & 63u; mn = b[j + 4] & 63u;
  } else {
    sc = (b[j + 4] & 15u) | ((b[j - 4] >> 6) << 4);
    mn = (b[j + 4] >> 4) | ((b[j] >> 6) << 4);
  }
}

template <u32 F> struct Span;

// F32 rows (router, shared gate): 32 floats as eight 16-byte loads
template <> struct Span<FM_F32> {
  DEV void w(const u8* row, u32 c0, float* w) {
    const float4* p = (const float4*)(row + 4 * (u64)c0);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float4 v = p[k];
      w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
    }
  }
};

// Q8_0 GGUF block c0 / 32: [f16 d][32 x i8]; w = q * d (exact: 11-bit d times a 7-bit q)
// as fma(d, q + 128, -128 d), q + 128 the unsigned byte of q ^ 0x80
template <> struct Span<FM_Q8_0> {
  DEV void w(const u8* row, u32 c0, float* w) {
    const u8* B = row + (u64)(c0 >> 5) * 34u;
    const u32* a = (const u32*)((uintptr_t)B & ~(uintptr_t)3);
    const bool odd = ((uintptr_t)B & 2u) != 0;
    u32 v[9];
#pragma unroll
    for (int k = 0; k < 9; k++) v[k] = a[k];
    const float d = f16v(odd ? v[0] >> 16 : v[0] & 0xffffu);
    const float nd = d * -128.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u32 q = (odd ? v[k + 1] : __builtin_amdgcn_alignbit(v[k + 1], v[k], 16)) ^ 0x80808080u;
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = __builtin_fmaf(d, ubyte(q, t), nd);
    }
  }
};

// Q4_K super-block c0 / 256, sub-block j = (c0 % 256) / 32: w = (d sc) q - (dmin m); d sc and
// (d sc) q are exact, so fma(d sc, q, -(dmin m)) is the reference's one rounding
template <> struct Span<FM_Q4_K> {
  DEV void w(const u8* row, u32 c0, float* w) {
    const u8* B = row + (u64)(c0 >> 8) * 144u;
    const u32 j = (c0 & 255u) >> 5;
    const uint4 h = *(const uint4*)B;
    const uint4* qp = (const uint4*)(B + 16 + 32 * (j >> 1));
    const uint4 q0 = qp[0], q1 = qp[1];
    u32 sc, mn;
    k4_scmin(h, j, sc, mn);
    const float d1 = f16v(h.x & 0xffffu) * (float)sc, m1 = f16v(h.x >> 16) * (float)mn;
    const u32 sh = 4u * (j & 1u);
    const u32 q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u32 v = (q[k] >> sh) & 0x0F0F0F0Fu;
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = __builtin_fmaf(d1, ubyte(v, t), -m1);
    }
  }
};

// Q5_K (176 B: d, dmin, scales[12], qh[32] @16, qs[128] @48): Q4_K's scales, the fifth bit of
// column 64 g + 32 hi + l is bit 2 g + hi (= j) of qh[l]
template <> struct Span<FM_Q5_K> {
  DEV void w(const u8* row, u32 c0, float* w) {
    const u8* B = row + (u64)(c0 >> 8) * 176u;
    const u32 j = (c0 & 255u) >> 5;
    const uint4 h = *(const uint4*)B;
    const uint4 h0 = *(const uint4*)(B + 16), h1 = *(const uint4*)(B + 32);
    const uint4* qp = (const uint4*)(B + 48 + 32 * (j >> 1));
    const uint4 q0 = qp[0], q1 = qp[1];
    u32 sc, mn;
    k4_scmin(h, j, sc, mn);
    const float d1 = f16v(h.x & 0xffffu) * (float)sc, m1 = f16v(h.x >> 16) * (float)mn;
    const u32 sh = 4u * (j & 1u);
    const u32 q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const u32 qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u32 v = ((q[k] >> sh) & 0x0F0F0F0Fu) | (((qh[k] >> j) & 0x01010101u) << 4);
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = __builtin_fmaf(d1, ubyte(v, t), -m1);
    }
  }
};

// Q6_K (210 B: ql[128], qh[64] @128, int8 scales[16] @192, f16 d @208; 2-aligned). Column c:
// n = c / 128, quad = (c % 128) / 32, l = c % 32: low nibble bits from ql[64 n + 32 (quad & 1) + l]
// (upper nibble when quad >= 2), two high bits from qh[32 n + l] >> 2 quad, scale sc[c / 16].
// w = (d sc) (q - 32): d sc and the product are exact, so fma(d sc, q, -32 d sc) is that value
template <> struct Span<FM_Q6_K> {
  DEV void w(const u8* row, u32 c0, float* w) {
    const u8* B = row + (u64)(c0 >> 8) * 210u;
    const u32 r = c0 & 255u, n = r >> 7, quad = (r & 127u) >> 5;
    u32 ql[8], qh[8];
    ld32_a2(B + 64 * n + 32 * (quad & 1u), ql);
    ld32_a2(B + 128 + 32 * n, qh);
    const u32 scw = ld_u16(B + 192 + 8 * n + 2 * quad);
    const float d = f16v(ld_u16(B + 208));
    const float ds0 = d * (float)(int)(signed char)(scw & 255u), ds1 = d * (float)(int)(signed char)(scw >> 8);
    const float n0 = ds0 * -32.0f, n1 = ds1 * -32.0f;
    const u32 nsh = quad >= 2u ? 4u : 0u, hsh = 2u * quad;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u32 v = ((ql[k] >> nsh) & 0x0F0F0F0Fu) | (((qh[k] >> hsh) & 0x03030303u) << 4);
#pragma unroll
      for (int t = 0; t < 4; t++)
        w[4 * k + t] = k < 4 ? __builtin_fmaf(ds0, ubyte(v, t), n0) : __builtin_fmaf(ds1, ubyte(v, t), n1);
    }
  }
};

// the leaf of every exact GEMV: (w0 x0 + w1 x1) + (w2 x2 + w3 x3)
DEV float leaf4(const float* w, float4 x) {
  return ((w[0] * x.x) + (w[1] * x.y)) + ((w[2] * x.z) + (w[3] * x.w));
}

// llb_moe_gu's epilogue (tools/payload-moeany.patch:495): (g / (1 + exp(-g))) * u, the exp
// through double as attn_exp (tools/payload-attn.patch:57-59)
DEV float exp_f(float x) { return (float)exp((double)x); }
DEV float silu_mul(float g, float u) { return (g / (1.0f + exp_f(-g))) * u; }
