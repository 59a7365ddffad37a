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
// final subtract (Q4_K / Q5_K) rounds once, at the same place, and with the same sign of zero.
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
#define MDEV __device__ __forceinline__  // member functions

DEV float bits_f(u32 u) { return __uint_as_float(u); }

// llb_f16 (tools/quant-fix.patch:11-21): (m [+ 1024]) * 2^(e' - 25), exact; exponent 31 keeps
// the mantissa as an f32 inf / NaN payload
// the value of every finite / infinite half is what v_cvt_f32_f16 gives; a NaN keeps its payload
// unquieted as llb_f16 does (a select, no branch)
DEV float f16v(u32 h) {
  const float hw = (float)__builtin_bit_cast(_Float16, (unsigned short)h);
  const u32 nan = ((h >> 15) << 31) | 0x7f800000u | (h & 1023u) << 13;
  return bits_f(((h & 0x7c00u) == 0x7c00u && (h & 1023u)) ? nan : __float_as_uint(hw));
}

// a word the compiler may not look through: keeps "mask 4 bytes, then v_cvt_f32_ubyte{0..3}" from
// being rewritten into one bit-field extract per byte
DEV u32 opq(u32 v) {
  __asm__("" : "+v"(v));
  return v;
}
// byte k of v as an exact float (v_cvt_f32_ubyte{0..3})
DEV float ubyte(u32 v, u32 k) { return (float)((v >> (8 * k)) & 255u); }

DEV u32 ld_u16(const u8* p) { return (u32)*(const unsigned short*)p; }

// p rounded down to 4 bytes by pointer arithmetic (a cast through an integer would hide the global
// address space and turn every load through it into a flat load, which also holds up LDS waits)
DEV const u32* al4(const u8* p) { return (const u32*)(p - ((u32)(uintptr_t)p & 3u)); }

// 32 bytes from a 2-aligned address: nine aligned dwords, funnel-shifted by 16 when p % 4 == 2.
// Reads at most 4 bytes past p + 32 (every caller's span has them inside its own block).
DEV void ld32_a2(const u8* p, u32 o[8]) {
  const u32* a = al4(p);
  const u32 sh = ((u32)(uintptr_t)p & 2u) * 8u;
  u32 w[9];
#pragma unroll
  for (int k = 0; k < 9; k++) w[k] = a[k];
#pragma unroll
  for (int k = 0; k < 8; k++) o[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
}

// ggml get_scale_min_k4 (tools/q4k.py:20-23) from the 12 scale bytes held in h.y (bytes 0..3),
// h.z (4..7), h.w (8..11): shifts and masks, no indexed array (a runtime index into a register array
// becomes a compare / select chain)
DEV void k4_scmin(uint4 h, u32 j, u32& sc, u32& mn) {
  const u32 k = 8u * (j & 3u);
  const u32 A = (h.y >> k) & 255u, B = (h.z >> k) & 255u, Cc = (h.w >> k) & 255u;
  if (j < 4) {
    sc = A & 63u; mn = B & 63u;
  } else {
    sc = (Cc & 15u) | ((A >> 6) << 4);
    mn = (Cc >> 4) | ((B >> 6) << 4);
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

// Q8_0 GGUF block c0 / 32: [f16 d][32 x i8]; w = q * d (exact: 11-bit d times a 7-bit q), q as
// (the unsigned byte of q ^ 0x80) - 128, exact. (An FMA with a -128 d addend would give +0 where
// q * d is -0.)
template <> struct Span<FM_Q8_0> {
  DEV void w(const u8* row, u32 c0, float* w) {
    const u8* B = row + (u64)(c0 >> 5) * 34u;
    const u32* a = al4(B);
    const bool odd = ((uintptr_t)B & 2u) != 0;
    u32 v[9];
#pragma unroll
    for (int k = 0; k < 9; k++) v[k] = a[k];
    const float d = f16v(odd ? v[0] >> 16 : v[0] & 0xffffu);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u32 q = (odd ? v[k + 1] : __builtin_amdgcn_alignbit(v[k + 1], v[k], 16)) ^ 0x80808080u;
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = (ubyte(q, t) - 128.0f) * d;
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
// w = (d sc) (q - 32): d sc, q - 32 and their product are exact
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
    const u32 nsh = quad >= 2u ? 4u : 0u, hsh = 2u * quad;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u32 v = ((ql[k] >> nsh) & 0x0F0F0F0Fu) | (((qh[k] >> hsh) & 0x03030303u) << 4);
#pragma unroll
      for (int t = 0; t < 4; t++)
        w[4 * k + t] = (k < 4 ? ds0 : ds1) * (ubyte(v, t) - 32.0f);
    }
  }
};

// ---- half spans: columns c0 + 16 jh .. c0 + 16 jh + 15 of the span at c0, in two steps -- ld
// issues the raw loads (so a caller can put a row's loads in flight before it waits on anything
// else), dec turns them into the same 16 weights span_w gives for those columns.

template <u32 F> struct Half;

template <> struct Half<FM_F32> {
  float4 v[4];
  MDEV void ld(const u8* row, u32 c0, u32 jh) {
    const float4* p = (const float4*)(row + 4 * (u64)(c0 + 16 * jh));
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = p[k];
  }
  MDEV void dec(u32, u32, float* w) const {
#pragma unroll
    for (int k = 0; k < 4; k++) { w[4 * k] = v[k].x; w[4 * k + 1] = v[k].y; w[4 * k + 2] = v[k].z; w[4 * k + 3] = v[k].w; }
  }
};

// 16 bytes from any address in one load (global loads need no alignment on this target: the
// compiler itself turns an unaligned 16-byte copy into one global_load_dwordx4)
DEV uint4 ldu16(const u8* p) {
  uint4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}

template <> struct Half<FM_Q8_0> {
  uint4 q;
  u32 d;
  MDEV void ld(const u8* row, u32 c0, u32 jh) {
    const u8* B = row + (u64)(c0 >> 5) * 34u;
    d = ld_u16(B);
    q = ldu16(B + 2 + 16 * jh);
  }
  MDEV void dec(u32, u32, float* w) const {
    const float dv = f16v(d);
    const u32 o[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32 v = opq(o[k] ^ 0x80808080u);
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = (ubyte(v, t) - 128.0f) * dv;
    }
  }
};

template <> struct Half<FM_Q4_K> {
  uint4 h, q;
  MDEV void ld(const u8* row, u32 c0, u32 jh) {
    const u8* B = row + (u64)(c0 >> 8) * 144u;
    const u32 j = (c0 & 255u) >> 5;
    h = *(const uint4*)B;
    q = *(const uint4*)(B + 16 + 32 * (j >> 1) + 16 * jh);
  }
  // an odd sub-block's codes are the high nibbles: masked in place they read 16 q, and d sc / 16
  // (exact: a power-of-two scale of a normal float) times 16 q is the same exact product
  MDEV void dec(u32 c0, u32, float* w) const {
    const u32 j = (c0 & 255u) >> 5;
    u32 sc, mn;
    k4_scmin(h, j, sc, mn);
    const float d1 = f16v(h.x & 0xffffu) * (float)sc * ((j & 1u) ? 0.0625f : 1.0f), m1 = f16v(h.x >> 16) * (float)mn;
    const u32 mask = (j & 1u) ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    const u32 qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32 v = opq(qq[k] & mask);
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = __builtin_fmaf(d1, ubyte(v, t), -m1);
    }
  }
};

template <> struct Half<FM_Q5_K> {
  uint4 h, qh, q;
  MDEV void ld(const u8* row, u32 c0, u32 jh) {
    const u8* B = row + (u64)(c0 >> 8) * 176u;
    const u32 j = (c0 & 255u) >> 5;
    h = *(const uint4*)B;
    qh = *(const uint4*)(B + 16 + 16 * jh);
    q = *(const uint4*)(B + 48 + 32 * (j >> 1) + 16 * jh);
  }
  MDEV void dec(u32 c0, u32, float* w) const {
    const u32 j = (c0 & 255u) >> 5;
    u32 sc, mn;
    k4_scmin(h, j, sc, mn);
    const float d1 = f16v(h.x & 0xffffu) * (float)sc, m1 = f16v(h.x >> 16) * (float)mn;
    const u32 sh = 4u * (j & 1u);
    const u32 qq[4] = {q.x, q.y, q.z, q.w}, hh[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32 v = opq(((qq[k] >> sh) & 0x0F0F0F0Fu) | (((hh[k] >> j) & 0x01010101u) << 4));
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = __builtin_fmaf(d1, ubyte(v, t), -m1);
    }
  }
};

template <> struct Half<FM_Q6_K> {
  uint4 ql, qh;
  u32 sc, d;
  MDEV void ld(const u8* row, u32 c0, u32 jh) {
    const u8* B = row + (u64)(c0 >> 8) * 210u;
    const u32 r = c0 & 255u, n = r >> 7, quad = (r & 127u) >> 5;
    ql = ldu16(B + 64 * n + 32 * (quad & 1u) + 16 * jh);
    qh = ldu16(B + 128 + 32 * n + 16 * jh);
    sc = (u32)B[192 + (r >> 4) + jh];
    d = ld_u16(B + 208);
  }
  // each byte built as (q ^ 0x20) << 2, which read as a signed byte is 4 (q - 32); (d sc / 4)
  // (exact: d sc is a normal float or 0) times it is d sc (q - 32), the same exact product, with
  // the same sign of zero (+0 times d sc)
  MDEV void dec(u32 c0, u32, float* w) const {
    const u32 r = c0 & 255u, quad = (r & 127u) >> 5;
    const float ds = f16v(d) * (float)(int)(signed char)sc * 0.25f;
    const u32 l4[4] = {ql.x, ql.y, ql.z, ql.w}, h4[4] = {qh.x, qh.y, qh.z, qh.w};
    // the nibble into bits 2..5 of its byte: a rotate by 2 either way (bits that wrap are masked)
    const u32 rot = quad >= 2u ? 2u : 30u, hs = 6u - 2u * quad;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32 lo = __builtin_amdgcn_alignbit(l4[k], l4[k], rot);
      const u32 hi = h4[k] << hs;  // bits 2 quad, 2 quad + 1 into 6, 7
      const u32 v = opq(((lo & 0x3C3C3C3Cu) | (hi & 0xC0C0C0C0u)) ^ 0x80808080u);
#pragma unroll
      for (int t = 0; t < 4; t++) w[4 * k + t] = ds * (float)(int)(signed char)((v >> (8 * t)) & 255u);
    }
  }
};

// ---- half spans straight to f16 (the grouped-GEMM tier): packed 16-bit arithmetic, two weights an
// op. A code byte u becomes the half 1024 + u by v_perm with 0x64 as its high byte; subtracting the
// bias leaves the code exactly. Q8_0: q d rounded once to f16, as rounding the exact f32 product.
// K-quants: the f32 scale and min products are rounded to f16 first, then one packed FMA a pair
// (tolerance class, like the f16 activations).
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
DEV h2v as_h2(u32 v) { return __builtin_bit_cast(h2v, v); }
DEV u32 as_u(h2v v) { return __builtin_bit_cast(u32, v); }
// bytes 0, 1 (lo) and 2, 3 (hi) of v as 1024 + byte halves
DEV h2v mag_lo(u32 v) { return as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)); }
DEV h2v mag_hi(u32 v) { return as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)); }
DEV h2v h2s(float f) { const _Float16 h = (_Float16)f; return h2v{h, h}; }

template <u32 F> DEV void half_f16(const Half<F>& h, u32 c0, u32 jh, u32* o);
template <> DEV void half_f16<FM_Q8_0>(const Half<FM_Q8_0>& h, u32, u32, u32* o) {
  const h2v d = as_h2((h.d & 0xffffu) * 0x10001u), bias = h2s(1152.0f);
  const u32 q[4] = {h.q.x, h.q.y, h.q.z, h.q.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const u32 u = q[k] ^ 0x80808080u;  // q + 128
    o[2 * k] = as_u((mag_lo(u) - bias) * d);
    o[2 * k + 1] = as_u((mag_hi(u) - bias) * d);
  }
}
template <> DEV void half_f16<FM_Q4_K>(const Half<FM_Q4_K>& h, u32 c0, u32, u32* o) {
  const u32 j = (c0 & 255u) >> 5;
  u32 sc, mn;
  k4_scmin(h.h, j, sc, mn);
  const h2v d1 = h2s(f16v(h.h.x & 0xffffu) * (float)sc), m1 = h2s(-(f16v(h.h.x >> 16) * (float)mn)), bias = h2s(1024.0f);
  const u32 sh = 4u * (j & 1u);
  const u32 q[4] = {h.q.x, h.q.y, h.q.z, h.q.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const u32 v = (q[k] >> sh) & 0x0F0F0F0Fu;
    o[2 * k] = as_u(__builtin_elementwise_fma(mag_lo(v) - bias, d1, m1));
    o[2 * k + 1] = as_u(__builtin_elementwise_fma(mag_hi(v) - bias, d1, m1));
  }
}
template <> DEV void half_f16<FM_Q5_K>(const Half<FM_Q5_K>& h, u32 c0, u32, u32* o) {
  const u32 j = (c0 & 255u) >> 5;
  u32 sc, mn;
  k4_scmin(h.h, j, sc, mn);
  const h2v d1 = h2s(f16v(h.h.x & 0xffffu) * (float)sc), m1 = h2s(-(f16v(h.h.x >> 16) * (float)mn)), bias = h2s(1024.0f);
  const u32 sh = 4u * (j & 1u);
  const u32 q[4] = {h.q.x, h.q.y, h.q.z, h.q.w}, hh[4] = {h.qh.x, h.qh.y, h.qh.z, h.qh.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const u32 v = ((q[k] >> sh) & 0x0F0F0F0Fu) | (((hh[k] >> j) & 0x01010101u) << 4);
    o[2 * k] = as_u(__builtin_elementwise_fma(mag_lo(v) - bias, d1, m1));
    o[2 * k + 1] = as_u(__builtin_elementwise_fma(mag_hi(v) - bias, d1, m1));
  }
}
template <> DEV void half_f16<FM_Q6_K>(const Half<FM_Q6_K>& h, u32 c0, u32, u32* o) {
  const u32 r = c0 & 255u, quad = (r & 127u) >> 5;
  const h2v ds = h2s(f16v(h.d) * (float)(int)(signed char)h.sc), bias = h2s(1056.0f);  // 1024 + 32
  const u32 nsh = quad >= 2u ? 4u : 0u, hsh = 2u * quad;
  const u32 l4[4] = {h.ql.x, h.ql.y, h.ql.z, h.ql.w}, h4[4] = {h.qh.x, h.qh.y, h.qh.z, h.qh.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const u32 v = ((l4[k] >> nsh) & 0x0F0F0F0Fu) | (((h4[k] >> hsh) & 0x03030303u) << 4);
    o[2 * k] = as_u((mag_lo(v) - bias) * ds);
    o[2 * k + 1] = as_u((mag_hi(v) - bias) * ds);
  }
}

// ---- cross-lane pair sums at ALU latency (DPP and the gfx950 permlane swaps; ds_bpermute, which
// __shfl_xor uses, costs about 60 ns a step). xaddM(v) = v + v[lane ^ M]; IEEE addition commutes, so
// the value is the exact pair sum. Lanes where it holds: M = 1, 2, 8, 16, 32 every lane; M = 4 the
// lanes whose index mod 16 is < 4 or is 8..11 (row_ror:12 reads lane + 4 of the row).
template <int CTRL> DEV float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL> DEV u32 dppu(u32 v) { return (u32)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false); }
#define DPP_XOR1 0xB1   // quad_perm [1, 0, 3, 2]
#define DPP_XOR2 0x4E   // quad_perm [2, 3, 0, 1]
#define DPP_UP4 0x12C   // row_ror:12: lane l reads lane (l + 4) mod 16 of its row
#define DPP_XOR8 0x128  // row_ror:8
DEV float xadd1(float v) { return v + dppf<DPP_XOR1>(v); }
DEV float xadd2(float v) { return v + dppf<DPP_XOR2>(v); }
DEV float xadd4(float v) { return v + dppf<DPP_UP4>(v); }
DEV float xadd8(float v) { return v + dppf<DPP_XOR8>(v); }
DEV float xadd16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
DEV float xadd32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// lane ^ 32's value
DEV float xpeer32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}
// moe_dot's tree over the 32 lanes of each half-wave, levels 16, 8, 4, 2, 1: exact at lanes 0, 32
DEV float tree32_desc(float v) { return xadd1(xadd2(xadd4(xadd8(xadd16(v))))); }
// the engine tree across a wave, levels 1, 2, 4, 8, 16, 32 (lower lane bits first): exact at lane 0
DEV float tree64_asc(float v) { return xadd32(xadd16(xadd8(xadd4(xadd2(xadd1(v)))))); }

// the leaf of every exact GEMV: (w0 x0 + w1 x1) + (w2 x2 + w3 x3)
DEV float leaf4(const float* w, float4 x) {
  return ((w[0] * x.x) + (w[1] * x.y)) + ((w[2] * x.z) + (w[3] * x.w));
}

// llb_moe_gu's epilogue (tools/payload-moeany.patch:495): (g / (1 + exp(-g))) * u, the exp
// through double as attn_exp (tools/payload-attn.patch:57-59)
DEV float exp_f(float x) { return (float)exp((double)x); }
DEV float silu_mul(float g, float u) { return (g / (1.0f + exp_f(-g))) * u; }
