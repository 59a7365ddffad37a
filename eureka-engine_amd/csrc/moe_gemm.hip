// moe_gemm.hip -- the grouped-GEMM tier for many tokens (prefill, large batches): the expert products
// on CDNA4 MFMA (v_mfma_f32_32x32x16_f16, f32 accumulate). The reference's fast prefill
// (host/llb_pf.h:286-389, pfx_* on int8 mma.sync) groups slots by expert and runs one GEMM per
// expert over its slots; so does this. Weights are dequantized with the exact tier's decoders (a
// 32-column span at a time) and rounded to f16 in registers; activations are f16. Tolerance class.
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

#define G3_MF 2                // 32-row fragments a tile
#define GM_BM (32 * G3_MF)     // slots a tile (an expert's slots split into tiles of this many)
#define G3_BM GM_BM


// ---- packed weights: a matrix of R rows x K columns re-laid in tiles of 32 rows x 64 columns, tile
// (g, t) = rows 32 g .. 32 g + 31, columns 64 t .. 64 t + 63 at byte (g K / 64 + t) PK_TB<F>. In a
// tile, lane l = 32 h + r owns row r, columns 32 h .. 32 h + 31: exactly the GEMM's B operand for a
// k-tile, so a wave reads a tile with a few fully coalesced loads (planes of 64 lanes x 16 bytes)
// instead of 64 scattered rows. The contents are the codes and f16 scales half_f16 derives from the
// GGUF blocks (bit for bit the same weights):
//   Q8_0  planes 0, 1: the codes of columns 0..15, 16..31 (q bytes); then 64 x u16 d
//   Q4_K  plane 0: byte b = code b | code b + 16 << 4; then 64 x u32 {f16 d sc, f16 -dmin m}
//   Q5_K  planes 0, 1: code bytes; then 64 x u32 {f16 d sc, f16 -dmin m}
//   Q6_K  plane 0: low nibbles as Q4_K; then 64 x u64 {H0, H1}: bits 2 k, 2 k + 1 of byte i of Hj
//         are the high two bits of code 16 j + 4 k + i; then 64 x u32 {f16 d sc0, f16 d sc1}
template <u32 F> struct PK;
template <> struct PK<FM_Q8_0> { static constexpr u32 TB = 2176; };
template <> struct PK<FM_Q4_K> { static constexpr u32 TB = 1280; };
template <> struct PK<FM_Q5_K> { static constexpr u32 TB = 2304; };
template <> struct PK<FM_Q6_K> { static constexpr u32 TB = 1792; };

// the codes half_f16 builds for half jh (byte 4 k + i of v[k] = code of column 16 jh + 4 k + i) and
// its f16 scale pair {scale, min} as u32 (min 0 where the format has none)
template <u32 F> DEV void half_codes(const Half<F>& h, u32 c0, u32 jh, u32* v, u32& s);
template <> DEV void half_codes<FM_Q8_0>(const Half<FM_Q8_0>& h, u32, u32, u32* v, u32& s) {
  v[0] = h.q.x; v[1] = h.q.y; v[2] = h.q.z; v[3] = h.q.w;
  s = h.d & 0xffffu;
}
template <> DEV void half_codes<FM_Q4_K>(const Half<FM_Q4_K>& h, u32 c0, u32, u32* v, u32& s) {
  const u32 j = (c0 & 255u) >> 5;
  u32 sc, mn;
  k4_scmin(h.h, j, sc, mn);
  const h2v d1 = h2s(f16v(h.h.x & 0xffffu) * (float)sc), m1 = h2s(-(f16v(h.h.x >> 16) * (float)mn));
  s = (as_u(d1) & 0xffffu) | (as_u(m1) << 16);
  const u32 sh = 4u * (j & 1u);
  const u32 q[4] = {h.q.x, h.q.y, h.q.z, h.q.w};
#pragma unroll
  for (int k = 0; k < 4; k++) v[k] = (q[k] >> sh) & 0x0F0F0F0Fu;
}
template <> DEV void half_codes<FM_Q5_K>(const Half<FM_Q5_K>& h, u32 c0, u32, u32* v, u32& s) {
  const u32 j = (c0 & 255u) >> 5;
  u32 sc, mn;
  k4_scmin(h.h, j, sc, mn);
  const h2v d1 = h2s(f16v(h.h.x & 0xffffu) * (float)sc), m1 = h2s(-(f16v(h.h.x >> 16) * (float)mn));
  s = (as_u(d1) & 0xffffu) | (as_u(m1) << 16);
  const u32 sh = 4u * (j & 1u);
  const u32 q[4] = {h.q.x, h.q.y, h.q.z, h.q.w}, hh[4] = {h.qh.x, h.qh.y, h.qh.z, h.qh.w};
#pragma unroll
  for (int k = 0; k < 4; k++) v[k] = ((q[k] >> sh) & 0x0F0F0F0Fu) | (((hh[k] >> j) & 0x01010101u) << 4);
}
template <> DEV void half_codes<FM_Q6_K>(const Half<FM_Q6_K>& h, u32 c0, u32, u32* v, u32& s) {
  const u32 r = c0 & 255u, quad = (r & 127u) >> 5;
  const h2v ds = h2s(f16v(h.d) * (float)(int)(signed char)h.sc);
  s = as_u(ds) & 0xffffu;
  const u32 nsh = quad >= 2u ? 4u : 0u, hsh = 2u * quad;
  const u32 l4[4] = {h.ql.x, h.ql.y, h.ql.z, h.ql.w}, h4[4] = {h.qh.x, h.qh.y, h.qh.z, h.qh.w};
#pragma unroll
  for (int k = 0; k < 4; k++) v[k] = ((l4[k] >> nsh) & 0x0F0F0F0Fu) | (((h4[k] >> hsh) & 0x03030303u) << 4);
}

// one wave a tile: grid (tiles of one matrix, ne), tiles = R / 32 * K / 64. W: GGUF rows (expert
// stride es), P: packed (expert stride R / 32 * K / 64 * TB)
template <u32 F>
__global__ void __launch_bounds__(64) k_pack(const u8* __restrict__ W, u64 es, u64 rb, u32 K, u8* __restrict__ P) {
  const u32 nkt = K / 64, tix = blockIdx.x, g = tix / nkt, t = tix % nkt, l = threadIdx.x, h = l >> 5, r = l & 31;
  const u8* row = W + (u64)blockIdx.y * es + (u64)(32 * g + r) * rb;
  u8* T = P + ((u64)blockIdx.y * gridDim.x + tix) * PK<F>::TB;
  const u32 c0 = 64 * t + 32 * h;
  Half<F> h0, h1;
  h0.ld(row, c0, 0);
  h1.ld(row, c0, 1);
  u32 v0[4], v1[4], s0, s1;
  half_codes<F>(h0, c0, 0, v0, s0);
  half_codes<F>(h1, c0, 1, v1, s1);
  if constexpr (F == FM_Q8_0 || F == FM_Q5_K) {
    *(uint4*)(T + 16 * l) = make_uint4(v0[0], v0[1], v0[2], v0[3]);
    *(uint4*)(T + 1024 + 16 * l) = make_uint4(v1[0], v1[1], v1[2], v1[3]);
    if constexpr (F == FM_Q8_0) *(unsigned short*)(T + 2048 + 2 * l) = (unsigned short)s0;
    else *(u32*)(T + 2048 + 4 * l) = s0;
  } else {
    u32 n[4];
#pragma unroll
    for (int k = 0; k < 4; k++) n[k] = (v0[k] & 0x0F0F0F0Fu) | ((v1[k] & 0x0F0F0F0Fu) << 4);
    *(uint4*)(T + 16 * l) = make_uint4(n[0], n[1], n[2], n[3]);
    if constexpr (F == FM_Q4_K) {
      *(u32*)(T + 1024 + 4 * l) = s0;
    } else {
      u32 H0 = 0, H1 = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        H0 |= ((v0[k] >> 4) & 0x03030303u) << (2 * k);
        H1 |= ((v1[k] >> 4) & 0x03030303u) << (2 * k);
      }
      *(uint2*)(T + 1024 + 8 * l) = make_uint2(H0, H1);
      *(u32*)(T + 1536 + 4 * l) = (s0 & 0xffffu) | (s1 << 16);
    }
  }
}

// a lane's share of one packed tile: ld issues the loads, f16(jh, o) gives the same eight u32 (16
// halves, columns 16 jh .. 16 jh + 15 of the lane's span) as half_f16 on the GGUF blocks
template <u32 F> struct PkB;
template <> struct PkB<FM_Q8_0> {
  uint4 q0, q1;
  u32 d;
  MDEV void ld(const u8* T, u32 l) {
    q0 = *(const uint4*)(T + 16 * l);
    q1 = *(const uint4*)(T + 1024 + 16 * l);
    d = *(const unsigned short*)(T + 2048 + 2 * l);
  }
  MDEV void f16(u32 jh, u32* o) const {
    const h2v dd = as_h2(d * 0x10001u), bias = h2s(1152.0f);
    const uint4 q = jh ? q1 : q0;
    const u32 qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32 u = qq[k] ^ 0x80808080u;
      o[2 * k] = as_u((mag_lo(u) - bias) * dd);
      o[2 * k + 1] = as_u((mag_hi(u) - bias) * dd);
    }
  }
};
template <> struct PkB<FM_Q4_K> {
  uint4 n;
  u32 s;
  MDEV void ld(const u8* T, u32 l) {
    n = *(const uint4*)(T + 16 * l);
    s = *(const u32*)(T + 1024 + 4 * l);
  }
  MDEV void f16(u32 jh, u32* o) const {
    const h2v d1 = as_h2((s & 0xffffu) * 0x10001u), m1 = as_h2((s >> 16) * 0x10001u), bias = h2s(1024.0f);
    const u32 nn[4] = {n.x, n.y, n.z, n.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32 v = (nn[k] >> (4 * jh)) & 0x0F0F0F0Fu;
      o[2 * k] = as_u(__builtin_elementwise_fma(mag_lo(v) - bias, d1, m1));
      o[2 * k + 1] = as_u(__builtin_elementwise_fma(mag_hi(v) - bias, d1, m1));
    }
  }
};
template <> struct PkB<FM_Q5_K> {
  uint4 c0, c1;
  u32 s;
  MDEV void ld(const u8* T, u32 l) {
    c0 = *(const uint4*)(T + 16 * l);
    c1 = *(const uint4*)(T + 1024 + 16 * l);
    s = *(const u32*)(T + 2048 + 4 * l);
  }
  MDEV void f16(u32 jh, u32* o) const {
    const h2v d1 = as_h2((s & 0xffffu) * 0x10001u), m1 = as_h2((s >> 16) * 0x10001u), bias = h2s(1024.0f);
    const uint4 c = jh ? c1 : c0;
    const u32 cc[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      o[2 * k] = as_u(__builtin_elementwise_fma(mag_lo(cc[k]) - bias, d1, m1));
      o[2 * k + 1] = as_u(__builtin_elementwise_fma(mag_hi(cc[k]) - bias, d1, m1));
    }
  }
};
template <> struct PkB<FM_Q6_K> {
  uint4 n;
  uint2 H;
  u32 s;
  MDEV void ld(const u8* T, u32 l) {
    n = *(const uint4*)(T + 16 * l);
    H = *(const uint2*)(T + 1024 + 8 * l);
    s = *(const u32*)(T + 1536 + 4 * l);
  }
  MDEV void f16(u32 jh, u32* o) const {
    const h2v ds = as_h2((jh ? s >> 16 : s & 0xffffu) * 0x10001u), bias = h2s(1056.0f);
    const u32 hh = jh ? H.y : H.x;
    const u32 nn[4] = {n.x, n.y, n.z, n.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const u32 v = ((nn[k] >> (4 * jh)) & 0x0F0F0F0Fu) | (((hh >> (2 * k)) & 0x03030303u) << 4);
      o[2 * k] = as_u((mag_lo(v) - bias) * ds);
      o[2 * k + 1] = as_u((mag_hi(v) - bias) * ds);
    }
  }
};

// a lane's weights of one k-tile for one of its rows: from the GGUF row (base = the row) or from the
// packed tiles (base = the row group's tile 0); f16(jh, o) = half_f16 of half jh of the span
template <u32 F, bool PKD> struct BRow;
template <u32 F> struct BRow<F, false> {
  Half<F> a, b;
  u32 c0;
  MDEV void ld(const u8* base, u32 t, u32 l) {
    c0 = 64 * t + 32 * (l >> 5);
    a.ld(base, c0, 0);
    b.ld(base, c0, 1);
  }
  MDEV void f16(u32 jh, u32* o) const { half_f16<F>(jh ? b : a, c0, jh, o); }
};
template <u32 F> struct BRow<F, true> {
  PkB<F> p;
  MDEV void ld(const u8* base, u32 t, u32 l) { p.ld(base + (u64)t * PK<F>::TB, l); }
  MDEV void f16(u32 jh, u32* o) const { p.f16(jh, o); }
};

// ---- the grouped GEMM, weights in registers. Block: 4 waves, a tile of up to G3_BM = 64 slots
// (two 32-row fragments) x 256 weight rows (mode 0: 128 gate + 128 up features, mode 1: 256
// features); wave w owns 64 weight rows (mode 0: gate and up rows of features 32 w .. 32 w + 31, so
// the SwiGLU epilogue pairs them in registers) for every slot of the tile. Each lane dequantizes its
// own weight rows straight into the MFMA B operand: within a k-tile of 64 columns the K order is
// permuted (MFMA k-slot 8 h + e of step s is column 32 h + 8 s + e, lane half h = lane / 32, for A
// and B alike), so a lane's columns for the whole k-tile are one 32-column quant span, decoded once.
// Only the activations go through LDS (two stages of 64 rows x 64 halves, padded to 72), read by
// all four waves. The number of live fragments NL = ceil(rows / 32) is a compile-time variant, so
// dead rows cost neither loads nor MFMAs. Three register slots rotate: at k-tile t a slot's weights
// are decoded and multiplied, the next tile's activations are stored, and the slot is refilled with
// tile t + 3; one barrier a k-tile.
#define G3_BK 64  // columns a k-tile
#define G3_LD 72
#define G3_STAGE (G3_BM * G3_LD)  // halves

template <u32 F, u32 MODE, bool PKD, u32 NL>
DEV void gemm3_body(const GemmArgs& g, _Float16* lds, u32 e, u32 base, u32 m0, u32 M, u32 ntile) {
  const u32 tid = threadIdx.x, w = tid >> 6, l = tid & 63, h = l >> 5, lr = l & 31;
  // A: chunk i of a thread is row 32 i + tid / 8, 16-byte chunk tid % 8 of the k-tile; rows past the
  // tile's slots get an offset past the buffer bound (zeros, no access), so loads stay unconditional
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)g.A, (short)0, (int)(g.arows * g.K * 2u), 0x00020000);
  u32 aoff[NL], src[NL];
#pragma unroll
  for (u32 i = 0; i < NL; i++) src[i] = base + m0 + min(32 * i + (tid >> 3), M - m0 - 1);  // a live slot
  if (MODE == 0 && g.xmap) {
#pragma unroll
    for (u32 i = 0; i < NL; i++) src[i] = g.xmap[src[i]];
  }
#pragma unroll
  for (u32 i = 0; i < NL; i++)
    aoff[i] = m0 + 32 * i + (tid >> 3) < M ? (src[i] * g.K + 8 * (tid & 7)) * 2u : 0x80000000u;
  const u32 nk = g.K / G3_BK;
  // B: this lane's two weight rows (GGUF rows, or their row groups' packed tiles)
  const u8 *br0, *br1;
  if constexpr (PKD) {
    const u64 g0 = MODE == 0 ? 4 * ntile + w : 8 * ntile + 2 * w, tb = (u64)nk * PK<F>::TB;
    br0 = g.P0 + (u64)e * g.pes + g0 * tb;
    br1 = MODE == 0 ? g.P1 + (u64)e * g.pes + g0 * tb : br0 + tb;
  } else if (MODE == 0) {
    const u64 f = (u64)ntile * 128 + 32 * w + lr;
    br0 = g.W0 + (u64)e * g.es + f * g.rb;
    br1 = g.W1 + (u64)e * g.es + f * g.rb;
  } else {
    const u64 n = (u64)ntile * 256 + 64 * w + lr;
    br0 = g.W0 + (u64)e * g.es + n * g.rb;
    br1 = br0 + 32 * g.rb;
  }
  struct Slot {
    uint4 a[NL];
    BRow<F, PKD> b0, b1;
  };
  Slot s0, s1, s2;
  auto load = [&](Slot& s, u32 t) {
    const u32 tc = min(t, nk - 1), k0 = tc * G3_BK;  // past the end: a repeat of the last tile, never used
#pragma unroll
    for (u32 i = 0; i < NL; i++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(arsrc, (int)(aoff[i] + 2 * k0), 0, 0);
      s.a[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    s.b0.ld(br0, tc, l);
    s.b1.ld(br1, tc, l);
  };
  auto store = [&](const Slot& s, u32 t) {
    _Float16* As = lds + (t & 1) * G3_STAGE;
#pragma unroll
    for (u32 i = 0; i < NL; i++) *(uint4*)(As + (32 * i + (tid >> 3)) * G3_LD + 8 * (tid & 7)) = s.a[i];
  };
  f32x16 acc[NL][2];
#pragma unroll
  for (u32 a = 0; a < NL; a++)
#pragma unroll
    for (u32 b = 0; b < 2; b++)
#pragma unroll
      for (u32 i = 0; i < 16; i++) acc[a][b][i] = 0.0f;
  // decode the slot's weights (step s of row b: halves o[4 (s % 2) ..] of half s / 2), multiply tile t
  auto mma = [&](const Slot& s, u32 t) {
    u32 o00[8], o01[8], o10[8], o11[8];
    s.b0.f16(0, o00);
    s.b0.f16(1, o01);
    s.b1.f16(0, o10);
    s.b1.f16(1, o11);
    const _Float16* As = lds + (t & 1) * G3_STAGE + lr * G3_LD + 32 * h;
#pragma unroll
    for (u32 st = 0; st < 4; st++) {
      const u32* p0 = st < 2 ? o00 : o01;
      const u32* p1 = st < 2 ? o10 : o11;
      const u32 j = 4 * (st & 1);
      h8 b0, b1;
      __builtin_memcpy(&b0, p0 + j, 16);
      __builtin_memcpy(&b1, p1 + j, 16);
#pragma unroll
      for (u32 mf = 0; mf < NL; mf++) {
        const h8 a = *(const h8*)(As + 32 * mf * G3_LD + 8 * st);
        acc[mf][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b0, acc[mf][0], 0, 0, 0);
        acc[mf][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b1, acc[mf][1], 0, 0, 0);
      }
    }
  };
  // k-tile t with slot X (holding tile t) and Y (tile t + 1): store Y's activations into the other
  // stage, multiply X, refill X with tile t + 3
  auto step = [&](Slot& X, const Slot& Y, u32 t) {
    if (t + 1 < nk) store(Y, t + 1);
    mma(X, t);
    load(X, t + 3);
    __syncthreads();
  };
  load(s0, 0);
  load(s1, 1);
  load(s2, 2);
  store(s0, 0);
  __syncthreads();
  u32 t = 0;
  for (; t + 3 <= nk; t += 3) {
    step(s0, s1, t);
    step(s1, s2, t + 1);
    step(s2, s0, t + 2);
  }
  if (t < nk) step(s0, s1, t);  // nk % 3 tiles left
  if (t + 1 < nk) step(s1, s2, t + 1);
  // epilogue: acc[mf][b][i] is slot row 32 mf + 8 (i / 4) + 4 h + i % 4 of the tile, weight row lr
  // of the wave's row block b
#pragma unroll
  for (u32 mf = 0; mf < NL; mf++)
#pragma unroll
    for (u32 i = 0; i < 16; i++) {
      const u32 row = 32 * mf + 8 * (i >> 2) + 4 * h + (i & 3);
      if (m0 + row >= M) continue;
      const u64 s = base + m0 + row;
      if (MODE == 0) {
        const float gv = acc[mf][0][i], uv = acc[mf][1][i];
        ((_Float16*)g.out)[s * g.N + ntile * 128 + 32 * w + lr] = (_Float16)(gv / (1.0f + __expf(-gv)) * uv);
      } else {
#pragma unroll
        for (u32 b = 0; b < 2; b++) {
          const u64 o = s * g.N + ntile * 256 + 64 * w + 32 * b + lr;
          if (g.o16) {
            // an output past f16's range keeps its f32 value in the spill, which the combine reads
            // wherever the f16 holds +-inf
            const _Float16 hv = (_Float16)acc[mf][b][i];
            ((_Float16*)g.out)[o] = hv;
            if (__builtin_isinf((float)hv)) g.spill[o] = acc[mf][b][i];
          } else {
            ((float*)g.out)[o] = acc[mf][b][i];
          }
        }
      }
    }
}

// XCD-aware order: the hardware deals block b to XCD b % 8. XCD x takes the contiguous chunk of the
// tile list [x C, x C + C), C = ceil(tiles / 8), and walks it tile by tile, each tile's NT weight-row
// tiles in a row (block b: tile x C + (b / 8) / NT, weight-row tile (b / 8) % NT). So a tile's blocks
// share its activation rows in one L2, and an expert's consecutive slot tiles -- the same weights --
// run on one XCD at about the same time and share its weight slices there (1-D grid,
// 8 NT ceil(max tiles / 8) blocks). Blocks a CU: three on packed weights, two on GGUF rows (whose
// wider per-lane loads need more registers) and for packed Q8_0 gate / up (which would spill at three).
constexpr int g3_blocks(u32 F, u32 MODE, bool PKD) { return PKD && !(F == FM_Q8_0 && MODE == 0) ? 3 : 2; }
// The tile list, read off the slot offsets: expert e has ceil(M_e / BM) slot tiles, listed in expert
// order. Every wave loads the ne + 1 offsets once (16 chunks of 64 experts at most, all loads in
// flight together), sums the tile counts, and finds tile `tile` by an inclusive scan of the counts
// and a ballot -- no list to build, so no launch between the dispatch and the GEMM.
#define G3_NEC 16  // chunks of 64 experts: ne <= 1024
DEV u32 wave_scan_incl(u32 v, u32 L) {
#pragma unroll
  for (u32 m = 1; m < 64; m <<= 1) {
    const u32 o = __shfl_up(v, m, 64);
    if (L >= m) v += o;
  }
  return v;
}
DEV void tiles_load(const u32* __restrict__ off, u32 ne, u32 L, u32* te) {
#pragma unroll
  for (u32 c = 0; c < G3_NEC; c++) {
    const u32 e = 64 * c + L;
    te[c] = e < ne ? (off[e + 1] - off[e] + G3_BM - 1) / G3_BM : 0u;
  }
}
DEV u32 tiles_total(const u32* te, u32 ne) {
  u32 s = 0;
#pragma unroll
  for (u32 c = 0; c < G3_NEC; c++) s += 64 * c < ne ? te[c] : 0u;
#pragma unroll
  for (u32 m = 1; m < 64; m <<= 1) s += __shfl_xor(s, m, 64);
  return s;
}
// tile < the total: its expert and its slot tile within the expert
DEV void tiles_find(const u32* te, u32 ne, u32 tile, u32 L, u32& e, u32& k) {
  u32 acc = 0;
  e = 0;
  k = 0;
#pragma unroll
  for (u32 c = 0; c < G3_NEC; c++) {
    if (64 * c >= ne) break;
    const u32 inc = wave_scan_incl(te[c], L), tot = __shfl(inc, 63, 64);
    if (tile < acc + tot) {  // uniform: tile, acc and tot are the same on every lane
      const u64 b = __ballot(acc + inc > tile);
      const u32 f = (u32)__builtin_ctzll(b);
      e = 64 * c + f;
      k = tile - acc - __shfl(inc - te[c], (int)f, 64);
      break;
    }
    acc += tot;
  }
}

template <u32 F, u32 MODE, bool PKD>
__global__ void __launch_bounds__(256, g3_blocks(F, MODE, PKD)) k_moe_gemm3(GemmArgs g, u32 NT) {
  extern __shared__ _Float16 lds[];
  const u32 q = blockIdx.x >> 3, ntile = q % NT, L = threadIdx.x & 63;
  u32 te[G3_NEC];
  u32 ntl;
  if (g.off) {
    tiles_load(g.off, g.ne, L, te);
    ntl = __builtin_amdgcn_readfirstlane(tiles_total(te, g.ne));
  } else {
    ntl = (g.M + G3_BM - 1) / G3_BM;
  }
  const u32 C = (ntl + 7) / 8;
  const u32 tile = (blockIdx.x & 7) * C + q / NT;
  if (q / NT >= C || tile >= ntl) return;
  u32 e, m0, base, M;
  if (g.off) {
    u32 k;
    tiles_find(te, g.ne, tile, L, e, k);
    e = __builtin_amdgcn_readfirstlane(e);
    m0 = __builtin_amdgcn_readfirstlane(k) * G3_BM;
    base = g.off[e];
    M = g.off[e + 1] - base;
  } else {
    e = 0;
    m0 = tile * G3_BM;
    base = 0;
    M = g.M;
  }
  static_assert(G3_MF == 2, "one or two live fragments");
  if (M - m0 <= 32) gemm3_body<F, MODE, PKD, 1>(g, lds, e, base, m0, M, ntile);
  else gemm3_body<F, MODE, PKD, 2>(g, lds, e, base, m0, M, ntile);
}

// y[t][r] = (sum_j, rank order, wt[t][j] out[inv[t nk + j]][r]) + sgo[t] shd[t][r] + x1[t][r]; the slots'
// down outputs in f16 (half the bytes of the largest intermediate), their weighted sum in f32
template <typename OT>
__global__ void __launch_bounds__(256) k_combine(const OT* __restrict__ out, const float* __restrict__ spill,
                                                 const u32* __restrict__ inv,
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
      if (j0 + j < nk) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const u64 so = (u64)srow[j0 + j] * dm + r;
        if constexpr (sizeof(OT) == 4) {
          v[j] = *(const float4*)(out + so);
        } else {
          const h4 hv = *(const h4*)(out + so);
          v[j] = make_float4((float)hv[0], (float)hv[1], (float)hv[2], (float)hv[3]);
          if (__builtin_isinf(v[j].x)) v[j].x = spill[so];
          if (__builtin_isinf(v[j].y)) v[j].y = spill[so + 1];
          if (__builtin_isinf(v[j].z)) v[j].z = spill[so + 2];
          if (__builtin_isinf(v[j].w)) v[j].w = spill[so + 3];
        }
      }
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

// ---------------------------------------------------------------- the q8 tier's grouped GEMM (int8 MFMA)
//
// The q8 tier for many tokens (the reference's LLB_PREFILL=fast numerics, host/llb_pf.cuh:447-620): the
// slots grouped by expert as for the f16 tier, the activations as q8_1 (codes, {d, s} a 32-column block),
// the weights' codes straight from the GGUF blocks. A 32-column block's integer dot I (codes x codes) is
// one v_mfma_i32_32x32x32_i8 per 32 x 32 tile, exact; the block's value d_w d_x I - m_w s (mx_blk,
// host/llb_pf.cuh:468-515) goes into an f32 accumulator in the epilogue of every block. Q6_K's two
// 16-column scales take two v_mfma_i32_32x32x16_i8 a block. Tile and block order as k_moe_gemm3: 64 slots
// (one or two live 32-row fragments) x 256 weight rows (mode 0: 128 gate + 128 up features, SwiGLU in the
// epilogue), four waves, wave w the weight rows of features 32 w .. (mode 0) or rows 64 w .. (mode 1).
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// a lane's codes of block b of a weight row (GGUF bytes at row): columns 16 h .. 16 h + 15 as 16 signed
// bytes, and the block's scale dw and min mw (the block's value is dw d_x I - mw s)
template <u32 F> DEV void i8_codes(const u8* row, u32 b, u32 h, i32x4& c, float& dw, float& mw);
// Q8_0: the 16 code bytes [p, p + 16) exactly (a block is 34 bytes, so p is 2- or 4-aligned): four
// dwords, or a u16, three dwords and a u16. No byte past them is read: past the last block of the last
// row lies the end of the stack.
template <> DEV void i8_codes<FM_Q8_0>(const u8* row, u32 b, u32 h, i32x4& c, float& dw, float& mw) {
  const u8* B = row + 34u * b;
  const u8* p = B + 2 + 16 * h;
  if (((uintptr_t)p & 2u) == 0) {
    const u32* a = (const u32*)p;
#pragma unroll
    for (int k = 0; k < 4; k++) c[k] = (int)a[k];
  } else {
    const u32* m = (const u32*)(p + 2);
    const u32 lo = ld_u16(p), m0 = m[0], m1 = m[1], m2 = m[2], hi = ld_u16(p + 14);
    c[0] = (int)(lo | m0 << 16);
    c[1] = (int)(m0 >> 16 | m1 << 16);
    c[2] = (int)(m1 >> 16 | m2 << 16);
    c[3] = (int)(m2 >> 16 | hi << 16);
  }
  dw = f16v(ld_u16(B));
  mw = 0.0f;
}
template <> DEV void i8_codes<FM_Q4_K>(const u8* row, u32 b, u32 h, i32x4& c, float& dw, float& mw) {
  const u8* B = row + 144u * (b >> 3);
  const u32 j = b & 7u;
  const uint4 hd = *(const uint4*)B;
  const uint4 q = *(const uint4*)(B + 16 + 32 * (j >> 1) + 16 * h);
  const u32 sh = 4u * (j & 1u);
  c[0] = (int)((q.x >> sh) & 0x0F0F0F0Fu);
  c[1] = (int)((q.y >> sh) & 0x0F0F0F0Fu);
  c[2] = (int)((q.z >> sh) & 0x0F0F0F0Fu);
  c[3] = (int)((q.w >> sh) & 0x0F0F0F0Fu);
  u32 sc, mn;
  k4_scmin(hd, j, sc, mn);
  dw = f16v(hd.x & 0xffffu) * (float)sc;
  mw = f16v(hd.x >> 16) * (float)mn;
}
template <> DEV void i8_codes<FM_Q5_K>(const u8* row, u32 b, u32 h, i32x4& c, float& dw, float& mw) {
  const u8* B = row + 176u * (b >> 3);
  const u32 j = b & 7u;
  const uint4 hd = *(const uint4*)B;
  const uint4 qh = *(const uint4*)(B + 16 + 16 * h);
  const uint4 q = *(const uint4*)(B + 48 + 32 * (j >> 1) + 16 * h);
  const u32 sh = 4u * (j & 1u);
  c[0] = (int)(((q.x >> sh) & 0x0F0F0F0Fu) | (((qh.x >> j) & 0x01010101u) << 4));
  c[1] = (int)(((q.y >> sh) & 0x0F0F0F0Fu) | (((qh.y >> j) & 0x01010101u) << 4));
  c[2] = (int)(((q.z >> sh) & 0x0F0F0F0Fu) | (((qh.z >> j) & 0x01010101u) << 4));
  c[3] = (int)(((q.w >> sh) & 0x0F0F0F0Fu) | (((qh.w >> j) & 0x01010101u) << 4));
  u32 sc, mn;
  k4_scmin(hd, j, sc, mn);
  dw = f16v(hd.x & 0xffffu) * (float)sc;
  mw = f16v(hd.x >> 16) * (float)mn;
}
// Q6_K: half k (columns 16 k .. 16 k + 15) of block b, the lane's 8 columns 16 k + 8 h .. as q - 32
// (signed bytes), and that half's scale d sc_k
DEV void i8_q6_half(const u8* row, u32 b, u32 k, u32 h, long& c, float& ds) {
  const u8* B = row + 210u * (b >> 3);
  const u32 bb = b & 7u, n = bb >> 2, quad = bb & 3u, i0 = 16 * k + 8 * h;
  const u8* pl = B + 64 * n + 32 * (quad & 1u) + i0;
  const u8* ph = B + 128 + 32 * n + i0;
  const u32 nsh = quad >= 2u ? 4u : 0u, hsh = 2u * quad;
  u32 o[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const u32 lw = ld_u16(pl + 4 * t) | ld_u16(pl + 4 * t + 2) << 16;
    const u32 hw = ld_u16(ph + 4 * t) | ld_u16(ph + 4 * t + 2) << 16;
    const u32 v = ((lw >> nsh) & 0x0F0F0F0Fu) | (((hw >> hsh) & 0x03030303u) << 4);
    o[t] = ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;  // per byte q - 32
  }
  c = (long)((u64)o[0] | (u64)o[1] << 32);
  ds = f16v(ld_u16(B + 208)) * (float)(int)(signed char)B[192 + 8 * n + 2 * quad + k];
}


constexpr u32 QG_CH = 32;  // blocks of {d, s} staged in LDS at a time (64 slots x 32 blocks x 8 bytes)

template <u32 F, u32 MODE, u32 NL>
DEV void gemm_i8_body(const GemmQ8Args& g, float2* lsd, u32 e, u32 base, u32 m0, u32 M, u32 ntile) {
  const u32 tid = threadIdx.x, w = tid >> 6, l = tid & 63, h = l >> 5, lr = l & 31;
  const u32 nb = g.K / 32;
  const u32 live = M - m0;
  const int8_t* arow[NL];
#pragma unroll
  for (u32 mf = 0; mf < NL; mf++) {
    const u32 slot = base + m0 + min(32 * mf + lr, live - 1);  // rows past the tile repeat a live one
    const u32 src = g.xmap ? g.xmap[slot] : slot;
    arow[mf] = g.A + (u64)src * g.K + 16 * h;
  }
  const u8 *br0, *br1;
  if (MODE == 0) {
    const u64 f = (u64)ntile * 128 + 32 * w + lr;
    br0 = g.W0 + (u64)e * g.es + f * g.rb;
    br1 = g.W1 + (u64)e * g.es + f * g.rb;
  } else {
    const u64 n = (u64)ntile * 256 + 64 * w + lr;
    br0 = g.W0 + (u64)e * g.es + n * g.rb;
    br1 = br0 + 32 * g.rb;
  }
  float acc[NL][2][16];
#pragma unroll
  for (u32 mf = 0; mf < NL; mf++)
#pragma unroll
    for (u32 nf = 0; nf < 2; nf++)
#pragma unroll
      for (u32 i = 0; i < 16; i++) acc[mf][nf][i] = 0.0f;
  const i32x16 z16 = {};
  for (u32 c0 = 0; c0 < nb; c0 += QG_CH) {
    const u32 cn = min(QG_CH, nb - c0);
    __syncthreads();  // the previous chunk's readers are done
    for (u32 i = tid; i < 64 * cn; i += 256) {
      const u32 b = i / 64, r = i % 64;
      const u32 slot = base + m0 + min(r, live - 1);
      const u32 src = g.xmap ? g.xmap[slot] : slot;
      lsd[i] = g.Ad[(u64)src * nb + c0 + b];
    }
    __syncthreads();
#pragma unroll 2
    for (u32 bi = 0; bi < cn; bi++) {
      const u32 b = c0 + bi;
      if constexpr (F == FM_Q6_K) {
        long a0[NL], a1[NL], w00, w01, w10, w11;
        float s00, s01, s10, s11;
#pragma unroll
        for (u32 mf = 0; mf < NL; mf++) {
          a0[mf] = *(const long*)(arow[mf] + 32 * b - 8 * h);       // columns 8 h .. 8 h + 7
          a1[mf] = *(const long*)(arow[mf] + 32 * b + 16 - 8 * h);  // columns 16 + 8 h ..
        }
        i8_q6_half(br0, b, 0, h, w00, s00);
        i8_q6_half(br0, b, 1, h, w01, s01);
        i8_q6_half(br1, b, 0, h, w10, s10);
        i8_q6_half(br1, b, 1, h, w11, s11);
#pragma unroll
        for (u32 mf = 0; mf < NL; mf++) {
          const i32x16 p00 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0[mf], w00, z16, 0, 0, 0);
          const i32x16 p01 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1[mf], w01, z16, 0, 0, 0);
          const i32x16 p10 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0[mf], w10, z16, 0, 0, 0);
          const i32x16 p11 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1[mf], w11, z16, 0, 0, 0);
#pragma unroll
          for (u32 i = 0; i < 16; i++) {
            const float dx = lsd[bi * 64 + 32 * mf + 8 * (i >> 2) + 4 * h + (i & 3)].x;
            acc[mf][0][i] = __builtin_fmaf(dx, __builtin_fmaf(s01, (float)p01[i], s00 * (float)p00[i]), acc[mf][0][i]);
            acc[mf][1][i] = __builtin_fmaf(dx, __builtin_fmaf(s11, (float)p11[i], s10 * (float)p10[i]), acc[mf][1][i]);
          }
        }
      } else {
        i32x4 a[NL], w0, w1;
        float dw0, mw0, dw1, mw1;
#pragma unroll
        for (u32 mf = 0; mf < NL; mf++) a[mf] = *(const i32x4*)(arow[mf] + 32 * b);
        i8_codes<F>(br0, b, h, w0, dw0, mw0);
        i8_codes<F>(br1, b, h, w1, dw1, mw1);
#pragma unroll
        for (u32 mf = 0; mf < NL; mf++) {
          const i32x16 p0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[mf], w0, z16, 0, 0, 0);
          const i32x16 p1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[mf], w1, z16, 0, 0, 0);
#pragma unroll
          for (u32 i = 0; i < 16; i++) {
            const float2 ds = lsd[bi * 64 + 32 * mf + 8 * (i >> 2) + 4 * h + (i & 3)];
            float v0 = __builtin_fmaf(dw0 * ds.x, (float)p0[i], acc[mf][0][i]);
            float v1 = __builtin_fmaf(dw1 * ds.x, (float)p1[i], acc[mf][1][i]);
            if constexpr (F != FM_Q8_0) {
              v0 = __builtin_fmaf(-mw0, ds.y, v0);
              v1 = __builtin_fmaf(-mw1, ds.y, v1);
            }
            acc[mf][0][i] = v0;
            acc[mf][1][i] = v1;
          }
        }
      }
    }
  }
  // epilogue: acc[mf][b][i] is slot row 32 mf + 8 (i / 4) + 4 h + i % 4 of the tile, weight row lr of
  // the wave's row block b
#pragma unroll
  for (u32 mf = 0; mf < NL; mf++)
#pragma unroll
    for (u32 i = 0; i < 16; i++) {
      const u32 row = 32 * mf + 8 * (i >> 2) + 4 * h + (i & 3);
      if (m0 + row >= M) continue;
      const u64 s = base + m0 + row;
      if (MODE == 0) {
        g.out[s * g.N + ntile * 128 + 32 * w + lr] = silu_mul(acc[mf][0][i], acc[mf][1][i]);
      } else {
#pragma unroll
        for (u32 b = 0; b < 2; b++) g.out[s * g.N + ntile * 256 + 64 * w + 32 * b + lr] = acc[mf][b][i];
      }
    }
}

template <u32 F, u32 MODE>
__global__ void __launch_bounds__(256, 2) k_gemm_i8(GemmQ8Args g, u32 NT) {
  __shared__ float2 lsd[64 * QG_CH];
  const u32 q = blockIdx.x >> 3, ntile = q % NT, L = threadIdx.x & 63;
  u32 te[G3_NEC];
  u32 ntl;
  if (g.off) {
    tiles_load(g.off, g.ne, L, te);
    ntl = __builtin_amdgcn_readfirstlane(tiles_total(te, g.ne));
  } else {
    ntl = (g.M + G3_BM - 1) / G3_BM;
  }
  const u32 C = (ntl + 7) / 8;
  const u32 tile = (blockIdx.x & 7) * C + q / NT;
  if (q / NT >= C || tile >= ntl) return;
  u32 e, m0, base, M;
  if (g.off) {
    u32 k;
    tiles_find(te, g.ne, tile, L, e, k);
    e = __builtin_amdgcn_readfirstlane(e);
    m0 = __builtin_amdgcn_readfirstlane(k) * G3_BM;
    base = g.off[e];
    M = g.off[e + 1] - base;
  } else {
    e = 0;
    m0 = tile * G3_BM;
    base = 0;
    M = g.M;
  }
  if (M - m0 <= 32) gemm_i8_body<F, MODE, 1>(g, lsd, e, base, m0, M, ntile);
  else gemm_i8_body<F, MODE, 2>(g, lsd, e, base, m0, M, ntile);
}

int launch_gemm_i8(const GemmQ8Args& g, u32 fm, u32 mode, u32 grid_y, hipStream_t st) {
  const u32 nf = mode == 0 ? 128u : 256u;
  if (g.K % 32 || g.N % nf || fm == FM_F32) return -1;
  if ((fm != FM_Q8_0 && g.K % 256) || (g.off && (g.ne == 0 || g.ne > 64 * G3_NEC))) return -1;
  const u32 NT = g.N / nf;
  const dim3 grid(8 * NT * ((grid_y + 7) / 8));
#define GI_L(F) \
  if (fm == F) { \
    if (mode == 0) LAUNCH_K((k_gemm_i8<F, 0>), grid, dim3(256), 0, st, g, NT); \
    else LAUNCH_K((k_gemm_i8<F, 1>), grid, dim3(256), 0, st, g, NT); \
    return 0; \
  }
  GI_L(FM_Q8_0) GI_L(FM_Q4_K) GI_L(FM_Q5_K) GI_L(FM_Q6_K)
#undef GI_L
  return -1;
}

// ---------------------------------------------------------------- launchers

template <u32 F, u32 MODE, bool PKD> static void gemm3_go(const GemmArgs& g, dim3 grid, size_t sm, hipStream_t st) {
  static std::atomic<uint64_t> set{0};
  const uint64_t bit = dev_bit();
  if (dev_needs_setup(set, bit)) {
    (void)hipFuncSetAttribute((const void*)k_moe_gemm3<F, MODE, PKD>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sm);
    set.fetch_or(bit);
  }
  LAUNCH_K((k_moe_gemm3<F, MODE, PKD>), grid, dim3(256), sm, st, g, g.N / (MODE == 0 ? 128u : 256u));
}

int launch_moe_gemm(const GemmArgs& g, u32 fm, u32 mode, u32 grid_y, hipStream_t st) {
  const u32 nf = mode == 0 ? 128u : 256u;
  // A's buffer loads take 32-bit offsets below 2^31 (dead rows use 2^31)
  if (g.K % G3_BK || g.N % nf || fm == FM_F32 || (u64)g.arows * g.K * 2 >= (1ull << 31)) return -1;
  if (g.off && (g.ne == 0 || g.ne > 64 * G3_NEC)) return -1;
  const dim3 grid(8 * (g.N / nf) * ((grid_y + 7) / 8));
  const size_t sm = (size_t)2 * G3_STAGE * 2;
  const bool pk = g.P0 != nullptr;
#define G3_L(F) \
  if (fm == F) { \
    if (mode == 0) pk ? gemm3_go<F, 0, true>(g, grid, sm, st) : gemm3_go<F, 0, false>(g, grid, sm, st); \
    else pk ? gemm3_go<F, 1, true>(g, grid, sm, st) : gemm3_go<F, 1, false>(g, grid, sm, st); \
    return 0; \
  }
  G3_L(FM_Q8_0) G3_L(FM_Q4_K) G3_L(FM_Q6_K) G3_L(FM_Q5_K)
#undef G3_L
  return -1;
}

// packed copy of ne stacked matrices of R rows x K columns (GGUF expert stride es, row bytes rb)
u64 pack_bytes(u32 fm, u32 R, u32 K) {
  if (R % 32 || K % 64) return 0;
  u32 tb = 0;
  if (fm == FM_Q8_0) tb = PK<FM_Q8_0>::TB;
  else if (fm == FM_Q4_K) tb = PK<FM_Q4_K>::TB;
  else if (fm == FM_Q5_K) tb = PK<FM_Q5_K>::TB;
  else if (fm == FM_Q6_K) tb = PK<FM_Q6_K>::TB;
  return (u64)(R / 32) * (K / 64) * tb;
}
int launch_pack(u32 fm, const u8* W, u64 es, u64 rb, u32 R, u32 K, u32 ne, u8* P, hipStream_t st) {
  if (!pack_bytes(fm, R, K) || ne == 0) return -1;
  const dim3 grid((R / 32) * (K / 64), ne);
#define PK_L(F) \
  if (fm == F) { LAUNCH_K((k_pack<F>), grid, dim3(64), 0, st, W, es, rb, K, P); return 0; }
  PK_L(FM_Q8_0) PK_L(FM_Q4_K) PK_L(FM_Q6_K) PK_L(FM_Q5_K)
#undef PK_L
  return -1;
}

int launch_combine(const _Float16* out, const float* spill, const u32* inv, const float* wt, u32 nk, const float* shd,
                   const float* sgo, const float* x1, float* y, u32 dm, u32 T, hipStream_t st) {
  if (dm % 4 || nk > 64 || !spill) return -1;
  hipLaunchKernelGGL(k_combine<_Float16>, dim3((dm / 4 + 255) / 256, T), dim3(256), 0, st, out, spill, inv, wt, nk, shd,
                     sgo, x1, y, dm);
  return 0;
}
int launch_combine_f32(const float* out, const u32* inv, const float* wt, u32 nk, const float* shd, const float* sgo,
                       const float* x1, float* y, u32 dm, u32 T, hipStream_t st) {
  if (dm % 4 || nk > 64) return -1;
  hipLaunchKernelGGL(k_combine<float>, dim3((dm / 4 + 255) / 256, T), dim3(256), 0, st, out, nullptr, inv, wt, nk, shd,
                     sgo, x1, y, dm);
  return 0;
}
u32 gemm_bm() { return GM_BM; }
