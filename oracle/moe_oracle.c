/* moe_oracle.c -- CPU restatement of eureka-engine's MoE FFN hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never linked into the product.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp -shared).
 *
 * Each function cites the reference code it restates. The exact tier's float ops
 * are written one rounding per C operator, in the reference's order; with
 * -ffp-contract=off gcc emits them as written, so the results are the bits the
 * reference's exact CUDA kernels produce (and the bits the HIP exact tier must produce).
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef uint32_t u32;
typedef uint64_t u64;
typedef uint8_t u8;

static float as_f(u32 u) { float f; memcpy(&f, &u, 4); return f; }
static u32 as_u(float f) { u32 u; memcpy(&u, &f, 4); return u; }

/* ------------------------------------------------------------------ formats */

/* llb_f16 (tools/quant-fix.patch:11-21): (m [+1024]) * 2^(e' - 25), exact in f32;
 * exponent 31 -> inf / NaN with the mantissa kept */
float mo_f16(u32 h) {
  u32 e = (h >> 10) & 31u, m = h & 1023u, s = (h >> 15) << 31;
  float mag = (float)(e ? m + 1024u : m) * as_f(((e ? e : 1u) + 102u) << 23);
  return as_f(e == 31u ? (s | 0x7f800000u | m << 13) : (as_u(mag) | s));
}

/* IEEE binary16 from binary32, round to nearest even (integer-only, so host and device agree) */
uint16_t mo_f32_to_f16(float f) {
  u32 x = as_u(f), s = (x >> 16) & 0x8000u, e = (x >> 23) & 255u, m = x & 0x7fffffu;
  if (e == 255u) return (uint16_t)(s | 0x7c00u | (m ? 0x200u | (m >> 13) : 0u));
  int ee = (int)e - 127 + 15;
  if (ee >= 31) return (uint16_t)(s | 0x7c00u);
  if (ee <= 0) {
    if (ee < -10) return (uint16_t)s;
    u32 mm = m | 0x800000u, sh = (u32)(14 - ee);
    u32 hm = mm >> sh, rem = mm & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (hm & 1u))) hm += 1u;
    return (uint16_t)(s | hm);
  }
  u32 hm = m >> 13, rem = m & 0x1fffu;
  u32 r = s | ((u32)ee << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) r += 1u; /* carries into the exponent correctly */
  return (uint16_t)r;
}

/* LLB_FM_RB (host/llb_formats.h:16) */
uint64_t mo_row_bytes(u32 fm, u32 cols) {
  switch (fm) {
    case MO_F32: return (u64)cols * 4u;
    case MO_Q8_0: return (u64)cols / 32u * 34u;
    case MO_Q4_K: return (u64)cols / 256u * 144u;
    case MO_Q6_K: return (u64)cols / 256u * 210u;
    case MO_Q5_K: return (u64)cols / 256u * 176u;
  }
  return 0;
}

static float h2f(const u8* p) { return mo_f16((u32)p[0] | (u32)p[1] << 8); }

/* ggml get_scale_min_k4 (tools/qwen35_engine.c:64-70, tools/q4k.py:20-23) */
static void scmin(int j, const u8* q, int* sd, int* sm) {
  if (j < 4) { *sd = q[j] & 63; *sm = q[j + 4] & 63; }
  else { *sd = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4); *sm = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}

/* deq_row (tools/qwen35_engine.c:233-327) for the expert-stack formats; Q8_0 here is the GGUF
 * block layout the stacks keep (q8g_w, tools/payload-moeany.patch:85-91), not the trunk's row split.
 * Every value is the reference's: Q8_0 q*d, Q4_K (d*sc)*q - dmin*m, Q6_K (d*sc)*(q-32). */
int mo_deq_row(u32 fm, const u8* row, u32 cols, float* out) {
  if (fm == MO_F32) { memcpy(out, row, (size_t)cols * 4); return 0; }
  if (fm == MO_Q8_0) {
    if (cols % 32) return -1;
    for (u32 b = 0; b < cols / 32; b++) {
      const u8* B = row + (size_t)b * 34;
      float d = h2f(B);
      for (u32 j = 0; j < 32; j++) out[32 * b + j] = (float)(int8_t)B[2 + j] * d;
    }
    return 0;
  }
  if (cols % 256) return -1;
  for (u32 b = 0; b < cols / 256; b++) {
    float* o = out + 256 * (size_t)b;
    if (fm == MO_Q4_K || fm == MO_Q5_K) {
      const u32 sbb = fm == MO_Q4_K ? 144u : 176u;
      const u8* B = row + (size_t)b * sbb;
      float d = h2f(B), dmin = h2f(B + 2);
      const u8* sc = B + 4;
      const u8* qh = B + 16;
      const u8* qs = B + (fm == MO_Q4_K ? 16 : 48);
      for (int g = 0; g < 4; g++) {
        int sd, sm;
        scmin(2 * g, sc, &sd, &sm);
        float d1 = d * (float)sd, m1 = dmin * (float)sm;
        scmin(2 * g + 1, sc, &sd, &sm);
        float d2 = d * (float)sd, m2 = dmin * (float)sm;
        const u8* q = qs + 32 * g;
        for (int l = 0; l < 32; l++) {
          int lo = q[l] & 0xF, hi = q[l] >> 4;
          if (fm == MO_Q5_K) { lo += ((qh[l] >> (2 * g)) & 1) * 16; hi += ((qh[l] >> (2 * g + 1)) & 1) * 16; }
          o[64 * g + l] = d1 * (float)lo - m1;
          o[64 * g + 32 + l] = d2 * (float)hi - m2;
        }
      }
    } else if (fm == MO_Q6_K) {
      const u8* B = row + (size_t)b * 210;
      const u8 *ql = B, *qh = B + 128;
      const int8_t* scb = (const int8_t*)(B + 192);
      float d = h2f(B + 208);
      for (int half = 0; half < 2; half++) {
        for (int qd = 0; qd < 4; qd++) {
          const u8* qq = ql + 64 * half + 32 * (qd & 1);
          for (int l = 0; l < 32; l++) {
            int nib = qd < 2 ? (qq[l] & 0xF) : (qq[l] >> 4);
            int code = (nib | (((qh[32 * half + l] >> (2 * qd)) & 3) << 4)) - 32;
            o[128 * half + 32 * qd + l] = (d * (float)scb[8 * half + 2 * qd + (l >> 4)]) * (float)code;
          }
        }
      }
    } else {
      return -1;
    }
  }
  return 0;
}

/* ---- quantizers. The reference quantizes with llama.cpp's ggml routines
 * (tools/q4k.py:115-139), which are not vendored; these are this project's own
 * (Q8_0 is ggml's closed form, quantize_row_q8_0_ref; Q4_K / Q5_K are min-max
 * per 32-value sub-block with 6-bit scale / min codes against the super-block's
 * largest; Q6_K is max-abs per 16-value sub-block with int8 scale codes).
 * They define the bytes both sides read: parity is checked on dequantization,
 * which the reference fixes in closed form. */
static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

static void q8_0_block(const float* x, u8* B) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); amax = a > amax ? a : amax; }
  const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  uint16_t h = mo_f32_to_f16(d);
  B[0] = (u8)h; B[1] = (u8)(h >> 8);
  for (int j = 0; j < 32; j++) B[2 + j] = (u8)(int8_t)clampi((int)roundf(x[j] * id), -127, 127);
}

static void q45_block(const float* x, u8* B, int five) {
  const float lv = five ? 31.0f : 15.0f;
  const int qmax = five ? 31 : 15;
  float scale[8], mn[8], maxs = 0.0f, maxm = 0.0f;
  for (int j = 0; j < 8; j++) {
    float lo = 0.0f, hi = x[32 * j];
    for (int i = 0; i < 32; i++) {
      float v = x[32 * j + i];
      lo = v < lo ? v : lo;
      hi = v > hi ? v : hi;
    }
    scale[j] = (hi - lo) / lv;
    mn[j] = -lo;
    maxs = scale[j] > maxs ? scale[j] : maxs;
    maxm = mn[j] > maxm ? mn[j] : maxm;
  }
  const uint16_t hd = mo_f32_to_f16(maxs / 63.0f), hm = mo_f32_to_f16(maxm / 63.0f);
  const float dd = mo_f16(hd), dmd = mo_f16(hm);
  int sc[8], m[8];
  for (int j = 0; j < 8; j++) {
    sc[j] = dd > 0.0f ? clampi((int)roundf(scale[j] / dd), 0, 63) : 0;
    m[j] = dmd > 0.0f ? clampi((int)roundf(mn[j] / dmd), 0, 63) : 0;
  }
  memset(B, 0, five ? 176 : 144);
  B[0] = (u8)hd; B[1] = (u8)(hd >> 8); B[2] = (u8)hm; B[3] = (u8)(hm >> 8);
  u8* s = B + 4;
  for (int j = 0; j < 4; j++) {
    s[j] = (u8)(sc[j] | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (u8)(m[j] | ((m[j + 4] >> 4) << 6));
    s[j + 8] = (u8)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
  }
  u8* qh = B + 16;
  u8* qs = B + (five ? 48 : 16);
  for (int j = 0; j < 8; j++) {
    const float d1 = dd * (float)sc[j], m1 = dmd * (float)m[j];
    for (int i = 0; i < 32; i++) {
      int q = d1 > 0.0f ? clampi((int)roundf((x[32 * j + i] + m1) / d1), 0, qmax) : 0;
      /* col 64 g + 32 hi + l: nibble hi of qs[32 g + l]; fifth bit 2 g + hi of qh[l] */
      int g = j >> 1, hi = j & 1;
      qs[32 * g + i] |= (u8)((q & 15) << (4 * hi));
      if (five) qh[i] |= (u8)(((q >> 4) & 1) << (2 * g + hi));
    }
  }
}

static void q6_block(const float* x, u8* B) {
  float scale[16], maxs = 0.0f;
  for (int j = 0; j < 16; j++) {
    float a = 0.0f;
    for (int i = 0; i < 16; i++) { float v = fabsf(x[16 * j + i]); a = v > a ? v : a; }
    scale[j] = a / 31.0f;
    maxs = scale[j] > maxs ? scale[j] : maxs;
  }
  const uint16_t hd = mo_f32_to_f16(maxs / 127.0f);
  const float dd = mo_f16(hd);
  memset(B, 0, 210);
  for (int j = 0; j < 16; j++) {
    int sc = dd > 0.0f ? clampi((int)roundf(scale[j] / dd), 0, 127) : 0;
    B[192 + j] = (u8)(int8_t)sc;
    const float ds = dd * (float)sc;
    for (int i = 0; i < 16; i++) {
      int c = 16 * j + i;
      int q = ds > 0.0f ? clampi((int)roundf(x[c] / ds), -32, 31) : 0;
      u32 u = (u32)(q + 32);
      int n = c >> 7, r = c & 127, quad = r >> 5, l = r & 31;
      B[64 * n + 32 * (quad & 1) + l] |= (u8)((u & 15) << (quad >= 2 ? 4 : 0));
      B[128 + 32 * n + l] |= (u8)((u >> 4) << (2 * quad));
    }
  }
  B[208] = (u8)hd; B[209] = (u8)(hd >> 8);
}

int mo_quant_row(u32 fm, const float* x, u32 cols, u8* out) {
  if (fm == MO_F32) { memcpy(out, x, (size_t)cols * 4); return 0; }
  if (fm == MO_Q8_0) {
    if (cols % 32) return -1;
    for (u32 b = 0; b < cols / 32; b++) q8_0_block(x + 32 * b, out + 34 * (size_t)b);
    return 0;
  }
  if (cols % 256) return -1;
  for (u32 b = 0; b < cols / 256; b++) {
    if (fm == MO_Q4_K) q45_block(x + 256 * b, out + 144 * (size_t)b, 0);
    else if (fm == MO_Q5_K) q45_block(x + 256 * b, out + 176 * (size_t)b, 1);
    else if (fm == MO_Q6_K) q6_block(x + 256 * b, out + 210 * (size_t)b);
    else return -1;
  }
  return 0;
}

/* ---- synthetic normals: splitmix64 finaliser, Irwin-Hall sum of four 16-bit uniforms.
 * Integer arithmetic and one rounding (the final multiply), so the product's device
 * generator reproduces the same floats. sd of the 4-sum is sqrt(4 (2^32 - 1) / 12). */
static u64 mo_mix(u64 z) {
  z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27; z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}
float mo_gauss(u64 seed, u64 stream, u64 i, float sigma) {
  const u64 key = mo_mix(seed + 0x9E3779B97F4A7C15ull * (stream + 1u));
  const u64 h = mo_mix(key + 0x9E3779B97F4A7C15ull * (i + 1u));
  const u32 s = (u32)(h & 0xffffu) + (u32)((h >> 16) & 0xffffu) + (u32)((h >> 32) & 0xffffu) + (u32)(h >> 48);
  const float k = sigma * 2.6428983e-5f;
  return ((float)s - 131070.0f) * k;
}
void mo_gauss_fill(u64 seed, u64 stream, u64 i0, u64 n, float sigma, float* out) {
  for (u64 i = 0; i < n; i++) out[i] = mo_gauss(seed, stream, i0 + i, sigma);
}
/* rows are independent: split over OpenMP threads (each row's bytes depend only on its own index) */
int mo_gen_rows(u32 fm, u64 seed, u64 stream, u64 r0, u64 nr, u32 cols, float sigma, u8* out) {
  const u64 rb = mo_row_bytes(fm, cols);
  if (rb == 0) return -1;
  int rc = 0;
#pragma omp parallel if (nr >= 64)
  {
    float* x = (float*)malloc((size_t)cols * 4);
    int mine = x ? 0 : -2;
#pragma omp for schedule(static)
    for (long long r = 0; r < (long long)nr; r++) {
      if (mine) continue;
      mo_gauss_fill(seed, stream, (r0 + (u64)r) * cols, cols, sigma, x);
      mine = mo_quant_row(fm, x, cols, out + (u64)r * rb);
    }
#pragma omp critical
    if (mine && !rc) rc = mine;
    free(x);
  }
  return rc;
}

/* ------------------------------------------------------------------ dots */

/* llb_cdepth (host/llb_host.c:52-58): ceil(log2(cols)) - 2 */
u32 mo_cdepth(u32 cols) {
  u32 d = 0;
  while ((1u << d) < cols) d++;
  return d - 2;
}

/* llb_tuned (host/llb_host.c:64-76) for the formats this path takes. The Q8_0 tree
 * bodies read the trunk's row-split Q8_0, not GGUF blocks: none here. */
int mo_tuned(u32 fm, u32 cols) {
  u32 d = mo_cdepth(cols), cg = cols / 4;
  if (fm == MO_F32) return d >= 9 && d <= 12;
  if (fm == MO_Q4_K || fm == MO_Q6_K) return (cg % 256 == 0 && d >= 8 && d <= 13) || (d >= 9 && d <= 11);
  if (fm == MO_Q5_K) return cg % 256 == 0 && d >= 8 && d <= 13;
  return 0;
}

/* the leaf of every exact GEMV: (w0 x0 + w1 x1) + (w2 x2 + w3 x3) */
static float leaf(const float* w, const float* x) {
  return ((w[0] * x[0]) + (w[1] * x[1])) + ((w[2] * x[2]) + (w[3] * x[3]));
}

/* moe_dot (tools/payload-moeany.patch:95-109) = llb_gemv_any's order
 * (tools/payload-anyshape.patch:89-121): lane l of 32 sums the groups l, l + 32, ...
 * (a group = 4 columns) in ascending order, acc + leaf; then the xor butterfly
 * m = 16, 8, 4, 2, 1 (a + b commutes, so every lane ends with the same value). */
static float dot_stride_f(const float* w, u32 cols, const float* x) {
  const u32 cg = cols / 4;
  float acc[32];
  for (u32 l = 0; l < 32; l++) {
    float a = 0.0f;
    for (u32 g = l; g < cg; g += 32) a = a + leaf(w + 4 * g, x + 4 * g);
    acc[l] = a;
  }
  for (u32 m = 16; m > 0; m >>= 1) {
    float t[32];
    for (u32 l = 0; l < 32; l++) t[l] = acc[l] + acc[l ^ m];
    memcpy(acc, t, sizeof t);
  }
  return acc[0];
}

/* the engine tree (llb_warp, tools/remap.patch:116-171; kp_pair, tools/payload-kpair.patch):
 * 2^cdepth group leaves in index order (pad groups past cols / 4 count +0), summed by a
 * balanced pairwise tree, lower index on the left */
static float dot_tree_f(const float* w, u32 cols, const float* x) {
  const u32 cg = cols / 4, ng = 1u << mo_cdepth(cols);
  float* v = (float*)malloc((size_t)ng * 4);
  for (u32 g = 0; g < ng; g++) v[g] = g < cg ? leaf(w + 4 * g, x + 4 * g) : 0.0f;
  for (u32 st = 1; st < ng; st <<= 1)
    for (u32 g = 0; g < ng; g += 2 * st) v[g] = v[g] + v[g + st];
  float r = v[0];
  free(v);
  return r;
}

float mo_dot_stride(u32 fm, const u8* row, u32 cols, const float* x) {
  float* w = (float*)malloc((size_t)cols * 4);
  float r = mo_deq_row(fm, row, cols, w) == 0 ? dot_stride_f(w, cols, x) : NAN;
  free(w);
  return r;
}
float mo_dot_tree(u32 fm, const u8* row, u32 cols, const float* x) {
  float* w = (float*)malloc((size_t)cols * 4);
  float r = mo_deq_row(fm, row, cols, w) == 0 ? dot_tree_f(w, cols, x) : NAN;
  free(w);
  return r;
}
/* llb_kgemv (host/llb_host.c:100-152): the tuned body's tree where llb_tuned holds, else llb_gany */
float mo_gemv_row(u32 fm, const u8* row, u32 cols, const float* x) {
  return mo_tuned(fm, cols) ? mo_dot_tree(fm, row, cols, x) : mo_dot_stride(fm, row, cols, x);
}

/* attn_exp (tools/payload-attn.patch:57-59): exp through double, rounded once */
float mo_exp(float x) { return (float)exp((double)x); }
/* llb_moe_gu's epilogue (tools/payload-moeany.patch:495): silu(g) * u = (g / (1 + exp(-g))) * u */
float mo_silu_mul(float g, float u) { return (g / (1.0f + mo_exp(-g))) * u; }
/* llb_moe_topk's shared gate (tools/payload-moeany.patch:468): 1 / (1 + exp(-sg)) */
float mo_sigmoid(float x) { return 1.0f / (1.0f + mo_exp(-x)); }
/* llb_moe_topk's renormalisation (tools/payload-moeany.patch:459-467): s = the k weights summed in rank
 * order from 0.0f, clamped below at 2^-14; each weight divided by s */
void mo_renorm(float* wt, u32 nk) {
  float s = 0.0f;
  for (u32 j = 0; j < nk; j++) s = s + wt[j];
  s = s < 6.103515625e-5f ? 6.103515625e-5f : s;
  for (u32 j = 0; j < nk; j++) wt[j] = wt[j] / s;
}
/* llb_moe_dn's combine for one output row (tools/payload-moeany.patch:572-592): mo = v0 wt0 (the first
 * term itself, not 0 + v0 wt0), then mo + vj wtj in rank order, each product rounded before its add;
 * y = (mo + hv sgo) + res with the shared expert, mo + res without */
float mo_combine(const float* v, const float* wt, u32 nk, int shared, float hv, float sgo, float res) {
  float mo = 0.0f;
  for (u32 j = 0; j < nk; j++) mo = j == 0 ? v[0] * wt[0] : mo + v[j] * wt[j];
  return shared ? (mo + hv * sgo) + res : mo + res;
}

/* ------------------------------------------------------------------ routing */

void mo_router(const mo_layer* L, const float* h2, float* lg, float* sg) {
  for (u32 e = 0; e < L->ne; e++) {
    lg[e] = mo_gemv_row(MO_F32, (const u8*)(L->router + (size_t)e * L->dm), L->dm, h2);
    if (L->router_bias) lg[e] = lg[e] + L->router_bias[e];
  }
  *sg = L->shgate ? mo_gemv_row(MO_F32, (const u8*)L->shgate, L->dm, h2) : 0.0f;
}

/* llb_moe_topk block 0 (tools/payload-moeany.patch:311-470), one block of 1024 threads:
 * mx = max lg; v_e = exp(lg_e - mx); the sum: thread t adds e = t, t + 1024, ... in order,
 * a 32-lane xor tree per warp, then the 32 warp sums in warp order from 0; p_e = v_e * (1 / sum);
 * the k largest p, ties to the lower index; wt_j / max(sum of the k p in rank order, 2^-14);
 * sgo = 1 / (1 + exp(-sg)). */
void mo_topk(const float* lg, u32 ne, u32 nk, float sg, u32* ids, float* wt, float* sgo) {
  float mx = as_f(0xFF800000u);
  for (u32 e = 0; e < ne; e++) mx = fmaxf(mx, lg[e]);
  float* p = (float*)malloc((size_t)ne * 4);
  float th[1024];
  for (u32 t = 0; t < 1024; t++) th[t] = 0.0f;
  for (u32 e = 0; e < ne; e++) {
    p[e] = mo_exp(lg[e] - mx);
    th[e % 1024] = th[e % 1024] + p[e];
  }
  float tot = 0.0f;
  for (u32 w = 0; w < 32; w++) {
    float a[32];
    for (u32 l = 0; l < 32; l++) a[l] = th[32 * w + l];
    for (u32 m = 16; m > 0; m >>= 1) {
      float t2[32];
      for (u32 l = 0; l < 32; l++) t2[l] = a[l] + a[l ^ m];
      memcpy(a, t2, sizeof a);
    }
    tot = tot + a[0];
  }
  const float inv = 1.0f / tot;
  for (u32 e = 0; e < ne; e++) p[e] = p[e] * inv;
  for (u32 j = 0; j < nk; j++) {
    float bv = -1.0f;
    u32 bi = 0xffffffffu;
    for (u32 e = 0; e < ne; e++) {
      if (p[e] > bv) { bv = p[e]; bi = e; } /* strict >: the lower index keeps a tie */
    }
    if (bi == 0xffffffffu) {
      /* no p left to take (a NaN or +inf logit makes every p NaN): the reference's slot would hold
       * 0xffffffff (undefined input); the path keeps expert 0 with p 0 in such a slot, and so does this */
      ids[j] = 0;
      wt[j] = 0.0f;
      continue;
    }
    ids[j] = bi;
    wt[j] = bv;
    p[bi] = -2.0f;
  }
  mo_renorm(wt, nk);
  *sgo = mo_sigmoid(sg);
  free(p);
}

/* llb_mx_group (host/llb_pf.cuh:774-817): slot i = t * nk + j; off[e] = #{slots with id < e},
 * off[ne] = n; an expert's slots in ascending slot order: xmap[pos] = token, inv[slot] = pos */
void mo_group(const u32* ids, u32 n, u32 nk, u32 ne, u32* off, u32* xmap, u32* inv) {
  u32* cnt = (u32*)calloc((size_t)ne + 1, 4);
  for (u32 i = 0; i < n; i++) cnt[ids[i]]++;
  u32 a = 0;
  for (u32 e = 0; e < ne; e++) { off[e] = a; a += cnt[e]; cnt[e] = off[e]; }
  off[ne] = n;
  for (u32 i = 0; i < n; i++) {
    u32 pos = cnt[ids[i]]++;
    xmap[pos] = i / nk;
    inv[i] = pos;
  }
  free(cnt);
}

/* ------------------------------------------------------------------ the layer (exact) */

static int layer_ok(const mo_layer* L) {
  if (!L->dm || !L->ne || !L->nk || L->nk > L->ne || L->nk > 64 || !L->ef) return 0;
  if (!mo_row_bytes(L->fg, L->dm) || !mo_row_bytes(L->fu, L->dm) || !mo_row_bytes(L->fd, L->ef)) return 0;
  if (L->fg == MO_F32 || L->fu == MO_F32 || L->fd == MO_F32) return 0;
  if (L->dm % 256 || L->ef % 256) return 0;
  if (L->sf) {
    if (L->sf % 256 || !L->shgate || !L->SG || !L->SU || !L->SD) return 0;
    if (L->fsg == MO_Q8_0 || L->fsu == MO_Q8_0 || L->fsd == MO_Q8_0) return 0;
    if (!mo_row_bytes(L->fsg, L->dm) || !mo_row_bytes(L->fsu, L->dm) || !mo_row_bytes(L->fsd, L->sf)) return 0;
  }
  return 1;
}

/* act [nk][ef] of one token (llb_moe_gu, tools/payload-moeany.patch:504-525) */
static void token_act(const mo_layer* L, const float* h2, const u32* ids, float* act, int nt) {
  const u64 rbg = mo_row_bytes(L->fg, L->dm), rbu = mo_row_bytes(L->fu, L->dm);
  (void)nt;
#pragma omp parallel for num_threads(nt) if (nt > 1) schedule(static)
  for (long long q = 0; q < (long long)L->nk * L->ef; q++) {
    u32 j = (u32)(q / L->ef), r = (u32)(q % L->ef);
    u64 e = ids[j];
    float g = mo_dot_stride(L->fg, L->G + (e * L->ef + r) * rbg, L->dm, h2);
    float u = mo_dot_stride(L->fu, L->U + (e * L->ef + r) * rbu, L->dm, h2);
    act[q] = mo_silu_mul(g, u);
  }
}

int mo_moe_exact_act(const mo_layer* L, u32 T, const float* h2, const u32* ids, float* act) {
  if (!layer_ok(L)) return -1;
  for (u32 t = 0; t < T; t++)
    token_act(L, h2 + (size_t)t * L->dm, ids + (size_t)t * L->nk, act + (size_t)t * L->nk * L->ef, 1);
  return 0;
}

int mo_moe_exact(const mo_layer* L, u32 T, const float* h2, const float* x1, float* y, u32* ids, float* wt,
                 float* sgo, int nt) {
  if (!layer_ok(L)) return -1;
  const u32 dm = L->dm, ne = L->ne, nk = L->nk, ef = L->ef, sf = L->sf;
  const u64 rbd = mo_row_bytes(L->fd, ef);
  float* lg = (float*)malloc((size_t)ne * 4);
  float* act = (float*)malloc((size_t)nk * ef * 4);
  float* sa = (float*)malloc((size_t)(sf ? sf : 1) * 4);
  (void)nt;
  for (u32 t = 0; t < T; t++) {
    const float* h = h2 + (size_t)t * dm;
    u32* id = ids + (size_t)t * nk;
    float* w = wt + (size_t)t * nk;
    float sg;
    mo_router(L, h, lg, &sg);
    mo_topk(lg, ne, nk, sg, id, w, &sgo[t]);
    if (sf) {
      const u64 rbsg = mo_row_bytes(L->fsg, dm), rbsu = mo_row_bytes(L->fsu, dm);
#pragma omp parallel for num_threads(nt) if (nt > 1) schedule(static)
      for (long long i = 0; i < (long long)sf; i++) {
        float g = mo_gemv_row(L->fsg, L->SG + (u64)i * rbsg, dm, h);
        float u = mo_gemv_row(L->fsu, L->SU + (u64)i * rbsu, dm, h);
        sa[i] = mo_silu_mul(g, u);
      }
    }
    token_act(L, h, id, act, nt);
    const u64 rbs = sf ? mo_row_bytes(L->fsd, sf) : 0;
    const float so = sgo[t];
#pragma omp parallel for num_threads(nt) if (nt > 1) schedule(static)
    for (long long r = 0; r < (long long)dm; r++) {
      /* llb_moe_dn (tools/payload-moeany.patch:543-594): the routed down dots, hv the shared down row
       * (llb_kgemv's order for it), then the combine */
      float v[64];
      for (u32 j = 0; j < nk; j++)
        v[j] = mo_dot_stride(L->fd, L->D + ((u64)id[j] * dm + (u64)r) * rbd, ef, act + (size_t)j * ef);
      const float res = x1 ? x1[(size_t)t * dm + r] : 0.0f;
      const float hv = sf ? mo_gemv_row(L->fsd, L->SD + (u64)r * rbs, sf, sa) : 0.0f;
      y[(size_t)t * dm + r] = mo_combine(v, w, nk, sf != 0, hv, so, res);
    }
  }
  free(lg); free(act); free(sa);
  return 0;
}

/* ------------------------------------------------------------------ q8 tier */

/* pf_q8x (tools/pf27/pfmm.cuh:39-54) / ref_q8x (tools/q4dp/q4dp_ref.h:18-30) */
void mo_q8_1(const float* x, u32 n, int8_t* q, float* d, float* s) {
  for (u32 b = 0; b < n / 32; b++) {
    /* the block's sum in pf_q8x's warp order: lane l adds lane l ^ m's value, m = 16, 8, 4, 2, 1;
     * lane 0's total is stored */
    float a = 0.0f, v[32];
    for (u32 i = 0; i < 32; i++) { a = fmaxf(a, fabsf(x[32 * b + i])); v[i] = x[32 * b + i]; }
    for (u32 m = 16; m > 0; m >>= 1) {
      float t[32];
      for (u32 l = 0; l < 32; l++) t[l] = v[l] + v[l ^ m];
      memcpy(v, t, sizeof v);
    }
    const float dd = a / 127.0f;
    for (u32 i = 0; i < 32; i++)
      q[32 * b + i] = a == 0.0f ? 0 : (int8_t)clampi((int)roundf(x[32 * b + i] / dd), -127, 127);
    d[b] = dd;
    s[b] = v[0];
  }
}

/* mx_blk / mx_dot (host/llb_pf.cuh:468-527): a 32-block's integer dot scaled by the weight's
 * scale and x's d, minus dmin * m * s for Q4_K / Q5_K; the blocks summed in order */
float mo_dot_q8(u32 fm, const u8* row, u32 cols, const int8_t* q, const float* d, const float* s) {
  float acc = 0.0f;
  for (u32 b = 0; b < cols / 32; b++) {
    const int8_t* qx = q + 32 * b;
    float v;
    if (fm == MO_Q4_K || fm == MO_Q5_K) {
      const u32 sbb = fm == MO_Q4_K ? 144u : 176u;
      const u32 sb = b >> 3, j = b & 7, hi = j & 1;
      const u8* B = row + (size_t)sb * sbb;
      const u8* qs = B + (fm == MO_Q4_K ? 16 : 48) + 32 * (j >> 1);
      int sc, m, ia = 0;
      scmin((int)j, B + 4, &sc, &m);
      for (u32 i = 0; i < 32; i++) {
        int nib = hi ? qs[i] >> 4 : qs[i] & 15;
        if (fm == MO_Q5_K) nib |= ((B[16 + i] >> j) & 1) << 4;
        ia += nib * qx[i];
      }
      v = h2f(B) * (float)sc * d[b] * (float)ia - h2f(B + 2) * (float)m * s[b];
    } else if (fm == MO_Q6_K) {
      const u32 sb = b >> 3, bb = b & 7, n = bb >> 2, quad = bb & 3;
      const u8* B = row + (size_t)sb * 210;
      const u8* ql = B + 64 * n + 32 * (quad & 1);
      const u8* qh = B + 128 + 32 * n;
      int a0 = 0, a1 = 0;
      for (u32 i = 0; i < 32; i++) {
        int nib = quad >= 2 ? ql[i] >> 4 : ql[i] & 15;
        int c = (nib | (((qh[i] >> (2 * quad)) & 3) << 4)) - 32;
        if (i < 16) a0 += c * qx[i]; else a1 += c * qx[i];
      }
      const int8_t* sc = (const int8_t*)(B + 192 + 8 * n + 2 * quad);
      v = h2f(B + 208) * d[b] * ((float)sc[0] * (float)a0 + (float)sc[1] * (float)a1);
    } else if (fm == MO_Q8_0) {
      const u8* B = row + (size_t)b * 34;
      int ia = 0;
      for (u32 i = 0; i < 32; i++) ia += (int8_t)B[2 + i] * qx[i];
      v = h2f(B) * d[b] * (float)ia;
    } else {
      return NAN;
    }
    acc = acc + v;
  }
  return acc;
}

int mo_moe_q8(const mo_layer* L, u32 T, const float* h2, const float* x1, float* y, u32* ids, float* wt,
              float* sgo, int nt) {
  if (!layer_ok(L)) return -1;
  const u32 dm = L->dm, ne = L->ne, nk = L->nk, ef = L->ef, sf = L->sf;
  const u64 rbg = mo_row_bytes(L->fg, dm), rbu = mo_row_bytes(L->fu, dm), rbd = mo_row_bytes(L->fd, ef);
  const u32 wmax = (dm > ef ? dm : ef) > sf ? (dm > ef ? dm : ef) : sf;
  float* lg = (float*)malloc((size_t)ne * 4);
  int8_t* hq = (int8_t*)malloc(dm);
  float *hd = (float*)malloc(dm / 32 * 4), *hs = (float*)malloc(dm / 32 * 4);
  float* act = (float*)malloc((size_t)nk * ef * 4);
  int8_t* aq = (int8_t*)malloc((size_t)nk * wmax);
  float *ad = (float*)malloc((size_t)nk * wmax / 32 * 4), *as = (float*)malloc((size_t)nk * wmax / 32 * 4);
  float* sa = (float*)malloc((size_t)(sf ? sf : 32) * 4);
  (void)nt;
  for (u32 t = 0; t < T; t++) {
    const float* h = h2 + (size_t)t * dm;
    u32* id = ids + (size_t)t * nk;
    float* w = wt + (size_t)t * nk;
    float sg;
    mo_router(L, h, lg, &sg);
    mo_topk(lg, ne, nk, sg, id, w, &sgo[t]);
    mo_q8_1(h, dm, hq, hd, hs);
#pragma omp parallel for num_threads(nt) if (nt > 1) schedule(static)
    for (long long qi = 0; qi < (long long)nk * ef; qi++) {
      u32 j = (u32)(qi / ef), r = (u32)(qi % ef);
      u64 e = id[j];
      float g = mo_dot_q8(L->fg, L->G + (e * ef + r) * rbg, dm, hq, hd, hs);
      float u = mo_dot_q8(L->fu, L->U + (e * ef + r) * rbu, dm, hq, hd, hs);
      act[qi] = mo_silu_mul(g, u);
    }
    for (u32 j = 0; j < nk; j++)
      mo_q8_1(act + (size_t)j * ef, ef, aq + (size_t)j * ef, ad + (size_t)j * ef / 32, as + (size_t)j * ef / 32);
    if (sf) {
      const u64 rbsg = mo_row_bytes(L->fsg, dm), rbsu = mo_row_bytes(L->fsu, dm);
#pragma omp parallel for num_threads(nt) if (nt > 1) schedule(static)
      for (long long i = 0; i < (long long)sf; i++) {
        float g = mo_dot_q8(L->fsg, L->SG + (u64)i * rbsg, dm, hq, hd, hs);
        float u = mo_dot_q8(L->fsu, L->SU + (u64)i * rbsu, dm, hq, hd, hs);
        sa[i] = mo_silu_mul(g, u);
      }
    }
    float *sd = (float*)malloc((size_t)(sf ? sf : 32) / 32 * 4), *ss = (float*)malloc((size_t)(sf ? sf : 32) / 32 * 4);
    int8_t* sqb = (int8_t*)malloc(sf ? sf : 32);
    if (sf) mo_q8_1(sa, sf, sqb, sd, ss);
    const u64 rbs = sf ? mo_row_bytes(L->fsd, sf) : 0;
    const float so = sgo[t];
#pragma omp parallel for num_threads(nt) if (nt > 1) schedule(static)
    for (long long r = 0; r < (long long)dm; r++) {
      float v[64];
      for (u32 j = 0; j < nk; j++)
        v[j] = mo_dot_q8(L->fd, L->D + ((u64)id[j] * dm + (u64)r) * rbd, ef, aq + (size_t)j * ef,
                         ad + (size_t)j * ef / 32, as + (size_t)j * ef / 32);
      const float res = x1 ? x1[(size_t)t * dm + r] : 0.0f;
      const float hv = sf ? mo_dot_q8(L->fsd, L->SD + (u64)r * rbs, sf, sqb, sd, ss) : 0.0f;
      y[(size_t)t * dm + r] = mo_combine(v, w, nk, sf != 0, hv, so, res);
    }
    free(sd); free(ss); free(sqb);
  }
  free(lg); free(hq); free(hd); free(hs); free(act); free(aq); free(ad); free(as); free(sa);
  return 0;
}

/* ------------------------------------------------------------------ float64 recompute */

/* reports/metal-catchup/tools/mx_ref.py:44-57: logits, softmax, renormalised weights, experts and
 * the sigmoid-gated shared expert, all in float64 from the dequantized weights (no residual).
 * ids: the routing to evaluate (the exact tier's), so only the products' rounding is measured. */
int mo_moe_f64(const mo_layer* L, u32 T, const float* h2, const u32* ids, double* y64) {
  if (!layer_ok(L)) return -1;
  const u32 dm = L->dm, ne = L->ne, nk = L->nk, ef = L->ef, sf = L->sf;
  const u32 wmax = dm > ef ? dm : ef;
  float* w = (float*)malloc((size_t)(wmax > sf ? wmax : sf) * 4);
  double* lg = (double*)malloc((size_t)ne * 8);
  double* act = (double*)malloc((size_t)(ef > sf ? ef : sf) * 8);
  const u64 rbg = mo_row_bytes(L->fg, dm), rbu = mo_row_bytes(L->fu, dm), rbd = mo_row_bytes(L->fd, ef);
  for (u32 t = 0; t < T; t++) {
    const float* h = h2 + (size_t)t * dm;
    double* y = y64 + (size_t)t * dm;
    double mx = -INFINITY, sum = 0.0;
    for (u32 e = 0; e < ne; e++) {
      double a = 0.0;
      for (u32 c = 0; c < dm; c++) a += (double)L->router[(size_t)e * dm + c] * (double)h[c];
      if (L->router_bias) a += (double)L->router_bias[e];
      lg[e] = a;
      mx = a > mx ? a : mx;
    }
    for (u32 e = 0; e < ne; e++) { lg[e] = exp(lg[e] - mx); sum += lg[e]; }
    double ws = 0.0;
    for (u32 j = 0; j < nk; j++) ws += lg[ids[(size_t)t * nk + j]] / sum;
    ws = ws < 6.103515625e-5 ? 6.103515625e-5 : ws;
    for (u32 r = 0; r < dm; r++) y[r] = 0.0;
    for (u32 j = 0; j < nk; j++) {
      const u64 e = ids[(size_t)t * nk + j];
      const double wj = lg[e] / sum / ws;
      for (u32 r = 0; r < ef; r++) {
        double g = 0.0, u = 0.0;
        mo_deq_row(L->fg, L->G + (e * ef + r) * rbg, dm, w);
        for (u32 c = 0; c < dm; c++) g += (double)w[c] * h[c];
        mo_deq_row(L->fu, L->U + (e * ef + r) * rbu, dm, w);
        for (u32 c = 0; c < dm; c++) u += (double)w[c] * h[c];
        act[r] = g / (1.0 + exp(-g)) * u;
      }
      for (u32 r = 0; r < dm; r++) {
        double v = 0.0;
        mo_deq_row(L->fd, L->D + (e * dm + r) * rbd, ef, w);
        for (u32 c = 0; c < ef; c++) v += (double)w[c] * act[c];
        y[r] += wj * v;
      }
    }
    if (sf) {
      double sgl = 0.0;
      for (u32 c = 0; c < dm; c++) sgl += (double)L->shgate[c] * h[c];
      const double so = 1.0 / (1.0 + exp(-sgl));
      const u64 rbsg = mo_row_bytes(L->fsg, dm), rbsu = mo_row_bytes(L->fsu, dm), rbs = mo_row_bytes(L->fsd, sf);
      for (u32 i = 0; i < sf; i++) {
        double g = 0.0, u = 0.0;
        mo_deq_row(L->fsg, L->SG + (u64)i * rbsg, dm, w);
        for (u32 c = 0; c < dm; c++) g += (double)w[c] * h[c];
        mo_deq_row(L->fsu, L->SU + (u64)i * rbsu, dm, w);
        for (u32 c = 0; c < dm; c++) u += (double)w[c] * h[c];
        act[i] = g / (1.0 + exp(-g)) * u;
      }
      for (u32 r = 0; r < dm; r++) {
        double v = 0.0;
        mo_deq_row(L->fsd, L->SD + (u64)r * rbs, sf, w);
        for (u32 c = 0; c < sf; c++) v += (double)w[c] * act[c];
        y[r] += so * v;
      }
    }
  }
  free(w); free(lg); free(act);
  return 0;
}

/* ---- llb_rmsnorm_add, the step before the router (tools/payload-fuse.patch:106-127, which takes
 * n = 4096 as 1024 threads x 4 leaves; tools/payload-w1024.patch:130-150 and
 * tools/payload-anyshape.patch:300-340 give the other widths 8 leaves a thread, or rms_wide's L, over a
 * tree of 1024 x that many leaves with +0 past n; rms_tree, tools/payload-fuse.patch:76-103, pairs
 * lanes t, t + 1, then t, t + 2, ..., then the warp sums the same way). Every branch is one balanced
 * pairwise tree in column order over a power of two >= n, whose +0 leaves leave the sums of squares
 * unchanged -- so: the tree over the next power of two >= n. Then s = 1 / sqrt(sum / n + eps) (each op
 * rounded once), x1 = x + z, h2 = (x1 s) w. */
static float rn_tree(const float* x, const float* z, u32 lo, u32 len, u32 n) {
  if (len == 1) {
    if (lo >= n) return 0.0f;
    const float v = x[lo] + z[lo];
    return v * v;
  }
  const float a = rn_tree(x, z, lo, len / 2, n);
  const float b = rn_tree(x, z, lo + len / 2, len / 2, n);
  return a + b;
}
float mo_rmsnorm_add(const float* x, const float* z, const float* w, float eps, u32 n, float* x1, float* h2) {
  u32 P = 1;
  while (P < n) P <<= 1;
  const float sum = rn_tree(x, z, 0, P, n);
  const float s = 1.0f / sqrtf(sum / (float)n + eps);
  for (u32 i = 0; i < n; i++) {
    const float v = x[i] + z[i];
    if (x1) x1[i] = v;
    h2[i] = (v * s) * w[i];
  }
  return s;
}
