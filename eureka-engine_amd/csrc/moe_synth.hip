// moe_synth.hip -- synthetic weights and activations generated on the device, so that benchmark
// layers (up to tens of GB of expert stacks) never cross PCIe.
//
// Normals: a splitmix64 finaliser keyed by (seed, stream) hashes the element index; the sum of the
// hash's four 16-bit fields (Irwin-Hall, mean 131070, sd sqrt(4 (2^32 - 1) / 12)) is centred and
// scaled by one f32 multiply. Integer work and one rounding, so the host generator used by the
// tests produces the same floats.
// Quantizers: Q8_0 ggml's closed form (d = amax / 127 as f16, q = round(x / d)); Q4_K / Q5_K
// min-max per 32 values with 6-bit scale / min codes against the super-block maxima; Q6_K max-abs
// per 16 values with int8 scale codes. The reference quantizes with llama.cpp's routines, which
// are not part of it; these define the bytes both sides read.
#include "moe_dev.h"

DEV u64 mix64(u64 z) {
  z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27; z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}
DEV float gauss(u64 key, u64 i, float k) {
  const u64 h = mix64(key + 0x9E3779B97F4A7C15ull * (i + 1u));
  const u32 s = (u32)(h & 0xffffu) + (u32)((h >> 16) & 0xffffu) + (u32)((h >> 32) & 0xffffu) + (u32)(h >> 48);
  return ((float)s - 131070.0f) * k;
}
static u64 host_key(u64 seed, u64 stream) {
  u64 z = seed + 0x9E3779B97F4A7C15ull * (stream + 1u);
  z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27; z *= 0x94D049BB133111EBull;
  z ^= z >> 31;
  return z;
}

DEV u32 f32_to_f16(float f) {
  const u32 x = __float_as_uint(f), s = (x >> 16) & 0x8000u, e = (x >> 23) & 255u, m = x & 0x7fffffu;
  if (e == 255u) return s | 0x7c00u | (m ? 0x200u | (m >> 13) : 0u);
  const int ee = (int)e - 127 + 15;
  if (ee >= 31) return s | 0x7c00u;
  if (ee <= 0) {
    if (ee < -10) return s;
    const u32 mm = m | 0x800000u, sh = (u32)(14 - ee);
    u32 hm = mm >> sh;
    const u32 rem = mm & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (hm & 1u))) hm += 1u;
    return s | hm;
  }
  const u32 hm = m >> 13, rem = m & 0x1fffu;
  u32 r = s | ((u32)ee << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) r += 1u;
  return r;
}
DEV int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

__global__ void __launch_bounds__(256) k_gauss(u64 key, u64 i0, u64 n, float k, float* __restrict__ out) {
  const u64 i = (u64)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = gauss(key, i0 + i, k);
}

// one thread a block: Q8_0 32 values, K-quants 256 values; element (r, c) is gauss(r cols + c)
template <u32 F>
__global__ void __launch_bounds__(64) k_gen(u64 key, float k, u64 r0, u64 nr, u32 cols, u8* __restrict__ out) {
  const u32 bv = F == FM_Q8_0 ? 32u : 256u, bb = F == FM_Q8_0 ? 34u : F == FM_Q4_K ? 144u : F == FM_Q5_K ? 176u : 210u;
  const u64 nbr = cols / bv, i = (u64)blockIdx.x * 64 + threadIdx.x;
  if (i >= nr * nbr) return;
  const u64 r = i / nbr, b = i % nbr;
  const u64 base = (r0 + r) * cols + b * bv;
  u8* B = out + r * (nbr * bb) + b * bb;
  if (F == FM_Q8_0) {
    float x[32], amax = 0.0f;
    for (int j = 0; j < 32; j++) { x[j] = gauss(key, base + j, k); float a = fabsf(x[j]); amax = a > amax ? a : amax; }
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const u32 h = f32_to_f16(d);
    B[0] = (u8)h; B[1] = (u8)(h >> 8);
    for (int j = 0; j < 32; j++) B[2 + j] = (u8)(signed char)clampi((int)roundf(x[j] * id), -127, 127);
  } else if (F == FM_Q4_K || F == FM_Q5_K) {
    const bool five = F == FM_Q5_K;
    const float lv = five ? 31.0f : 15.0f;
    const int qmax = five ? 31 : 15;
    float scale[8], mn[8], maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 8; j++) {
      float lo = 0.0f, hi = gauss(key, base + 32 * j, k);
      for (int q = 0; q < 32; q++) {
        const float v = gauss(key, base + 32 * j + q, k);
        lo = v < lo ? v : lo;
        hi = v > hi ? v : hi;
      }
      scale[j] = (hi - lo) / lv;
      mn[j] = -lo;
      maxs = scale[j] > maxs ? scale[j] : maxs;
      maxm = mn[j] > maxm ? mn[j] : maxm;
    }
    const u32 hd = f32_to_f16(maxs / 63.0f), hm = f32_to_f16(maxm / 63.0f);
    const float dd = f16v(hd), dmd = f16v(hm);
    int sc[8], m[8];
    for (int j = 0; j < 8; j++) {
      sc[j] = dd > 0.0f ? clampi((int)roundf(scale[j] / dd), 0, 63) : 0;
      m[j] = dmd > 0.0f ? clampi((int)roundf(mn[j] / dmd), 0, 63) : 0;
    }
    for (u32 q = 0; q < bb; q++) B[q] = 0;
    B[0] = (u8)hd; B[1] = (u8)(hd >> 8); B[2] = (u8)hm; B[3] = (u8)(hm >> 8);
    for (int j = 0; j < 4; j++) {
      B[4 + j] = (u8)(sc[j] | ((sc[j + 4] >> 4) << 6));
      B[8 + j] = (u8)(m[j] | ((m[j + 4] >> 4) << 6));
      B[12 + j] = (u8)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    u8* qh = B + 16;
    u8* qs = B + (five ? 48 : 16);
    for (int j = 0; j < 8; j++) {
      const float d1 = dd * (float)sc[j], m1 = dmd * (float)m[j];
      const int g = j >> 1, hi = j & 1;
      for (int q = 0; q < 32; q++) {
        const float v = gauss(key, base + 32 * j + q, k);
        const int c = d1 > 0.0f ? clampi((int)roundf((v + m1) / d1), 0, qmax) : 0;
        qs[32 * g + q] |= (u8)((c & 15) << (4 * hi));
        if (five) qh[q] |= (u8)(((c >> 4) & 1) << (2 * g + hi));
      }
    }
  } else {  // Q6_K
    float scale[16], maxs = 0.0f;
    for (int j = 0; j < 16; j++) {
      float a = 0.0f;
      for (int q = 0; q < 16; q++) { const float v = fabsf(gauss(key, base + 16 * j + q, k)); a = v > a ? v : a; }
      scale[j] = a / 31.0f;
      maxs = scale[j] > maxs ? scale[j] : maxs;
    }
    const u32 hd = f32_to_f16(maxs / 127.0f);
    const float dd = f16v(hd);
    for (u32 q = 0; q < 210; q++) B[q] = 0;
    for (int j = 0; j < 16; j++) {
      const int sc = dd > 0.0f ? clampi((int)roundf(scale[j] / dd), 0, 127) : 0;
      B[192 + j] = (u8)(signed char)sc;
      const float ds = dd * (float)sc;
      for (int q = 0; q < 16; q++) {
        const int c = 16 * j + q;
        const int v = ds > 0.0f ? clampi((int)roundf(gauss(key, base + c, k) / ds), -32, 31) : 0;
        const u32 u = (u32)(v + 32);
        const int n = c >> 7, rr = c & 127, quad = rr >> 5, l = rr & 31;
        B[64 * n + 32 * (quad & 1) + l] |= (u8)((u & 15) << (quad >= 2 ? 4 : 0));
        B[128 + 32 * n + l] |= (u8)((u >> 4) << (2 * quad));
      }
    }
    B[208] = (u8)hd; B[209] = (u8)(hd >> 8);
  }
}

int launch_gauss(u64 seed, u64 stream, u64 i0, u64 n, float sigma, float* out, hipStream_t st) {
  const float k = sigma * 2.6428983e-5f;
  hipLaunchKernelGGL(k_gauss, dim3((u32)((n + 255) / 256)), dim3(256), 0, st, host_key(seed, stream), i0, n, k, out);
  return 0;
}

int launch_gen_rows(u32 fm, u64 seed, u64 stream, u64 r0, u64 nr, u32 cols, float sigma, u8* out, hipStream_t st) {
  const float k = sigma * 2.6428983e-5f;
  const u64 key = host_key(seed, stream);
  if (fm == FM_F32) {
    // row-major floats: element (r, c) = gauss((r0 + r) cols + c)
    hipLaunchKernelGGL(k_gauss, dim3((u32)((nr * cols + 255) / 256)), dim3(256), 0, st, key, r0 * cols, nr * cols, k,
                       (float*)out);
    return 0;
  }
  const u32 bv = fm == FM_Q8_0 ? 32u : 256u;
  if (cols % bv) return -1;
  const u64 nb = nr * (cols / bv);
  const dim3 g((u32)((nb + 63) / 64));
#define GEN_L(F) \
  if (fm == F) { hipLaunchKernelGGL((k_gen<F>), g, dim3(64), 0, st, key, k, r0, nr, cols, out); return 0; }
  GEN_L(FM_Q8_0) GEN_L(FM_Q4_K) GEN_L(FM_Q5_K) GEN_L(FM_Q6_K)
#undef GEN_L
  return -1;
}
