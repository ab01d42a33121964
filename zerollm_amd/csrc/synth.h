// Synthetic random-init weights and this library's own block quantisers, one implementation for host and device.
//
// The same functions run on the CPU (GGUF writer for test models) and on the GPU (building a multi-GB model in HBM
// in well under a second), and produce the same bytes on both: the normal deviates come from a counter-based
// generator and a Box-Muller transform whose log and cos are written here with +, -, *, / and sqrt only (no libm
// calls, no contraction), so there is nothing for two math libraries to disagree on.
//
// Quantisers: Q8_0 and Q4_0 follow zerollm's quantizeQ8_0 / quantizeQ4_0 (src/compute/quant.js:15-74). zerollm has no
// K-quant quantiser (its synthetic K-quant models are random raw blocks, tools/random-blocks.js:20-37), so Q4_K, Q5_K,
// Q6_K and Q5_0 use this library's own min/max-search scheme in the ggml block layouts that zerollm dequantises
// (src/compute/quant.js:121-202).
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define ZL_HD __host__ __device__
#else
#define ZL_HD
#endif

#if defined(__clang__)
#define ZL_NOCONTRACT _Pragma("clang fp contract(off)")
#else
#define ZL_NOCONTRACT
#endif

namespace zl_synth {

ZL_HD inline uint64_t dbits(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
ZL_HD inline double bitsd(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }
ZL_HD inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

// splitmix64 finaliser over a counter: uniform in (0, 1), never 0 or 1.
ZL_HD inline double uniform(uint64_t seed, uint64_t n) {
  uint64_t z = seed + (n + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return ((double)(z >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

// ln(u) for u in (0, 1]: u = m * 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh((m-1)/(m+1)) by its series.
ZL_HD inline double ln01(double u) {
  ZL_NOCONTRACT
  uint64_t b = dbits(u);
  int e = (int)((b >> 52) & 0x7ff) - 1023;
  double m = bitsd((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
  if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
  double s = (m - 1.0) / (m + 1.0);
  double s2 = s * s;
  double t = 1.0 / 25.0;
  for (int k = 23; k >= 1; k -= 2) t = t * s2 + 1.0 / (double)k;
  return (double)e * 0.6931471805599453 + 2.0 * s * t;
}

// cos(2*pi*f) for f in [0, 1): quadrant reduction, then Taylor series on |theta| <= pi/4 in nested form.
ZL_HD inline double cos2pi(double f) {
  ZL_NOCONTRACT
  double q = (double)(int64_t)(4.0 * f + 0.5);
  double r = f - 0.25 * q;
  int qi = ((int)q) & 3;
  double th = 6.283185307179586 * r;
  double t2 = th * th;
  double c = 1.0, s = 1.0;
  for (int k = 11; k >= 1; k--) {
    c = 1.0 - t2 / (double)((2 * k - 1) * (2 * k)) * c;
    s = 1.0 - t2 / (double)((2 * k) * (2 * k + 1)) * s;
  }
  s = th * s;
  return qi == 0 ? c : qi == 1 ? -s : qi == 2 ? -c : s;
}

// Standard normal deviate number n of stream `seed` (Box-Muller, cosine branch; two uniforms per deviate).
ZL_HD inline double normal(uint64_t seed, uint64_t n) {
  ZL_NOCONTRACT
  double u1 = uniform(seed, 2 * n), u2 = uniform(seed, 2 * n + 1);
  return __builtin_sqrt(-2.0 * ln01(u1)) * cos2pi(u2);
}

// Weight (r, c) of a tensor whose values are std * normal(seed, r * srcCols + col0 + c): a tensor can take a column
// window of another tensor's values (same seed, wider srcCols).
ZL_HD inline float weight(uint64_t seed, double std, uint64_t srcCols, uint64_t col0, uint64_t r, uint64_t c) {
  ZL_NOCONTRACT
  return (float)(std * normal(seed, r * srcCols + col0 + c));
}

// ---------------------------------------------------------------------------------------------- f16 (RNE)
// Same algorithm as zerollm's f32ToF16 (src/util/f16.js:27-50).
ZL_HD inline uint16_t f32_to_f16(float xf) {
  uint32_t b = fbits(xf);
  uint32_t sign = (b >> 16) & 0x8000u;
  int exp = (int)((b >> 23) & 0xff);
  uint32_t mant = b & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  exp = exp - 127 + 15;
  if (exp >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (exp <= 0) {
    if (exp < -10) return (uint16_t)sign;
    uint32_t m = mant | 0x800000u;
    int shift = 14 - exp;
    uint32_t half = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = sign | ((uint32_t)exp << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
  return (uint16_t)half;
}

ZL_HD inline double f16_to_f64(uint16_t h) {
  ZL_NOCONTRACT
  double sign = (h & 0x8000) ? -1.0 : 1.0;
  int exp = (h >> 10) & 0x1f;
  int mant = h & 0x3ff;
  if (exp == 0) return sign * (double)mant * (1.0 / 16777216.0);
  if (exp == 0x1f) return sign * 65504.0 * 65536.0;  // inf/nan are never produced by the quantisers below
  double p = 1.0;
  for (int i = 15; i < exp; i++) p *= 2.0;
  for (int i = exp; i < 15; i++) p *= 0.5;
  return sign * (1.0 + (double)mant / 1024.0) * p;
}

ZL_HD inline double dmax(double a, double b) { return a > b ? a : b; }
ZL_HD inline double dmin(double a, double b) { return a < b ? a : b; }
ZL_HD inline double dabs(double a) { return a < 0 ? -a : a; }
// round half away from zero (C round; zerollm's roundf, src/compute/quant.js:8)
ZL_HD inline double rnd(double v) {
  ZL_NOCONTRACT
  double a = v < 0 ? -v : v;
  double t = (double)(int64_t)a;
  if (a - t >= 0.5) t += 1.0;  // a - t is exact
  return v < 0 ? -t : t;
}
ZL_HD inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

ZL_HD inline void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)(v & 0xff); p[1] = (uint8_t)(v >> 8); }

// ---------------------------------------------------------------------------------------------- quantisers
// Each quantises one block of floats x into `out` (bytes of one ggml block).

// Q8_0: d = amax/127 (f16), q = round(x / d) with the unrounded d (src/compute/quant.js:15-31).
ZL_HD inline void quant_q8_0(const float *x, uint8_t *out) {
  ZL_NOCONTRACT
  double amax = 0;
  for (int i = 0; i < 32; i++) amax = dmax(amax, dabs((double)x[i]));
  double d = amax / 127.0;
  double id = d != 0.0 ? 1.0 / d : 0.0;
  put16(out, f32_to_f16((float)d));
  for (int i = 0; i < 32; i++) out[2 + i] = (uint8_t)(int8_t)rnd((double)x[i] * id);
}

// Q4_0: the largest-magnitude value maps to -8; q = min(15, trunc(x/d + 8.5)) (src/compute/quant.js:52-74).
ZL_HD inline void quant_q4_0(const float *x, uint8_t *out) {
  ZL_NOCONTRACT
  double amax = 0, mx = 0;
  for (int i = 0; i < 32; i++) { double v = x[i]; if (dabs(v) > amax) { amax = dabs(v); mx = v; } }
  double d = mx / -8.0;
  double id = d != 0.0 ? 1.0 / d : 0.0;
  put16(out, f32_to_f16((float)d));
  for (int j = 0; j < 16; j++) {
    int lo = (int)dmin(15.0, (double)(int64_t)((double)x[j] * id + 8.5));
    int hi = (int)dmin(15.0, (double)(int64_t)((double)x[j + 16] * id + 8.5));
    out[2 + j] = (uint8_t)(clampi(lo, 0, 15) | (clampi(hi, 0, 15) << 4));
  }
}

// Q5_0 (own, same scheme as Q4_0 with 5 bits): the largest-magnitude value maps to -16.
ZL_HD inline void quant_q5_0(const float *x, uint8_t *out) {
  ZL_NOCONTRACT
  double amax = 0, mx = 0;
  for (int i = 0; i < 32; i++) { double v = x[i]; if (dabs(v) > amax) { amax = dabs(v); mx = v; } }
  double d = mx / -16.0;
  double id = d != 0.0 ? 1.0 / d : 0.0;
  put16(out, f32_to_f16((float)d));
  uint32_t qh = 0;
  uint8_t q[32];
  for (int i = 0; i < 32; i++) {
    int v = clampi((int)(int64_t)((double)x[i] * id + 16.5), 0, 31);
    q[i] = (uint8_t)v;
    qh |= (uint32_t)((v >> 4) & 1) << i;
  }
  out[2] = qh & 0xff; out[3] = (qh >> 8) & 0xff; out[4] = (qh >> 16) & 0xff; out[5] = (qh >> 24) & 0xff;
  for (int j = 0; j < 16; j++) out[6 + j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
}

// Smallest f16 >= v (v >= 0), and ceil for non-negative doubles.
ZL_HD inline uint16_t f16_up(double v) {
  uint16_t h = f32_to_f16((float)v);
  if (f16_to_f64(h) < v) h++;
  return h;
}
ZL_HD inline double ceilp(double v) {
  double c = (double)(int64_t)v;
  return c < v ? c + 1.0 : c;
}

// Q4_K / Q5_K (own): per 32-value sub-block the range [lo, hi] with lo <= 0. Super-block f16 dmin and d are rounded up
// and the 6-bit min / scale codes are ceil'd, so that every value of a sub-block lies inside the code range:
// off = dmin*mn >= -lo, step = d*sc >= (hi + off)/qmax; q = round((x + off) / step).
ZL_HD inline void quant_k_affine(const float *x, uint8_t *out, int five) {
  ZL_NOCONTRACT
  const int qmax = five ? 31 : 15;
  double lo[8], hi[8], maxmn = 0;
  for (int s = 0; s < 8; s++) {
    double a = 0, b = -1e300;
    for (int i = 0; i < 32; i++) { double v = x[s * 32 + i]; a = dmin(a, v); b = dmax(b, v); }
    if (b < a) b = a;
    lo[s] = a; hi[s] = b;
    maxmn = dmax(maxmn, -a);
  }
  uint16_t mh = f16_up(maxmn / 63.0);
  double dm = f16_to_f64(mh);
  int sc[8], mn[8];
  double need[8], maxneed = 0;
  for (int s = 0; s < 8; s++) {
    mn[s] = dm > 0 ? clampi((int)ceilp(-lo[s] / dm), 0, 63) : 0;
    need[s] = (hi[s] + dm * (double)mn[s]) / (double)qmax;
    maxneed = dmax(maxneed, need[s]);
  }
  uint16_t dh = f16_up(maxneed / 63.0);
  double d = f16_to_f64(dh);
  for (int s = 0; s < 8; s++) sc[s] = d > 0 ? clampi((int)ceilp(need[s] / d), 0, 63) : 0;
  put16(out, dh);
  put16(out + 2, mh);
  uint8_t *S = out + 4;
  for (int j = 0; j < 4; j++) {
    S[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    S[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
    S[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
  }
  uint8_t q[256];
  for (int s = 0; s < 8; s++) {
    double step = d * (double)sc[s], off = dm * (double)mn[s];
    for (int i = 0; i < 32; i++) q[s * 32 + i] = (uint8_t)(step > 0 ? clampi((int)rnd(((double)x[s * 32 + i] + off) / step), 0, qmax) : 0);
  }
  uint8_t *qs = out + (five ? 48 : 16);
  if (five) {
    uint8_t *qh = out + 16;
    for (int l = 0; l < 32; l++) {
      int h = 0;
      for (int s = 0; s < 8; s++) h |= ((q[s * 32 + l] >> 4) & 1) << s;
      qh[l] = (uint8_t)h;
    }
  }
  for (int c = 0; c < 4; c++)
    for (int l = 0; l < 32; l++) qs[c * 32 + l] = (uint8_t)((q[(2 * c) * 32 + l] & 15) | ((q[(2 * c + 1) * 32 + l] & 15) << 4));
}

// Q6_K (own): per 16-value group a signed scale mapping the largest-magnitude value to -32; the f16 super-block d is
// rounded up and the int8 group codes are rounded away from zero, so |x / (d*sc)| <= 32; q = round(x/(d*sc)) + 32
// clamped to [0, 63] (the negation of the largest value, which would need 64, takes 63).
ZL_HD inline void quant_q6_k(const float *x, uint8_t *out) {
  ZL_NOCONTRACT
  double gs[16], maxabs = 0;
  for (int g = 0; g < 16; g++) {
    double amax = 0, mx = 0;
    for (int i = 0; i < 16; i++) { double v = x[g * 16 + i]; if (dabs(v) > amax) { amax = dabs(v); mx = v; } }
    gs[g] = mx / -32.0;
    maxabs = dmax(maxabs, dabs(gs[g]));
  }
  uint16_t dh = f16_up(maxabs / 127.0);
  double d = f16_to_f64(dh);
  int sc[16];
  for (int g = 0; g < 16; g++) {
    int c = d > 0 ? clampi((int)ceilp(dabs(gs[g]) / d), 0, 127) : 0;
    sc[g] = gs[g] < 0 ? -c : c;
  }
  uint8_t q[256];
  for (int g = 0; g < 16; g++) {
    double step = d * (double)sc[g];
    for (int i = 0; i < 16; i++) q[g * 16 + i] = (uint8_t)(step != 0 ? clampi((int)rnd((double)x[g * 16 + i] / step) + 32, 0, 63) : 32);
  }
  uint8_t *ql = out, *qh = out + 128;
  for (int h = 0; h < 2; h++) {
    for (int l = 0; l < 32; l++) {
      int q0 = q[128 * h + l], q1 = q[128 * h + 32 + l], q2 = q[128 * h + 64 + l], q3 = q[128 * h + 96 + l];
      ql[64 * h + l] = (uint8_t)((q0 & 15) | ((q2 & 15) << 4));
      ql[64 * h + 32 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
      qh[32 * h + l] = (uint8_t)((q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6));
    }
  }
  for (int g = 0; g < 16; g++) out[192 + g] = (uint8_t)(int8_t)sc[g];
  put16(out + 208, dh);
}

// Block geometry: values per block and bytes per block for the types this generator writes (0 = unsupported).
ZL_HD inline int block_values(int type) { return type == 0 ? 1 : (type == 2 || type == 6 || type == 8) ? 32 : (type == 12 || type == 13 || type == 14) ? 256 : 0; }
ZL_HD inline int block_bytes(int type) {
  switch (type) { case 0: return 4; case 2: return 18; case 6: return 22; case 8: return 34; case 12: return 144; case 13: return 176; case 14: return 210; default: return 0; }
}

// Quantise block b of row r of a synthetic tensor into out (one ggml block). type 0 (F32) writes one float.
ZL_HD inline void synth_block(int type, uint64_t seed, double std, uint64_t srcCols, uint64_t col0, uint64_t r,
                              uint64_t b, uint8_t *out) {
  float x[256];
  int n = block_values(type);
  for (int i = 0; i < n; i++) x[i] = weight(seed, std, srcCols, col0, r, b * (uint64_t)n + i);
  switch (type) {
    case 0: memcpy(out, &x[0], 4); break;
    case 2: quant_q4_0(x, out); break;
    case 6: quant_q5_0(x, out); break;
    case 8: quant_q8_0(x, out); break;
    case 12: quant_k_affine(x, out, 0); break;
    case 13: quant_k_affine(x, out, 1); break;
    case 14: quant_q6_k(x, out); break;
  }
}

}  // namespace zl_synth
