/*
 * ORACLE — test infrastructure only. CPU restatement of zerollm's plain-JS reference path, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker. Nothing in zerollm_amd/ links or
 * calls it. Every function cites the reference file:line it restates.
 *
 * Numerics contract (as the reference): JS numbers are f64, storage arrays are Float32Array (every store
 * rounds to f32). Here: every arithmetic step is written in double, every store into a float array rounds
 * to f32, in the reference's evaluation order. Build with -ffp-contract=off so no step is fused.
 *
 * Pinning (see tests/test_oracle.py):
 *  - f16 conversions: known encodings + exhaustive round trip (test/f16.test.js:5-26).
 *  - dequantisers Q5_0/Q4_K/Q5_K/Q6_K: gguf-py golden vectors (test/data/quant-vectors.json).
 *  - Q8_0/Q4_0: closed-form known answers (test/quant.test.js:7-29), round-trip bound.
 *  - unpackScaleMinK4: hand-packed table (test/quant-vectors.test.js:30-40).
 *  - matvec per format: brute force against dequantise-then-dot in f64 over the same int8 activation.
 *  - quantizeAct: closed form (amax maps to +-127, |q*d - x| <= d/2).
 *  - mulberry32: known first outputs computed from the integer recurrence by hand in the test.
 *  - forward: naive whole-sequence f64 oracle (as test/naive-forward.js:45-99) on tiny models.
 *  - sampler: known-answer distributions (test/spec-sampler.test.js:110-141), drawResidual known answers
 *    (test/spec-generate.test.js:243-261).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

/* ------------------------------------------------------------------ f16 (src/util/f16.js:7-70) */

/* f32 -> f16 bits, round-to-nearest-even incl. subnormals (src/util/f16.js:27-50) */
uint16_t orc_f32_to_f16(float xf) {
  uint32_t b; memcpy(&b, &xf, 4);
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

/* f16 bits -> f32 (src/util/f16.js:53-60): sign * mant * 2^-24 or sign * (1 + mant/1024) * 2^(exp-15) */
float orc_f16_to_f32(uint16_t h) {
  double sign = (h & 0x8000) ? -1.0 : 1.0;
  int exp = (h >> 10) & 0x1f;
  int mant = h & 0x3ff;
  if (exp == 0) return (float)(sign * mant * ldexp(1.0, -24));
  if (exp == 0x1f) return mant ? NAN : (float)(sign * INFINITY);
  return (float)(sign * (1.0 + mant / 1024.0) * ldexp(1.0, exp - 15));
}

static float F16_TBL[65536];
static int f16_tbl_ready = 0;
static void f16_tbl_init(void) {
  if (f16_tbl_ready) return;
  for (int i = 0; i < 65536; i++) F16_TBL[i] = orc_f16_to_f32((uint16_t)i);
  f16_tbl_ready = 1;
}
static inline double H(const uint8_t *p) { return (double)F16_TBL[p[0] | (p[1] << 8)]; }

float orc_bf16_to_f32(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ mulberry32 (src/util/rng.js:4-13) */
typedef struct { uint32_t a; } orc_rng;
void orc_rng_seed(orc_rng *r, uint32_t seed) { r->a = seed; }
double orc_rng_next(orc_rng *r) {
  r->a = r->a + 0x6d2b79f5u;
  uint32_t t = r->a;
  t = (t ^ (t >> 15)) * (t | 1u);
  t ^= t + (t ^ (t >> 7)) * (t | 61u);
  return (double)(t ^ (t >> 14)) / 4294967296.0;
}

/* ------------------------------------------------------------------ activation quantisation (src/compute/ref-kernels.js:44-62) */
/* d = amax/127 (f64, stored f32); inv = 1/d (f64, from the unrounded d); q = round-half-away(x*inv); s = sum q */
void orc_quantize_act(const float *x, int n, int8_t *q, float *d, int32_t *s) {
  int nb = n / QK;
  for (int b = 0; b < nb; b++) {
    int o = b * QK;
    double amax = 0;
    for (int i = 0; i < QK; i++) { double a = fabs((double)x[o + i]); if (a > amax) amax = a; }
    double scale = amax / 127.0;
    d[b] = (float)scale;
    double inv = scale != 0.0 ? 1.0 / scale : 0.0;
    int32_t sum = 0;
    for (int i = 0; i < QK; i++) {
      double v = (double)x[o + i] * inv;
      double r = round(v); /* == (v < 0 ? -Math.round(-v) : Math.round(v)) for every finite v */
      q[o + i] = (int8_t)r;
      sum += (int32_t)r;
    }
    if (s) s[b] = sum;
  }
}

/* ------------------------------------------------------------------ row sizes (src/compute/ref-kernels.js:65-77) */
long orc_row_bytes(int type, long cols) {
  switch (type) {
    case T_F32: return cols * 4;
    case T_F16: case T_BF16: return cols * 2;
    case T_Q8_0: return cols / QK * 34;
    case T_Q4_0: return cols / QK * 18;
    case T_Q5_0: return cols / QK * 22;
    case T_Q4_K: return cols / 256 * 144;
    case T_Q5_K: return cols / 256 * 176;
    case T_Q6_K: return cols / 256 * 210;
    default: return -1;
  }
}

/* ------------------------------------------------------------------ unpackScaleMinK4 (src/compute/quant.js:109-118) */
void orc_unpack_scale_min_k4(const uint8_t *q, int *sc, int *mn) {
  for (int j = 0; j < 4; j++) {
    sc[j] = q[j] & 63;
    mn[j] = q[j + 4] & 63;
    sc[j + 4] = (q[j + 8] & 0x0f) | ((q[j] >> 6) << 4);
    mn[j + 4] = (q[j + 8] >> 4) | ((q[j + 4] >> 6) << 4);
  }
}

/* ------------------------------------------------------------------ dequantRow (src/compute/ref-kernels.js:80-120, src/compute/quant.js:33-202) */
int orc_dequant_row(int type, const uint8_t *data, long cols, long row, float *out) {
  f16_tbl_init();
  long rb = orc_row_bytes(type, cols);
  if (rb < 0) return -1;
  const uint8_t *u = data + row * rb;
  switch (type) {
    case T_F32: memcpy(out, u, cols * 4); return 0;
    case T_F16: for (long i = 0; i < cols; i++) out[i] = F16_TBL[u[2 * i] | (u[2 * i + 1] << 8)]; return 0;
    case T_BF16: for (long i = 0; i < cols; i++) out[i] = orc_bf16_to_f32((uint16_t)(u[2 * i] | (u[2 * i + 1] << 8))); return 0;
    case T_Q8_0:
      for (long b = 0; b < cols / QK; b++) {
        const uint8_t *o = u + b * 34; double d = H(o);
        for (int i = 0; i < QK; i++) out[b * QK + i] = (float)(d * (double)(int8_t)o[2 + i]);
      }
      return 0;
    case T_Q4_0:
      for (long b = 0; b < cols / QK; b++) {
        const uint8_t *o = u + b * 18; double d = H(o);
        for (int j = 0; j < 16; j++) {
          int byte = o[2 + j];
          out[b * QK + j] = (float)(d * (double)((byte & 0x0f) - 8));
          out[b * QK + j + 16] = (float)(d * (double)((byte >> 4) - 8));
        }
      }
      return 0;
    case T_Q5_0: /* src/compute/quant.js:121-135 */
      for (long b = 0; b < cols / 32; b++) {
        const uint8_t *o = u + b * 22; double d = H(o);
        uint32_t qh = (uint32_t)o[2] | ((uint32_t)o[3] << 8) | ((uint32_t)o[4] << 16) | ((uint32_t)o[5] << 24);
        for (int j = 0; j < 16; j++) {
          int byte = o[6 + j];
          int lo = (byte & 0x0f) | (int)(((qh >> j) & 1) << 4), hi = (byte >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
          out[b * 32 + j] = (float)(d * (double)(lo - 16));
          out[b * 32 + j + 16] = (float)(d * (double)(hi - 16));
        }
      }
      return 0;
    case T_Q4_K: case T_Q5_K: { /* src/compute/quant.js:138-175: d*sc[s]*v - dmin*mn[s] */
      int five = type == T_Q5_K; int bs = five ? 176 : 144; int qs = five ? 48 : 16;
      for (long b = 0; b < cols / 256; b++) {
        const uint8_t *o = u + b * bs;
        double d = H(o), dmin = H(o + 2);
        int sc[8], mn[8]; orc_unpack_scale_min_k4(o + 4, sc, mn);
        for (int s = 0; s < 8; s++) {
          int chunk = s >> 1, hi = s & 1;
          for (int l = 0; l < 32; l++) {
            int byte = o[qs + chunk * 32 + l];
            int v = hi ? byte >> 4 : byte & 0x0f;
            if (five) v |= ((o[16 + l] >> s) & 1) << 4;
            out[b * 256 + s * 32 + l] = (float)(d * sc[s] * v - dmin * mn[s]);
          }
        }
      }
      return 0;
    }
    case T_Q6_K: /* src/compute/quant.js:178-202 */
      for (long b = 0; b < cols / 256; b++) {
        const uint8_t *o = u + b * 210;
        double d = H(o + 208);
        for (int half = 0; half < 2; half++) {
          const uint8_t *ql = o + 64 * half, *qh = o + 128 + 32 * half;
          const int8_t *sc = (const int8_t *)(o + 192 + 8 * half);
          for (int l = 0; l < 32; l++) {
            int h = qh[l];
            int q1 = ((ql[l] & 0x0f) | (((h >> 0) & 3) << 4)) - 32;
            int q2 = ((ql[l + 32] & 0x0f) | (((h >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
            int g = l >> 4;
            long e = b * 256 + half * 128;
            out[e + l] = (float)(d * sc[g] * q1);
            out[e + l + 32] = (float)(d * sc[g + 2] * q2);
            out[e + l + 64] = (float)(d * sc[g + 4] * q3);
            out[e + l + 96] = (float)(d * sc[g + 6] * q4);
          }
        }
      }
      return 0;
    default: return -1;
  }
}

/* ------------------------------------------------------------------ quantisers (src/compute/quant.js:15-74) */
void orc_quantize_q8_0(const float *x, long n, uint8_t *out) {
  for (long b = 0; b < n / QK; b++) {
    double amax = 0;
    for (int i = 0; i < QK; i++) amax = fmax(amax, fabs((double)x[b * QK + i]));
    double d = amax / 127.0;
    double id = d != 0.0 ? 1.0 / d : 0.0;
    uint8_t *o = out + b * 34;
    uint16_t h = orc_f32_to_f16((float)d);
    o[0] = h & 0xff; o[1] = h >> 8;
    for (int i = 0; i < QK; i++) o[2 + i] = (uint8_t)(int8_t)round((double)x[b * QK + i] * id);
  }
}

void orc_quantize_q4_0(const float *x, long n, uint8_t *out) {
  for (long b = 0; b < n / QK; b++) {
    double amax = 0, max = 0;
    for (int i = 0; i < QK; i++) { double v = x[b * QK + i]; if (fabs(v) > amax) { amax = fabs(v); max = v; } }
    double d = max / -8.0;
    double id = d != 0.0 ? 1.0 / d : 0.0;
    uint8_t *o = out + b * 18;
    uint16_t h = orc_f32_to_f16((float)d);
    o[0] = h & 0xff; o[1] = h >> 8;
    for (int j = 0; j < 16; j++) {
      double lo = fmin(15.0, trunc((double)x[b * QK + j] * id + 8.5));
      double hi = fmin(15.0, trunc((double)x[b * QK + j + 16] * id + 8.5));
      o[2 + j] = (uint8_t)((int)lo | ((int)hi << 4));
    }
  }
}

/* ------------------------------------------------------------------ matvec (src/compute/ref-kernels.js:127-302) */
/* Activation: x (f32, for float weights), q/d/s from orc_quantize_act. y[r] = f32(acc) for r in [r0, r1). */
static void matvec_rows(int type, const uint8_t *u8, long cols, const float *x, const int8_t *xq, const float *xd,
                        const int32_t *xs, float *y, long r0, long r1) {
  long nb = cols / QK;
  switch (type) {
    case T_Q8_0:
      for (long r = r0; r < r1; r++) {
        const uint8_t *o = u8 + r * nb * 34;
        double acc = 0;
        for (long b = 0; b < nb; b++) {
          const int8_t *w = (const int8_t *)(o + 2);
          const int8_t *a = xq + b * QK;
          int32_t s = 0;
          for (int i = 0; i < QK; i += 4) s += w[i] * a[i] + w[i + 1] * a[i + 1] + w[i + 2] * a[i + 2] + w[i + 3] * a[i + 3];
          acc += (double)s * H(o) * (double)xd[b];
          o += 34;
        }
        y[r] = (float)acc;
      }
      return;
    case T_Q4_0:
      for (long r = r0; r < r1; r++) {
        const uint8_t *o = u8 + r * nb * 18;
        double acc = 0;
        for (long b = 0; b < nb; b++) {
          const int8_t *a = xq + b * QK;
          int32_t s = 0;
          for (int j = 0; j < 16; j++) { int byte = o[2 + j]; s += ((byte & 0x0f) - 8) * a[j] + ((byte >> 4) - 8) * a[j + 16]; }
          acc += (double)s * H(o) * (double)xd[b];
          o += 18;
        }
        y[r] = (float)acc;
      }
      return;
    case T_Q5_0:
      for (long r = r0; r < r1; r++) {
        const uint8_t *o = u8 + r * nb * 22;
        double acc = 0;
        for (long b = 0; b < nb; b++) {
          const int8_t *a = xq + b * QK;
          uint32_t qh = (uint32_t)o[2] | ((uint32_t)o[3] << 8) | ((uint32_t)o[4] << 16) | ((uint32_t)o[5] << 24);
          int32_t s = 0;
          for (int j = 0; j < 16; j++) {
            int byte = o[6 + j];
            int lo = (byte & 0x0f) | (int)(((qh >> j) & 1) << 4), hi = (byte >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
            s += (lo - 16) * a[j] + (hi - 16) * a[j + 16];
          }
          acc += (double)s * H(o) * (double)xd[b];
          o += 22;
        }
        y[r] = (float)acc;
      }
      return;
    case T_Q4_K: case T_Q5_K: {
      int five = type == T_Q5_K; int bs = five ? 176 : 144; int qs = five ? 48 : 16;
      long nsb = cols / 256;
      for (long r = r0; r < r1; r++) {
        double acc = 0;
        for (long sb = 0; sb < nsb; sb++) {
          const uint8_t *o = u8 + (r * nsb + sb) * bs;
          double d = H(o), dmin = H(o + 2);
          int sc[8], mn[8]; orc_unpack_scale_min_k4(o + 4, sc, mn);
          for (int c = 0; c < 4; c++) {
            const uint8_t *qo = o + qs + c * 32; long xo = sb * 256 + c * 64;
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
              int byte = qo[l];
              int vlo = byte & 0x0f, vhi = byte >> 4;
              if (five) { int h5 = o[16 + l]; vlo |= ((h5 >> (2 * c)) & 1) << 4; vhi |= ((h5 >> (2 * c + 1)) & 1) << 4; }
              lo += vlo * xq[xo + l];
              hi += vhi * xq[xo + 32 + l];
            }
            long b0 = sb * 8 + 2 * c;
            acc += (double)xd[b0] * (d * sc[2 * c] * (double)lo - dmin * mn[2 * c] * (double)xs[b0]);
            acc += (double)xd[b0 + 1] * (d * sc[2 * c + 1] * (double)hi - dmin * mn[2 * c + 1] * (double)xs[b0 + 1]);
          }
        }
        y[r] = (float)acc;
      }
      return;
    }
    case T_Q6_K: {
      long nsb = cols / 256;
      for (long r = r0; r < r1; r++) {
        double acc = 0;
        for (long sb = 0; sb < nsb; sb++) {
          const uint8_t *o = u8 + (r * nsb + sb) * 210;
          double d = H(o + 208);
          double gsum[16];
          for (int half = 0; half < 2; half++) {
            const uint8_t *ql = o + 64 * half, *qh = o + 128 + 32 * half;
            long e = sb * 256 + half * 128;
            for (int g = 0; g < 2; g++) {
              int32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
              for (int l = g * 16; l < g * 16 + 16; l++) {
                int h = qh[l], lo0 = ql[l], lo1 = ql[l + 32];
                a0 += (((lo0 & 0x0f) | ((h & 3) << 4)) - 32) * xq[e + l];
                a1 += (((lo1 & 0x0f) | (((h >> 2) & 3) << 4)) - 32) * xq[e + l + 32];
                a2 += (((lo0 >> 4) | (((h >> 4) & 3) << 4)) - 32) * xq[e + l + 64];
                a3 += (((lo1 >> 4) | (((h >> 6) & 3) << 4)) - 32) * xq[e + l + 96];
              }
              gsum[half * 8 + g] = a0; gsum[half * 8 + 2 + g] = a1; gsum[half * 8 + 4 + g] = a2; gsum[half * 8 + 6 + g] = a3;
            }
          }
          for (int g = 0; g < 16; g++) {
            double scale = (double)(int8_t)o[192 + g];
            acc += (double)xd[sb * 8 + (g >> 1)] * d * scale * gsum[g];
          }
        }
        y[r] = (float)acc;
      }
      return;
    }
    case T_F32:
      for (long r = r0; r < r1; r++) {
        const float *f = (const float *)(u8) + r * cols;
        double acc = 0;
        for (long i = 0; i < cols; i++) acc += (double)f[i] * (double)x[i];
        y[r] = (float)acc;
      }
      return;
    case T_F16: case T_BF16: {
      float *tmp = (float *)malloc(cols * sizeof(float));
      for (long r = r0; r < r1; r++) {
        orc_dequant_row(type, u8, cols, r, tmp);
        double acc = 0;
        for (long i = 0; i < cols; i++) acc += (double)tmp[i] * (double)x[i];
        y[r] = (float)acc;
      }
      free(tmp);
      return;
    }
  }
}

/* One worker's rows [r0, r1) with the single-thread arithmetic (the CPU baseline's scalar formats). */
void orc_matvec_rows(int type, const uint8_t *data, long cols, const float *x, const int8_t *xq, const float *xd,
                     const int32_t *xs, float *y, long r0, long r1) {
  matvec_rows(type, data, cols, x, xq, xd, xs, y, r0, r1);
}

/* The f16 table every decoder reads; call once before several threads decode. */
void orc_tables_init(void) { f16_tbl_init(); }

/* Row-split across threads like the reference pool (src/compute/layout.js:39-43): each row is computed by one
 * thread with the single-thread arithmetic, so the result does not depend on the thread count. */
static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

int orc_matvec(int type, const uint8_t *data, long rows, long cols, const float *x, const int8_t *xq,
               const float *xd, const int32_t *xs, float *y) {
  f16_tbl_init();
  if (orc_row_bytes(type, cols) < 0) return -1;
#ifdef _OPENMP
  if (g_threads > 1 && rows >= 64) {
    int nt = g_threads;
#pragma omp parallel num_threads(nt)
    {
      int w = omp_get_thread_num(), n = omp_get_num_threads();
      long per = (rows + n - 1) / n; per = (per + 3) & ~3L;
      long r0 = w * per, r1 = r0 + per; if (r1 > rows) r1 = rows;
      if (r0 < r1) matvec_rows(type, data, cols, x, xq, xd, xs, y, r0, r1);
    }
    return 0;
  }
#endif
  matvec_rows(type, data, cols, x, xq, xd, xs, y, 0, rows);
  return 0;
}

/* ------------------------------------------------------------------ rmsnorm / softmax / silu (src/compute/ref-kernels.js:305-322) */
void orc_rmsnorm(float *out, const float *x, const float *w, double eps, int n) {
  double ss = 0;
  for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
  double s = 1.0 / sqrt(ss / n + eps);
  for (int i = 0; i < n; i++) out[i] = (float)((double)x[i] * s * (double)w[i]);
}

void orc_softmax(float *x, int n) {
  double max = -INFINITY;
  for (int i = 0; i < n; i++) if ((double)x[i] > max) max = x[i];
  double sum = 0;
  for (int i = 0; i < n; i++) { double e = exp((double)x[i] - max); x[i] = (float)e; sum += e; }
  double inv = 1.0 / sum;
  for (int i = 0; i < n; i++) x[i] = (float)((double)x[i] * inv);
}

double orc_silu(double z) { return z / (1.0 + exp(-z)); }

/* ------------------------------------------------------------------ RoPE (src/compute/ref-kernels.js:329-363) */
void orc_rope_tables(int nRot, double base, int ctx, const float *freqFactors, float *cosT, float *sinT) {
  int half = nRot / 2;
  for (int i = 0; i < half; i++) {
    double freq = pow(base, (-2.0 * i) / nRot);
    if (freqFactors) freq /= (double)freqFactors[i];
    for (int p = 0; p < ctx; p++) {
      cosT[(long)p * half + i] = (float)cos(p * freq);
      sinT[(long)p * half + i] = (float)sin(p * freq);
    }
  }
}

/* type 0 = 'norm' (adjacent pairs), 1 = 'neox' (i, i + nRot/2) */
void orc_apply_rope(float *v, int nHeads, int headDim, int nRot, int neox, const float *cosT, const float *sinT, int pos) {
  int half = nRot / 2;
  long to = (long)pos * half;
  for (int h = 0; h < nHeads; h++) {
    int o = h * headDim;
    for (int i = 0; i < half; i++) {
      double c = cosT[to + i], s = sinT[to + i];
      int i0 = neox ? o + i : o + 2 * i;
      int i1 = neox ? o + i + half : o + 2 * i + 1;
      double a = v[i0], b = v[i1];
      v[i0] = (float)(a * c - b * s);
      v[i1] = (float)(a * s + b * c);
    }
  }
}

/* ------------------------------------------------------------------ the forward pass (src/model/forward.js:94-158) */
typedef struct { int type; long rows, cols; const uint8_t *data; } orc_w;

typedef struct {
  /* config (src/model/config.js:275-325) */
  int nEmbd, nLayer, nFF, nHead, nHeadKv, headDim, nRot, vocab, neox, ctx, kvF16;
  double eps, ropeBase;
  /* qwen35 hybrid (src/model/config.js:126-156): layer l is recurrent unless (l + 1) % interval == 0; the
   * attention layers project [query | gate] per head */
  int hybrid, interval, convK, dk, dv, nK, nV;
} orc_cfg;

typedef struct {
  const float *attnNorm, *ffnNorm, *qNorm, *kNorm, *bq, *bk, *bv;
  orc_w wq, wk, wv, wo, wgate, wup, wdown;
  /* Gated DeltaNet layer (src/model/forward-qwen35.js:111-132, 186-194) */
  int recurrent;
  orc_w wqkv, wz, walpha, wbeta, wout;
  const float *conv, *dtBias, *ssmA, *ssmNorm;
} orc_layer;

typedef struct {
  orc_cfg c;
  orc_w tokEmbd, output;
  const float *outputNorm;
  orc_layer *layers;
  float *cosT, *sinT;
  float *kcache, *vcache;       /* f32 KV: [layer][pos][kvDim] (src/model/kvcache.js:3-14) */
  uint16_t *kcache16, *vcache16; /* f16 KV (src/compute/worker.js:304-306) */
  int pos;
  float *x, *xb, *q, *k, *v, *att, *attOut, *proj, *gate, *up, *hb, *logits;
  int8_t *aq; float *ad; int32_t *as;
  /* hybrid: KV cache index of each layer (-1: recurrent), recurrent index, the live recurrent state
   * (src/model/recurrent-state.js:8-37: conv [layer][channel][kernel-1], ssm [layer][vHead][dv][dk]) and scratch */
  int *attnIdx, *recIdx, nAttn, nRec;
  long convSize, ssmSize;
  float *conv, *ssm;
  float *qkv, *z, *alpha, *beta, *core, *qfull, *agate;
} orc_model;

orc_model *orc_model_new(const orc_cfg *c, const float *ropeFreqs) {
  f16_tbl_init();
  orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
  m->c = *c;
  m->layers = (orc_layer *)calloc(c->nLayer, sizeof(orc_layer));
  int half = c->nRot / 2;
  m->cosT = (float *)malloc(sizeof(float) * (long)c->ctx * half);
  m->sinT = (float *)malloc(sizeof(float) * (long)c->ctx * half);
  orc_rope_tables(c->nRot, c->ropeBase, c->ctx, ropeFreqs, m->cosT, m->sinT);
  long kvDim = (long)c->nHeadKv * c->headDim;
  m->attnIdx = (int *)calloc(c->nLayer, sizeof(int));
  m->recIdx = (int *)calloc(c->nLayer, sizeof(int));
  for (int l = 0; l < c->nLayer; l++) {
    int rec = c->hybrid && (l + 1) % c->interval != 0;
    m->attnIdx[l] = rec ? -1 : m->nAttn++;
    m->recIdx[l] = rec ? m->nRec++ : -1;
  }
  long kvN = (long)m->nAttn * c->ctx * kvDim;
  if (c->kvF16) { m->kcache16 = (uint16_t *)calloc(kvN, 2); m->vcache16 = (uint16_t *)calloc(kvN, 2); }
  else { m->kcache = (float *)calloc(kvN, 4); m->vcache = (float *)calloc(kvN, 4); }
  long qDim = (long)c->nHead * c->headDim;
  long big = c->nFF > c->nEmbd ? c->nFF : c->nEmbd; if (qDim > big) big = qDim;
  m->x = (float *)calloc(c->nEmbd, 4); m->xb = (float *)calloc(c->nEmbd, 4);
  m->q = (float *)calloc(qDim, 4); m->k = (float *)calloc(kvDim, 4); m->v = (float *)calloc(kvDim, 4);
  m->att = (float *)calloc(c->ctx, 4); m->attOut = (float *)calloc(qDim, 4); m->proj = (float *)calloc(c->nEmbd, 4);
  m->gate = (float *)calloc(c->nFF, 4); m->up = (float *)calloc(c->nFF, 4); m->hb = (float *)calloc(c->nFF, 4);
  m->logits = (float *)calloc(c->vocab, 4);
  if (c->hybrid) {
    long keyDim = (long)c->nK * c->dk, inner = (long)c->nV * c->dv, convDim = 2 * keyDim + inner;
    m->convSize = (long)(c->convK - 1) * convDim;
    m->ssmSize = (long)c->nV * c->dv * c->dk;
    m->conv = (float *)calloc(m->nRec * m->convSize + 1, 4);
    m->ssm = (float *)calloc(m->nRec * m->ssmSize + 1, 4);
    m->qkv = (float *)calloc(convDim, 4); m->z = (float *)calloc(inner, 4);
    m->alpha = (float *)calloc(c->nV, 4); m->beta = (float *)calloc(c->nV, 4); m->core = (float *)calloc(inner, 4);
    m->qfull = (float *)calloc(2 * qDim, 4); m->agate = (float *)calloc(qDim, 4);
    if (inner > big) big = inner;
    if (2 * qDim > big) big = 2 * qDim;
  }
  m->aq = (int8_t *)calloc(big, 1); m->ad = (float *)calloc(big / QK + 1, 4); m->as = (int32_t *)calloc(big / QK + 1, 4);
  return m;
}

void orc_model_set_global(orc_model *m, int type_e, long ve, long de, const uint8_t *embd, int type_o, const uint8_t *out,
                          const float *outNorm) {
  m->tokEmbd = (orc_w){type_e, ve, de, embd};
  m->output = (orc_w){type_o, ve, de, out};
  m->outputNorm = outNorm;
}

void orc_model_set_layer(orc_model *m, int l, const float *attnNorm, const float *ffnNorm, const float *qNorm,
                         const float *kNorm, const float *bq, const float *bk, const float *bv, const int *types,
                         const uint8_t *const *datas) {
  orc_cfg *c = &m->c; orc_layer *L = &m->layers[l];
  long qDim = (long)c->nHead * c->headDim, kvDim = (long)c->nHeadKv * c->headDim;
  L->attnNorm = attnNorm; L->ffnNorm = ffnNorm; L->qNorm = qNorm; L->kNorm = kNorm; L->bq = bq; L->bk = bk; L->bv = bv;
  L->wq = (orc_w){types[0], qDim, c->nEmbd, datas[0]};
  L->wk = (orc_w){types[1], kvDim, c->nEmbd, datas[1]};
  L->wv = (orc_w){types[2], kvDim, c->nEmbd, datas[2]};
  L->wo = (orc_w){types[3], c->nEmbd, qDim, datas[3]};
  L->wgate = (orc_w){types[4], c->nFF, c->nEmbd, datas[4]};
  L->wup = (orc_w){types[5], c->nFF, c->nEmbd, datas[5]};
  L->wdown = (orc_w){types[6], c->nEmbd, c->nFF, datas[6]};
}

/* A qwen35 layer (src/model/forward-qwen35.js:111-132, 186-194). types/datas: recurrent layer [attn_qkv, attn_gate, ssm_alpha,
 * ssm_beta, ssm_out, ffn_gate, ffn_up, ffn_down]; attention layer [attn_q, attn_k, attn_v, attn_output, -, ffn_gate,
 * ffn_up, ffn_down]. ffnNorm is post_attention_norm (the pre-FFN norm). */
void orc_model_set_layer_hybrid(orc_model *m, int l, const float *attnNorm, const float *ffnNorm, const float *qNorm,
                                const float *kNorm, const float *conv, const float *dtBias, const float *ssmA,
                                const float *ssmNorm, const int *types, const uint8_t *const *datas) {
  orc_cfg *c = &m->c; orc_layer *L = &m->layers[l];
  long qDim = (long)c->nHead * c->headDim, kvDim = (long)c->nHeadKv * c->headDim;
  long keyDim = (long)c->nK * c->dk, inner = (long)c->nV * c->dv, convDim = 2 * keyDim + inner;
  L->attnNorm = attnNorm; L->ffnNorm = ffnNorm; L->qNorm = qNorm; L->kNorm = kNorm;
  L->recurrent = m->recIdx[l] >= 0;
  if (L->recurrent) {
    L->wqkv = (orc_w){types[0], convDim, c->nEmbd, datas[0]};
    L->wz = (orc_w){types[1], inner, c->nEmbd, datas[1]};
    L->walpha = (orc_w){types[2], c->nV, c->nEmbd, datas[2]};
    L->wbeta = (orc_w){types[3], c->nV, c->nEmbd, datas[3]};
    L->wout = (orc_w){types[4], c->nEmbd, inner, datas[4]};
    L->conv = conv; L->dtBias = dtBias; L->ssmA = ssmA; L->ssmNorm = ssmNorm;
  } else {
    L->wq = (orc_w){types[0], 2 * qDim, c->nEmbd, datas[0]};
    L->wk = (orc_w){types[1], kvDim, c->nEmbd, datas[1]};
    L->wv = (orc_w){types[2], kvDim, c->nEmbd, datas[2]};
    L->wo = (orc_w){types[3], c->nEmbd, qDim, datas[3]};
  }
  L->wgate = (orc_w){types[5], c->nFF, c->nEmbd, datas[5]};
  L->wup = (orc_w){types[6], c->nFF, c->nEmbd, datas[6]};
  L->wdown = (orc_w){types[7], c->nEmbd, c->nFF, datas[7]};
}

void orc_model_free(orc_model *m) {
  if (!m) return;
  free(m->attnIdx); free(m->recIdx); free(m->conv); free(m->ssm); free(m->qkv); free(m->z); free(m->alpha);
  free(m->beta); free(m->core); free(m->qfull); free(m->agate);
  free(m->layers); free(m->cosT); free(m->sinT); free(m->kcache); free(m->vcache); free(m->kcache16); free(m->vcache16);
  free(m->x); free(m->xb); free(m->q); free(m->k); free(m->v); free(m->att); free(m->attOut); free(m->proj);
  free(m->gate); free(m->up); free(m->hb); free(m->logits); free(m->aq); free(m->ad); free(m->as);
  free(m);
}

int orc_model_pos(orc_model *m) { return m->pos; }
void orc_model_truncate(orc_model *m, int n) { if (n < m->pos) m->pos = n < 0 ? 0 : n; }
/* The live recurrent state arrays (hybrid models): conv then ssm; sizes in floats through the out arguments. */
float *orc_model_conv_state(orc_model *m, long *n) { *n = m->nRec * m->convSize; return m->conv; }
float *orc_model_ssm_state(orc_model *m, long *n) { *n = m->nRec * m->ssmSize; return m->ssm; }
const float *orc_model_logits(orc_model *m) { return m->logits; }

/* matvec with a fresh Act over `in` (new Act(xb) in src/model/forward.js:201) */
static void mv(orc_model *m, const orc_w *w, const float *in, float *y) {
  if (w->type != T_F32 && w->type != T_F16 && w->type != T_BF16) orc_quantize_act(in, (int)w->cols, m->aq, m->ad, m->as);
  orc_matvec(w->type, w->data, w->rows, w->cols, in, m->aq, m->ad, m->as, y);
}

/* ------------------------------------------------------------------ Gated DeltaNet (src/compute/ref-deltanet.js:11-106) */
double orc_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

/* log(1 + e^x), linear above 20 (src/compute/ref-deltanet.js:14) */
double orc_softplus(double x) { return x > 20 ? x : log1p(exp(x)); }

/* convStep (src/compute/ref-deltanet.js:42-55): depthwise causal conv over [state oldest .. newest, x] + SiLU,
 * updating the window; out may alias x. */
void orc_conv_step(float *state, const float *w, const float *x, float *out, int channels, int kernel) {
  int m = kernel - 1;
  for (int c = 0; c < channels; c++) {
    long so = (long)c * m, wo = (long)c * kernel;
    float cur = x[c];
    double acc = 0;
    for (int t = 0; t < m; t++) acc += (double)w[wo + t] * (double)state[so + t];
    acc += (double)w[wo + m] * (double)cur;
    for (int t = 0; t + 1 < m; t++) state[so + t] = state[so + t + 1];
    if (m > 0) state[so + m - 1] = cur;
    out[c] = (float)orc_silu(acc);
  }
}

/* l2normHeads (src/compute/ref-deltanet.js:61-69): v *= scale / sqrt(sum v^2 + eps) per head */
void orc_l2norm_heads(float *v, int nHeads, int dim, double eps, double scale) {
  for (int h = 0; h < nHeads; h++) {
    float *o = v + (long)h * dim;
    double ss = 0;
    for (int i = 0; i < dim; i++) ss += (double)o[i] * (double)o[i];
    double s = scale / sqrt(ss + eps);
    for (int i = 0; i < dim; i++) o[i] = (float)((double)o[i] * s);
  }
}

/* deltaRuleHead (src/compute/ref-deltanet.js:86-96): S <- gExp S; d = beta (v - S^T k); S <- S + k d^T; o = S^T q.
 * S is this head's [dv][dk] block. The decayed value feeds the sum unrounded, as the reference's local does. */
void orc_delta_rule_head(float *S, const float *q, const float *k, const float *v, float *out, int dk, int dv,
                         double gExp, double beta) {
  for (int j = 0; j < dv; j++) {
    float *r = S + (long)j * dk;
    double sk = 0;
    for (int i = 0; i < dk; i++) { double s = (double)r[i] * gExp; r[i] = (float)s; sk += s * (double)k[i]; }
    double d = ((double)v[j] - sk) * beta;
    double o = 0;
    for (int i = 0; i < dk; i++) { double s = (double)r[i] + (double)k[i] * d; r[i] = (float)s; o += s * (double)q[i]; }
    out[j] = (float)o;
  }
}

/* gatedRmsNormHead (src/compute/ref-deltanet.js:102-106): o = o / sqrt(mean o^2 + eps) * w * silu(z) */
void orc_gated_rmsnorm_head(float *o, const float *z, const float *w, int dim, double eps) {
  double ss = 0;
  for (int i = 0; i < dim; i++) ss += (double)o[i] * (double)o[i];
  double s = 1.0 / sqrt(ss / dim + eps);
  for (int i = 0; i < dim; i++) o[i] = (float)((double)o[i] * s * (double)w[i] * orc_silu((double)z[i]));
}

/* softmax attention of every query head over cache slot ai, positions 0..pos (src/model/forward.js:123-140); the
 * weighted sum of V accumulates in f32 (Float32Array) */
static void attend(orc_model *m, int ai, int pos, const float *q, float *attOut) {
  orc_cfg *c = &m->c;
  int hd = c->headDim, group = c->nHead / c->nHeadKv;
  long kvDim = (long)c->nHeadKv * hd, lo = (long)ai * c->ctx * kvDim;
  double scale = 1.0 / sqrt((double)hd);
  float *att = m->att;
  for (int h = 0; h < c->nHead; h++) {
    int kvh = h / group, qo = h * hd;
    for (int t = 0; t <= pos; t++) {
      long ko = lo + t * kvDim + (long)kvh * hd;
      double s = 0;
      if (c->kvF16) for (int i = 0; i < hd; i++) s += (double)q[qo + i] * (double)F16_TBL[m->kcache16[ko + i]];
      else for (int i = 0; i < hd; i++) s += (double)q[qo + i] * (double)m->kcache[ko + i];
      att[t] = (float)(s * scale);
    }
    orc_softmax(att, pos + 1);
    for (int i = 0; i < hd; i++) attOut[qo + i] = 0;
    for (int t = 0; t <= pos; t++) {
      double p = att[t];
      long vo = lo + t * kvDim + (long)kvh * hd;
      if (c->kvF16) for (int i = 0; i < hd; i++) attOut[qo + i] = (float)((double)attOut[qo + i] + p * (double)F16_TBL[m->vcache16[vo + i]]);
      else for (int i = 0; i < hd; i++) attOut[qo + i] = (float)((double)attOut[qo + i] + p * (double)m->vcache[vo + i]);
    }
  }
}

/* append k, v at position pos of cache slot ai (f16 by RNE when the cache is f16) */
static void kv_store(orc_model *m, int ai, int pos, const float *k, const float *v) {
  orc_cfg *c = &m->c;
  long kvDim = (long)c->nHeadKv * c->headDim, o = (long)ai * c->ctx * kvDim + (long)pos * kvDim;
  if (c->kvF16) {
    for (long i = 0; i < kvDim; i++) { m->kcache16[o + i] = orc_f32_to_f16(k[i]); m->vcache16[o + i] = orc_f32_to_f16(v[i]); }
  } else {
    memcpy(m->kcache + o, k, kvDim * 4);
    memcpy(m->vcache + o, v, kvDim * 4);
  }
}

/* matvec of several matrices over one Act of xb (new Act(h) shared by the projections of one input) */
static void mv_shared(orc_model *m, const float *xb, int n, const orc_w *const *ws, float *const *ys) {
  orc_quantize_act(xb, m->c.nEmbd, m->aq, m->ad, m->as);
  for (int i = 0; i < n; i++) orc_matvec(ws[i]->type, ws[i]->data, ws[i]->rows, ws[i]->cols, xb, m->aq, m->ad, m->as, ys[i]);
}

/* ssmLayerStep (src/model/forward-qwen35.js:45-61): Gated DeltaNet layer of one token; value head hv reads key head
 * hv % nK (keyHeadOfValueHead, src/compute/ref-deltanet.js:27-29) */
static void ssm_layer(orc_model *m, orc_layer *L, int ri, const float *xb, float *out) {
  orc_cfg *c = &m->c;
  int dk = c->dk, dv = c->dv, nK = c->nK, nV = c->nV;
  long keyDim = (long)nK * dk, convDim = 2 * keyDim + (long)nV * dv;
  const orc_w *ws[4] = {&L->wqkv, &L->wz, &L->wbeta, &L->walpha};
  float *ys[4] = {m->qkv, m->z, m->beta, m->alpha};
  mv_shared(m, xb, 4, ws, ys);
  orc_conv_step(m->conv + ri * m->convSize, L->conv, m->qkv, m->qkv, (int)convDim, c->convK);
  orc_l2norm_heads(m->qkv, nK, dk, c->eps, 1.0 / sqrt((double)dk));
  orc_l2norm_heads(m->qkv + keyDim, nK, dk, c->eps, 1.0);
  float *S = m->ssm + ri * m->ssmSize;
  for (int hv = 0; hv < nV; hv++) {
    int kh = hv % nK;
    double beta = orc_sigmoid((double)m->beta[hv]);
    double g = orc_softplus((double)m->alpha[hv] + (double)L->dtBias[hv]) * (double)L->ssmA[hv];
    orc_delta_rule_head(S + (long)hv * dv * dk, m->qkv + (long)kh * dk, m->qkv + keyDim + (long)kh * dk,
                        m->qkv + 2 * keyDim + (long)hv * dv, m->core + (long)hv * dv, dk, dv, exp(g), beta);
    orc_gated_rmsnorm_head(m->core + (long)hv * dv, m->z + (long)hv * dv, L->ssmNorm, dv, c->eps);
  }
  mv(m, &L->wout, m->core, out);
}

/* attnLayerStep (src/model/forward-qwen35.js:71-105): gated attention; attn_q rows per head are [query | gate] */
static void gated_attn_layer(orc_model *m, orc_layer *L, int ai, int pos, const float *xb, float *out) {
  orc_cfg *c = &m->c;
  int D = c->headDim, nHead = c->nHead;
  long qDim = (long)nHead * D;
  const orc_w *ws[3] = {&L->wq, &L->wk, &L->wv};
  float *ys[3] = {m->qfull, m->k, m->v};
  mv_shared(m, xb, 3, ws, ys);
  for (int h = 0; h < nHead; h++) {
    for (int i = 0; i < D; i++) { m->q[h * D + i] = m->qfull[(long)h * 2 * D + i]; m->agate[h * D + i] = m->qfull[(long)h * 2 * D + D + i]; }
    orc_rmsnorm(m->q + h * D, m->q + h * D, L->qNorm, c->eps, D);
  }
  for (int h = 0; h < c->nHeadKv; h++) orc_rmsnorm(m->k + h * D, m->k + h * D, L->kNorm, c->eps, D);
  orc_apply_rope(m->q, nHead, D, c->nRot, 1, m->cosT, m->sinT, pos);
  orc_apply_rope(m->k, c->nHeadKv, D, c->nRot, 1, m->cosT, m->sinT, pos);
  kv_store(m, ai, pos, m->k, m->v);
  attend(m, ai, pos, m->q, m->attOut);
  for (long i = 0; i < qDim; i++) m->attOut[i] = (float)((double)m->attOut[i] * orc_sigmoid((double)m->agate[i]));
  mv(m, &L->wo, m->attOut, out);
}

/* RefModel.forward (src/model/forward.js:184-248) and Qwen35Model.forward (src/model/forward-qwen35.js:305-341);
 * with kvF16 the K/V stores round to f16 as the pool's js-kernel path does (src/compute/worker.js:304-306, 324, 332).
 * Returns 0, or -1 when the context is full, -2 for an out-of-range token. */
int orc_model_forward(orc_model *m, int token, int wantLogits) {
  orc_cfg *c = &m->c;
  int pos = m->pos;
  if (pos >= c->ctx) return -1;
  if (token < 0 || token >= c->vocab) return -2;
  int nEmbd = c->nEmbd, nHead = c->nHead, nHeadKv = c->nHeadKv, hd = c->headDim;
  long kvDim = (long)nHeadKv * hd;
  float *x = m->x, *xb = m->xb, *q = m->q, *k = m->k, *v = m->v, *proj = m->proj;

  orc_dequant_row(m->tokEmbd.type, m->tokEmbd.data, nEmbd, token, x);
  for (int l = 0; l < c->nLayer; l++) {
    orc_layer *L = &m->layers[l];
    orc_rmsnorm(xb, x, L->attnNorm, c->eps, nEmbd);
    if (c->hybrid) {
      if (L->recurrent) ssm_layer(m, L, m->recIdx[l], xb, proj);
      else gated_attn_layer(m, L, m->attnIdx[l], pos, xb, proj);
    } else {
      /* one Act shared by q, k, v (src/model/forward.js:201-202) */
      const orc_w *ws[3] = {&L->wq, &L->wk, &L->wv};
      float *ys[3] = {q, k, v};
      mv_shared(m, xb, 3, ws, ys);
      if (L->bq) for (long i = 0; i < (long)nHead * hd; i++) q[i] = (float)((double)q[i] + (double)L->bq[i]);
      if (L->bk) for (long i = 0; i < kvDim; i++) k[i] = (float)((double)k[i] + (double)L->bk[i]);
      if (L->bv) for (long i = 0; i < kvDim; i++) v[i] = (float)((double)v[i] + (double)L->bv[i]);
      if (L->qNorm) for (int h = 0; h < nHead; h++) orc_rmsnorm(q + h * hd, q + h * hd, L->qNorm, c->eps, hd);
      if (L->kNorm) for (int h = 0; h < nHeadKv; h++) orc_rmsnorm(k + h * hd, k + h * hd, L->kNorm, c->eps, hd);
      orc_apply_rope(q, nHead, hd, c->nRot, c->neox, m->cosT, m->sinT, pos);
      orc_apply_rope(k, nHeadKv, hd, c->nRot, c->neox, m->cosT, m->sinT, pos);
      kv_store(m, m->attnIdx[l], pos, k, v);
      attend(m, m->attnIdx[l], pos, q, m->attOut);
      mv(m, &L->wo, m->attOut, proj);
    }
    for (int i = 0; i < nEmbd; i++) x[i] = (float)((double)x[i] + (double)proj[i]);

    orc_rmsnorm(xb, x, L->ffnNorm, c->eps, nEmbd);
    orc_quantize_act(xb, nEmbd, m->aq, m->ad, m->as);
    orc_matvec(L->wgate.type, L->wgate.data, L->wgate.rows, L->wgate.cols, xb, m->aq, m->ad, m->as, m->gate);
    orc_matvec(L->wup.type, L->wup.data, L->wup.rows, L->wup.cols, xb, m->aq, m->ad, m->as, m->up);
    for (int i = 0; i < c->nFF; i++) m->hb[i] = (float)(orc_silu((double)m->gate[i]) * (double)m->up[i]);
    mv(m, &L->wdown, m->hb, proj);
    for (int i = 0; i < nEmbd; i++) x[i] = (float)((double)x[i] + (double)proj[i]);
  }
  m->pos = pos + 1;
  if (!wantLogits) return 0;
  orc_rmsnorm(xb, x, m->outputNorm, c->eps, nEmbd);
  mv(m, &m->output, xb, m->logits);
  return 0;
}

/* ------------------------------------------------------------------ sampler (src/sampling/sampler.js:21-155) */

/* topKSelect: size-k min-heap over the logits in index order, then sort by value desc, id asc
 * (src/sampling/sampler.js:21-43). ids/vals must hold k entries. Returns the count. */
static void hswap(int32_t *ids, double *vals, int a, int b) { int32_t ti = ids[a]; ids[a] = ids[b]; ids[b] = ti; double tv = vals[a]; vals[a] = vals[b]; vals[b] = tv; }
typedef struct { int32_t id; double v; } orc_cand;
static int cand_cmp(const void *pa, const void *pb) {
  const orc_cand *a = (const orc_cand *)pa, *b = (const orc_cand *)pb;
  if (a->v != b->v) return a->v < b->v ? 1 : -1; /* vals[b] - vals[a] */
  return a->id < b->id ? -1 : (a->id > b->id); /* ids[a] - ids[b] */
}

int orc_topk_select(const float *logits, int n, int k, int32_t *outIds, double *outVals) {
  if (k > n) k = n;
  int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * k); double *vals = (double *)malloc(sizeof(double) * k);
  int size = 0;
  for (int i = 0; i < n; i++) {
    double v = logits[i];
    if (size < k) {
      ids[size] = i; vals[size] = v; size++;
      int j = size - 1;
      while (j > 0) { int p = (j - 1) >> 1; if (vals[j] >= vals[p]) break; hswap(ids, vals, j, p); j = p; }
    } else if (v > vals[0]) {
      ids[0] = i; vals[0] = v;
      int j = 0;
      for (;;) {
        int l = 2 * j + 1, r = l + 1, mm = j;
        if (l < size && vals[l] < vals[mm]) mm = l;
        if (r < size && vals[r] < vals[mm]) mm = r;
        if (mm == j) break;
        hswap(ids, vals, j, mm); j = mm;
      }
    }
  }
  orc_cand *c = (orc_cand *)malloc(sizeof(orc_cand) * (size ? size : 1));
  for (int i = 0; i < size; i++) { c[i].id = ids[i]; c[i].v = vals[i]; }
  qsort(c, size, sizeof(orc_cand), cand_cmp);
  for (int i = 0; i < size; i++) { outIds[i] = c[i].id; outVals[i] = c[i].v; }
  free(ids); free(vals); free(c);
  return size;
}

/* argmax: first maximum (src/model/generate.js:4-8, src/sampling/sampler.js:46-50) */
int orc_argmax(const float *l, int n) {
  int best = 0; double bv = -INFINITY;
  for (int i = 0; i < n; i++) if ((double)l[i] > bv) { bv = l[i]; best = i; }
  return best;
}

typedef struct {
  double temperature, topP, minP, repeatPenalty, presence, frequency;
  int topK, repeatLastN;
} orc_sampler_opts;

/* distribution(logits, history) (src/sampling/sampler.js:94-142). logits are modified in place by the penalties and
 * restored before returning, as the reference does. Returns keep (>= 1); ids/probs hold `keep` entries (capacity
 * must be >= topK, or n when topK is 0 or >= n); *total receives the sum; *greedy is set for temperature <= 0. */
int orc_distribution(const orc_sampler_opts *o, float *logits, int n, const int32_t *hist, int nh, int32_t *ids,
                     double *probs, double *total, int *greedy) {
  int penalized = o->repeatPenalty != 1 || o->presence != 0 || o->frequency != 0;
  int32_t *sv_t = NULL; float *sv_v = NULL; int nsv = 0;
  if (penalized && nh > 0) {
    int start = nh - o->repeatLastN; if (start < 0) start = 0;
    /* distinct tokens in first-occurrence order (Map insertion order) with counts */
    int cap = nh - start;
    int32_t *tok = (int32_t *)malloc(sizeof(int32_t) * (cap ? cap : 1)); int *cnt = (int *)malloc(sizeof(int) * (cap ? cap : 1)); int nd = 0;
    for (int i = start; i < nh; i++) {
      int j = 0; while (j < nd && tok[j] != hist[i]) j++;
      if (j == nd) { tok[nd] = hist[i]; cnt[nd] = 1; nd++; } else cnt[j]++;
    }
    sv_t = (int32_t *)malloc(sizeof(int32_t) * (nd ? nd : 1)); sv_v = (float *)malloc(sizeof(float) * (nd ? nd : 1));
    for (int j = 0; j < nd; j++) {
      int t = tok[j]; double l = logits[t];
      sv_t[nsv] = t; sv_v[nsv] = logits[t]; nsv++;
      double v = o->repeatPenalty != 1 ? (l > 0 ? l / o->repeatPenalty : l * o->repeatPenalty) : l;
      v -= cnt[j] * o->frequency + o->presence;
      logits[t] = (float)v;
    }
    free(tok); free(cnt);
  }
  int keep;
  if (o->temperature <= 0) {
    ids[0] = orc_argmax(logits, n); probs[0] = 1; *total = 1; *greedy = 1; keep = 1;
    for (int i = 0; i < nsv; i++) logits[sv_t[i]] = sv_v[i];
    free(sv_t); free(sv_v);
    return keep;
  }
  *greedy = 0;
  int m;
  double *vals;
  if (o->topK > 0 && o->topK < n) {
    vals = (double *)malloc(sizeof(double) * o->topK);
    m = orc_topk_select(logits, n, o->topK, ids, vals);
  } else {
    orc_cand *c = (orc_cand *)malloc(sizeof(orc_cand) * n);
    for (int i = 0; i < n; i++) { c[i].id = i; c[i].v = logits[i]; }
    qsort(c, n, sizeof(orc_cand), cand_cmp);
    vals = (double *)malloc(sizeof(double) * n);
    for (int i = 0; i < n; i++) { ids[i] = c[i].id; vals[i] = c[i].v; }
    free(c); m = n;
  }
  for (int i = 0; i < nsv; i++) logits[sv_t[i]] = sv_v[i];
  free(sv_t); free(sv_v);
  double max = vals[0], sum = 0;
  for (int i = 0; i < m; i++) { probs[i] = exp((vals[i] - max) / o->temperature); sum += probs[i]; }
  for (int i = 0; i < m; i++) probs[i] /= sum;
  free(vals);
  keep = m;
  if (o->minP > 0) { double thr = o->minP * probs[0]; keep = 1; while (keep < m && probs[keep] >= thr) keep++; }
  if (o->topP < 1) {
    double c = 0; int i = 0;
    while (i < keep) { c += probs[i]; i++; if (c >= o->topP) break; }
    keep = i > 1 ? i : 1;
  }
  double tot = 0;
  for (int i = 0; i < keep; i++) tot += probs[i];
  *total = tot;
  return keep;
}

/* draw (src/sampling/sampler.js:145-151) */
int orc_draw(orc_rng *r, const int32_t *ids, const double *probs, int keep, double total, int greedy) {
  if (greedy) return ids[0];
  double x = orc_rng_next(r) * total;
  for (int i = 0; i < keep; i++) { x -= probs[i]; if (x <= 0) return ids[i]; }
  return ids[keep - 1];
}

/* probOf (src/model/speculative.js:64-67) */
double orc_prob_of(const int32_t *ids, const double *probs, int keep, double total, int id) {
  for (int i = 0; i < keep; i++) if (ids[i] == id) return probs[i] / total;
  return 0;
}

/* drawResidual (src/model/speculative.js:75-87); scratch is an all-zero double[vocab], left all-zero. */
int orc_draw_residual(orc_rng *r, const int32_t *pIds, const double *pProbs, int pKeep, double pTotal, int pGreedy,
                      const int32_t *qIds, const double *qProbs, int qKeep, double qTotal, double *scratch) {
  for (int i = 0; i < qKeep; i++) scratch[qIds[i]] = qProbs[i] / qTotal;
  double *res = (double *)calloc(pKeep ? pKeep : 1, sizeof(double));
  double sum = 0;
  for (int i = 0; i < pKeep; i++) { double v = pProbs[i] / pTotal - scratch[pIds[i]]; if (v > 0) { res[i] = v; sum += v; } }
  for (int i = 0; i < qKeep; i++) scratch[qIds[i]] = 0;
  if (!(sum > 0)) { free(res); return orc_draw(r, pIds, pProbs, pKeep, pTotal, pGreedy); }
  double x = orc_rng_next(r) * sum;
  int last = 0;
  for (int i = 0; i < pKeep; i++) {
    if (res[i] > 0) { last = i; x -= res[i]; if (x <= 0) { int id = pIds[i]; free(res); return id; } }
  }
  int id = pIds[last];
  free(res);
  return id;
}
