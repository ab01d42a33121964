/*
 * CPU baseline — benchmark and test infrastructure only (bench.py's cpu_baseline leg and tests/ use it; nothing in
 * zerollm_amd/ links or calls it). A multi-threaded AVX-512 VNNI restatement of the reference's worker-pool pass
 * (PoolModel.forwardBatch, src/compute/pool.js:145-160, run by every worker in src/compute/worker.js:278-445):
 *  - one SPMD region per pass (OpenMP threads = the pool's workers), barriers between the phases of a layer
 *    (src/compute/worker.js:291, 341, 347, 415, 427, 433);
 *  - every worker owns an even slice of every matrix's rows (splitRows, src/compute/layout.js:39-43; 16-row tiles here
 *    instead of the WASM kernels' 4-row groups) and computes them for all B tokens of the pass from one read of the
 *    weights (mm_<fmt>, src/compute/wasm/kernels.js:127-240, src/compute/wasm/kquant-kernels.js:136-210, 337-504);
 *  - attention is split over (token, KV head) for the cache append and (token, query head) for the scores, softmax and
 *    weighted sum (src/compute/worker.js:296-337).
 * The arithmetic is the oracle's (oracle/zl_oracle.c, the reference's plain-JS path): exact int8 block dots (here
 * vpdpbusd over 16 rows x 4 columns per instruction), the f64 block terms and the per-row f64 chain in the oracle's order
 * (vectorised across rows, one row per f64 lane), f64 attention dots and f32-rounded weighted sums in position order.
 * Every logit equals the oracle's single-token forward bit for bit (tests/test_pool_simd.py). Build with
 * -ffp-contract=off: no step may be fused.
 *
 * Weight layout (repacked at load, per 16-row tile, 64-byte vectors of 16 rows x 4 bytes):
 *  Q8_0  per 32-block: 8 vectors of (w + 128) as u8, then a plane of 16 f16 scales per block;
 *  Q4_K  per 256-superblock: 4 x 8 vectors of the quants' bytes (low nibbles = sub-block 2c, high = 2c+1), then a plane
 *        of d, dmin (16 f16 each) and the unpacked 6-bit scales and mins ([8][16] u8 each);
 *  Q6_K  per 256-superblock: 4 chunks x (8 vectors of two 4-bit halves + 4 vectors of 2-bit high parts), then a plane of
 *        d (16 f16) and the 16 int8 group scales ([16][16]).
 * Other formats run the oracle's scalar rows (orc_matvec_rows) on each worker's slice.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

#define PS_TR 16   /* rows per tile */
#define PS_TG 4    /* tokens per weight-register group */
#define PS_MAXB 16 /* tokens per pass (DEFAULT_LOGITS_BATCH, src/compute/layout.js:49) */

/* the oracle's scalar pieces (oracle/zl_oracle.c) */
void orc_rmsnorm(float *out, const float *x, const float *w, double eps, int n);
void orc_softmax(float *x, int n);
double orc_silu(double z);
void orc_quantize_act(const float *x, int n, int8_t *q, float *d, int32_t *s);
void orc_rope_tables(int nRot, double base, int ctx, const float *freqFactors, float *cosT, float *sinT);
void orc_apply_rope(float *v, int nHeads, int headDim, int nRot, int neox, const float *cosT, const float *sinT, int pos);
uint16_t orc_f32_to_f16(float xf);
int orc_dequant_row(int type, const uint8_t *data, long cols, long row, float *out);
long orc_row_bytes(int type, long cols);
void orc_unpack_scale_min_k4(const uint8_t *q, int *sc, int *mn);
void orc_matvec_rows(int type, const uint8_t *data, long cols, const float *x, const int8_t *xq, const float *xd,
                     const int32_t *xs, float *y, long r0, long r1);
void orc_tables_init(void);

/* ------------------------------------------------------------------ repacked matrices */
typedef struct {
  int type;
  long rows, cols, tiles;
  uint8_t *data;         /* repacked tiles (64-byte aligned), NULL for formats that run the scalar rows */
  long tileBytes, qBytes; /* bytes per tile; bytes of a tile's quant vectors (its scale plane follows) */
  const uint8_t *raw;    /* the GGUF rows (scalar formats) */
} ps_mat;

static int ps_simd_type(int t) { return t == T_Q8_0 || t == T_Q4_K || t == T_Q6_K; }

static void put16(uint8_t *dst, const uint8_t *src) { dst[0] = src[0]; dst[1] = src[1]; }

/* q6 values (0..63) of one Q6_K row-superblock in activation order (src/compute/quant.js Q6_K layout, the oracle's
 * matvec_rows T_Q6_K loop) */
static void q6_decode(const uint8_t *o, uint8_t *q) {
  for (int half = 0; half < 2; half++) {
    const uint8_t *ql = o + 64 * half, *qh = o + 128 + 32 * half;
    int e = half * 128;
    for (int l = 0; l < 32; l++) {
      int h = qh[l];
      q[e + l] = (uint8_t)((ql[l] & 15) | ((h & 3) << 4));
      q[e + l + 32] = (uint8_t)((ql[l + 32] & 15) | (((h >> 2) & 3) << 4));
      q[e + l + 64] = (uint8_t)((ql[l] >> 4) | (((h >> 4) & 3) << 4));
      q[e + l + 96] = (uint8_t)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4));
    }
  }
}

static void repack_tile(ps_mat *w, long T) {
  uint8_t *tq = w->data + T * w->tileBytes, *tp = tq + w->qBytes;
  long nb = w->cols / 32, nsb = w->cols / 256, rb = orc_row_bytes(w->type, w->cols);
  for (int r = 0; r < PS_TR; r++) {
    long R = T * PS_TR + r;
    int live = R < w->rows;
    const uint8_t *row = live ? w->raw + R * rb : NULL;
    if (w->type == T_Q8_0) {
      for (long b = 0; b < nb; b++) {
        const uint8_t *o = live ? row + b * 34 : NULL;
        for (int j = 0; j < 8; j++)
          for (int k = 0; k < 4; k++) tq[b * 512 + j * 64 + r * 4 + k] = live ? (uint8_t)(o[2 + 4 * j + k] ^ 0x80) : 0x80;
        if (live) put16(tp + b * 32 + 2 * r, o); else tp[b * 32 + 2 * r] = tp[b * 32 + 2 * r + 1] = 0;
      }
    } else if (w->type == T_Q4_K) {
      for (long sb = 0; sb < nsb; sb++) {
        uint8_t *m = tp + sb * 320;
        const uint8_t *o = live ? row + sb * 144 : NULL;
        int sc[8] = {0}, mn[8] = {0};
        if (live) orc_unpack_scale_min_k4(o + 4, sc, mn);
        for (int c = 0; c < 4; c++)
          for (int j = 0; j < 8; j++)
            for (int k = 0; k < 4; k++) tq[((sb * 4 + c) * 8 + j) * 64 + r * 4 + k] = live ? o[16 + c * 32 + 4 * j + k] : 0;
        if (live) { put16(m + 2 * r, o); put16(m + 32 + 2 * r, o + 2); } else { m[2 * r] = m[2 * r + 1] = m[32 + 2 * r] = m[33 + 2 * r] = 0; }
        for (int s = 0; s < 8; s++) { m[64 + s * 16 + r] = (uint8_t)sc[s]; m[192 + s * 16 + r] = (uint8_t)mn[s]; }
      }
    } else { /* Q6_K */
      uint8_t q[256];
      for (long sb = 0; sb < nsb; sb++) {
        uint8_t *m = tp + sb * 288;
        const uint8_t *o = live ? row + sb * 210 : NULL;
        if (live) q6_decode(o, q); else memset(q, 0, sizeof q);
        for (int c = 0; c < 4; c++) {
          uint8_t *v = tq + (sb * 4 + c) * 12 * 64;
          for (int j = 0; j < 8; j++)
            for (int k = 0; k < 4; k++)
              v[j * 64 + r * 4 + k] = (uint8_t)((q[c * 64 + 4 * j + k] & 15) | ((q[c * 64 + 32 + 4 * j + k] & 15) << 4));
          for (int i = 0; i < 4; i++)
            for (int k = 0; k < 4; k++) {
              int byte = 0;
              for (int mm = 0; mm < 4; mm++) {
                int s = 4 * i + mm;
                int p = s < 8 ? c * 64 + 4 * s + k : c * 64 + 32 + 4 * (s - 8) + k;
                byte |= (q[p] >> 4) << (2 * mm);
              }
              v[(8 + i) * 64 + r * 4 + k] = (uint8_t)byte;
            }
        }
        if (live) put16(m + 2 * r, o + 208); else m[2 * r] = m[2 * r + 1] = 0;
        for (int g = 0; g < 16; g++) m[32 + g * 16 + r] = live ? o[192 + g] : 0;
      }
    }
  }
}

static void ps_mat_init(ps_mat *w, int type, long rows, long cols, const uint8_t *raw) {
  memset(w, 0, sizeof *w);
  w->type = type; w->rows = rows; w->cols = cols; w->raw = raw;
  w->tiles = (rows + PS_TR - 1) / PS_TR;
  if (!ps_simd_type(type)) return;
  if (type == T_Q8_0) { w->qBytes = cols / 32 * 512; w->tileBytes = w->qBytes + cols / 32 * 32; }
  else if (type == T_Q4_K) { w->qBytes = cols / 256 * 2048; w->tileBytes = w->qBytes + cols / 256 * 320; }
  else { w->qBytes = cols / 256 * 3072; w->tileBytes = w->qBytes + cols / 256 * 288; }
  w->tileBytes = (w->tileBytes + 63) & ~63L;
  w->data = (uint8_t *)aligned_alloc(64, w->tiles * w->tileBytes);
#pragma omp parallel for schedule(static)
  for (long T = 0; T < w->tiles; T++) repack_tile(w, T);
}

static void ps_mat_free(ps_mat *w) { free(w->data); w->data = NULL; }

/* ------------------------------------------------------------------ activations of a pass */
typedef struct {
  const float *x; long ldx;      /* f32 input rows (scalar formats) */
  const int8_t *q; long ldq;     /* quantised rows */
  const float *d; const int32_t *s; long ldd; /* per-32 scale and sum */
  const int32_t *s16; long lds16;             /* per-16 sums (Q6_K's -32 offset) */
} ps_act;

/* ------------------------------------------------------------------ AVX-512 VNNI tile kernels */
#pragma GCC push_options
#pragma GCC target("avx512f,avx512bw,avx512dq,avx512vl,avx512vnni,f16c")

static inline __m512i bc4(const int8_t *p) { int32_t v; memcpy(&v, p, 4); return _mm512_set1_epi32(v); }
static inline __m512d lo_pd(__m512i a) { return _mm512_cvtepi32_pd(_mm512_castsi512_si256(a)); }
static inline __m512d hi_pd(__m512i a) { return _mm512_cvtepi32_pd(_mm512_extracti64x4_epi64(a, 1)); }
static inline void h16_pd(const uint8_t *p, __m512d *lo, __m512d *hi) {
  __m512 f = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)p));
  *lo = _mm512_cvtps_pd(_mm512_castps512_ps256(f));
  *hi = _mm512_cvtps_pd(_mm512_extractf32x8_ps(f, 1));
}
static inline void u8_pd(const uint8_t *p, __m512d *lo, __m512d *hi) {
  __m512i v = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i *)p));
  *lo = lo_pd(v); *hi = hi_pd(v);
}
static inline void i8_pd(const uint8_t *p, __m512d *lo, __m512d *hi) {
  __m512i v = _mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)p));
  *lo = lo_pd(v); *hi = hi_pd(v);
}
static inline void store_rows(float *y, __m512d lo, __m512d hi, int n) {
  __m512 v = _mm512_insertf32x8(_mm512_castps256_ps512(_mm512_cvtpd_ps(lo)), _mm512_cvtpd_ps(hi), 1);
  _mm512_mask_storeu_ps(y, (__mmask16)(n >= 16 ? 0xFFFF : (1u << n) - 1), v);
}

/* y[t][row] for the 16 rows of one tile and NT tokens b0..b0+NT-1. Each row's chain runs over blocks in order:
 * acc += (s * d) * xd (oracle matvec_rows T_Q8_0). */
static inline __attribute__((always_inline)) void q8_tile(const ps_mat *w, long T, const ps_act *a, int b0, const int NT,
                                                         float *y, long ldy, int nrow) {
  const uint8_t *tq = w->data + T * w->tileBytes, *tp = tq + w->qBytes;
  long nb = w->cols / 32;
  __m512d A[PS_TG][2];
  for (int t = 0; t < NT; t++) A[t][0] = A[t][1] = _mm512_setzero_pd();
  for (long b = 0; b < nb; b++) {
    const __m512i *wv = (const __m512i *)(tq + b * 512);
    __m512i acc[PS_TG];
    for (int t = 0; t < NT; t++) acc[t] = _mm512_setzero_si512();
    for (int j = 0; j < 8; j++) {
      __m512i v = _mm512_load_si512(wv + j);
      for (int t = 0; t < NT; t++) acc[t] = _mm512_dpbusd_epi32(acc[t], v, bc4(a->q + (b0 + t) * a->ldq + b * 32 + 4 * j));
    }
    __m512d dl, dh;
    h16_pd(tp + b * 32, &dl, &dh);
    for (int t = 0; t < NT; t++) {
      /* sum (w + 128) x - 128 sum x = sum w x */
      __m512i s = _mm512_sub_epi32(acc[t], _mm512_set1_epi32(128 * a->s[(b0 + t) * a->ldd + b]));
      __m512d xd = _mm512_set1_pd((double)a->d[(b0 + t) * a->ldd + b]);
      A[t][0] = _mm512_add_pd(A[t][0], _mm512_mul_pd(_mm512_mul_pd(lo_pd(s), dl), xd));
      A[t][1] = _mm512_add_pd(A[t][1], _mm512_mul_pd(_mm512_mul_pd(hi_pd(s), dh), xd));
    }
  }
  for (int t = 0; t < NT; t++) store_rows(y + (b0 + t) * ldy, A[t][0], A[t][1], nrow);
}

/* acc += xd * (d*sc*lo - dmin*mn*xs) per 32 sub-block in order (oracle matvec_rows T_Q4_K) */
static inline __attribute__((always_inline)) void q4k_tile(const ps_mat *w, long T, const ps_act *a, int b0, const int NT,
                                                          float *y, long ldy, int nrow) {
  const uint8_t *tq = w->data + T * w->tileBytes, *tp = tq + w->qBytes;
  long nsb = w->cols / 256;
  const __m512i m4 = _mm512_set1_epi8(0x0f);
  __m512d A[PS_TG][2];
  for (int t = 0; t < NT; t++) A[t][0] = A[t][1] = _mm512_setzero_pd();
  for (long sb = 0; sb < nsb; sb++) {
    const uint8_t *m = tp + sb * 320;
    __m512d dl, dh, ml, mh;
    h16_pd(m, &dl, &dh);
    h16_pd(m + 32, &ml, &mh);
    for (int c = 0; c < 4; c++) {
      const __m512i *wv = (const __m512i *)(tq + (sb * 4 + c) * 512);
      __m512i al[PS_TG], ah[PS_TG];
      for (int t = 0; t < NT; t++) al[t] = ah[t] = _mm512_setzero_si512();
      for (int j = 0; j < 8; j++) {
        __m512i v = _mm512_load_si512(wv + j);
        __m512i lo = _mm512_and_si512(v, m4), hi = _mm512_and_si512(_mm512_srli_epi16(v, 4), m4);
        for (int t = 0; t < NT; t++) {
          const int8_t *xq = a->q + (b0 + t) * a->ldq + sb * 256 + c * 64 + 4 * j;
          al[t] = _mm512_dpbusd_epi32(al[t], lo, bc4(xq));
          ah[t] = _mm512_dpbusd_epi32(ah[t], hi, bc4(xq + 32));
        }
      }
      for (int h = 0; h < 2; h++) {
        int sub = 2 * c + h;
        __m512d sl, sh, nl, nh;
        u8_pd(m + 64 + sub * 16, &sl, &sh);
        u8_pd(m + 192 + sub * 16, &nl, &nh);
        __m512d dscl = _mm512_mul_pd(dl, sl), dsch = _mm512_mul_pd(dh, sh);
        __m512d dmnl = _mm512_mul_pd(ml, nl), dmnh = _mm512_mul_pd(mh, nh);
        for (int t = 0; t < NT; t++) {
          __m512i q = h ? ah[t] : al[t];
          long bi = (b0 + t) * a->ldd + sb * 8 + sub;
          __m512d xs = _mm512_set1_pd((double)a->s[bi]), xd = _mm512_set1_pd((double)a->d[bi]);
          __m512d tl = _mm512_sub_pd(_mm512_mul_pd(dscl, lo_pd(q)), _mm512_mul_pd(dmnl, xs));
          __m512d th = _mm512_sub_pd(_mm512_mul_pd(dsch, hi_pd(q)), _mm512_mul_pd(dmnh, xs));
          A[t][0] = _mm512_add_pd(A[t][0], _mm512_mul_pd(xd, tl));
          A[t][1] = _mm512_add_pd(A[t][1], _mm512_mul_pd(xd, th));
        }
      }
    }
  }
  for (int t = 0; t < NT; t++) store_rows(y + (b0 + t) * ldy, A[t][0], A[t][1], nrow);
}

/* acc += xd * d * scale * gsum per 16-group in order (oracle matvec_rows T_Q6_K); xd*d*scale is exact in f64, so the
 * product is formed as xd * (d*scale) */
static inline __attribute__((always_inline)) void q6k_tile(const ps_mat *w, long T, const ps_act *a, int b0, const int NT,
                                                          float *y, long ldy, int nrow) {
  const uint8_t *tq = w->data + T * w->tileBytes, *tp = tq + w->qBytes;
  long nsb = w->cols / 256;
  const __m512i m4 = _mm512_set1_epi8(0x0f), m2 = _mm512_set1_epi8(0x03);
  __m512d A[PS_TG][2];
  for (int t = 0; t < NT; t++) A[t][0] = A[t][1] = _mm512_setzero_pd();
  for (long sb = 0; sb < nsb; sb++) {
    const uint8_t *m = tp + sb * 288;
    __m512d dl, dh;
    h16_pd(m, &dl, &dh);
    for (int c = 0; c < 4; c++) {
      const __m512i *wv = (const __m512i *)(tq + (sb * 4 + c) * 12 * 64);
      __m512i H[4];
      for (int i = 0; i < 4; i++) H[i] = _mm512_load_si512(wv + 8 + i);
      for (int half = 0; half < 2; half++) {
        __m512i acc[2][PS_TG];
        for (int t = 0; t < NT; t++) acc[0][t] = acc[1][t] = _mm512_setzero_si512();
        for (int j = 0; j < 8; j++) {
          __m512i v = _mm512_load_si512(wv + j);
          __m512i nib = half ? _mm512_and_si512(_mm512_srli_epi16(v, 4), m4) : _mm512_and_si512(v, m4);
          int s = half * 8 + j;
          __m512i hb = _mm512_and_si512(_mm512_srl_epi16(H[s >> 2], _mm_cvtsi32_si128(2 * (s & 3))), m2);
          __m512i q6 = _mm512_or_si512(nib, _mm512_slli_epi16(hb, 4));
          for (int t = 0; t < NT; t++)
            acc[j >> 2][t] = _mm512_dpbusd_epi32(acc[j >> 2][t], q6, bc4(a->q + (b0 + t) * a->ldq + sb * 256 + c * 64 + half * 32 + 4 * j));
        }
        for (int gg = 0; gg < 2; gg++) {
          int G = c * 4 + half * 2 + gg;
          __m512d sl, sh;
          i8_pd(m + 32 + G * 16, &sl, &sh);
          __m512d dsl = _mm512_mul_pd(dl, sl), dsh = _mm512_mul_pd(dh, sh);
          for (int t = 0; t < NT; t++) {
            __m512i gs = _mm512_sub_epi32(acc[gg][t], _mm512_set1_epi32(32 * a->s16[(b0 + t) * a->lds16 + sb * 16 + G]));
            __m512d xd = _mm512_set1_pd((double)a->d[(b0 + t) * a->ldd + sb * 8 + (G >> 1)]);
            A[t][0] = _mm512_add_pd(A[t][0], _mm512_mul_pd(_mm512_mul_pd(xd, dsl), lo_pd(gs)));
            A[t][1] = _mm512_add_pd(A[t][1], _mm512_mul_pd(_mm512_mul_pd(xd, dsh), hi_pd(gs)));
          }
        }
      }
    }
  }
  for (int t = 0; t < NT; t++) store_rows(y + (b0 + t) * ldy, A[t][0], A[t][1], nrow);
}

#define PS_DISPATCH(FN)                                                  \
  static void FN##_n(const ps_mat *w, long T, const ps_act *a, int b0, int nt, float *y, long ldy, int nrow) { \
    switch (nt) {                                                        \
      case 1: FN(w, T, a, b0, 1, y, ldy, nrow); break;                   \
      case 2: FN(w, T, a, b0, 2, y, ldy, nrow); break;                   \
      case 3: FN(w, T, a, b0, 3, y, ldy, nrow); break;                   \
      default: FN(w, T, a, b0, 4, y, ldy, nrow); break;                  \
    }                                                                    \
  }
PS_DISPATCH(q8_tile)
PS_DISPATCH(q4k_tile)
PS_DISPATCH(q6k_tile)

/* tiles [t0, t1) of w for B tokens: y[b * ldy + row] */
static void mm_tiles(const ps_mat *w, int B, const ps_act *a, float *y, long ldy, long t0, long t1) {
  for (long T = t0; T < t1; T++) {
    long r0 = T * PS_TR;
    int nrow = (int)(w->rows - r0 < PS_TR ? w->rows - r0 : PS_TR);
    for (int b0 = 0; b0 < B; b0 += PS_TG) {
      int nt = B - b0 < PS_TG ? B - b0 : PS_TG;
      if (w->type == T_Q8_0) q8_tile_n(w, T, a, b0, nt, y + r0, ldy, nrow);
      else if (w->type == T_Q4_K) q4k_tile_n(w, T, a, b0, nt, y + r0, ldy, nrow);
      else q6k_tile_n(w, T, a, b0, nt, y + r0, ldy, nrow);
    }
  }
}

/* scores of one query head over positions 0..npos-1 of a transposed f16 K cache ([hd][ctxPad]): 16 positions per step,
 * each lane the oracle's sequential f64 dot over the head's dimensions */
static void attn_scores_t(const float *q, const uint16_t *kt, long ctxPad, int hd, int npos, double scale, float *att) {
  const __m512d sc = _mm512_set1_pd(scale);
  for (int t = 0; t < npos; t += 16) {
    __m512d a0 = _mm512_setzero_pd(), a1 = _mm512_setzero_pd();
    for (int i = 0; i < hd; i++) {
      __m512d qd = _mm512_set1_pd((double)q[i]), kl, kh;
      h16_pd((const uint8_t *)(kt + i * ctxPad + t), &kl, &kh);
      a0 = _mm512_add_pd(a0, _mm512_mul_pd(qd, kl));
      a1 = _mm512_add_pd(a1, _mm512_mul_pd(qd, kh));
    }
    int n = npos - t < 16 ? npos - t : 16;
    store_rows(att + t, _mm512_mul_pd(a0, sc), _mm512_mul_pd(a1, sc), n);
  }
}

/* out = sum_t p[t] * V[t] over an f16 [ctx][hd] cache, every step rounded to f32 as the oracle's Float32Array output */
static void attn_av_t(const float *p, const uint16_t *vc, int hd, int npos, float *out) {
  for (int i0 = 0; i0 < hd; i0 += 64) {
    int nc = (hd - i0) / 8 < 8 ? (hd - i0) / 8 : 8;
    __m512d acc[8];
    for (int c = 0; c < 8; c++) acc[c] = _mm512_setzero_pd();
    for (int t = 0; t < npos; t++) {
      __m512d pd = _mm512_set1_pd((double)p[t]);
      const uint16_t *v = vc + (long)t * hd + i0;
      for (int c = 0; c < nc; c++) {
        __m512d vv = _mm512_cvtps_pd(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(v + 8 * c))));
        acc[c] = _mm512_cvtps_pd(_mm512_cvtpd_ps(_mm512_add_pd(acc[c], _mm512_mul_pd(pd, vv))));
      }
    }
    for (int c = 0; c < nc; c++) _mm256_storeu_ps(out + i0 + 8 * c, _mm512_cvtpd_ps(acc[c]));
  }
}

#pragma GCC pop_options

/* ------------------------------------------------------------------ the pool model */
typedef struct {
  int nEmbd, nLayer, nFF, nHead, nHeadKv, headDim, nRot, vocab, neox, ctx;
  double eps, ropeBase;
} ps_cfg;

typedef struct {
  const float *attnNorm, *ffnNorm, *qNorm, *kNorm, *bq, *bk, *bv;
  ps_mat wq, wk, wv, wo, wg, wu, wd;
} ps_layer;

typedef struct {
  ps_cfg c;
  int threads;
  long ctxPad, maxDim;
  int embType; const uint8_t *emb;
  ps_mat out; const float *outNorm;
  ps_layer *L;
  float *cosT, *sinT;
  uint16_t *kt, *vc; /* K transposed [layer][kvHead][hd][ctxPad], V [layer][kvHead][ctx][hd] */
  int pos;
  float *x, *xb, *q, *k, *v, *ao, *proj, *gate, *up, *hb, *logits, *scores;
  int8_t *aq; float *ad; int32_t *as, *as16;
} ps_model;

int ps_supported(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
         __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl") &&
         __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("f16c");
}

static void *zalloc(long n) { void *p = aligned_alloc(64, (n + 63) & ~63L); memset(p, 0, (n + 63) & ~63L); return p; }

ps_model *ps_model_new(const ps_cfg *c, const float *ropeFreqs, int threads) {
  if (!ps_supported()) return NULL;
  orc_tables_init();
  ps_model *m = (ps_model *)calloc(1, sizeof(ps_model));
  m->c = *c;
  m->threads = threads < 1 ? 1 : threads;
  m->ctxPad = (c->ctx + 15) & ~15L;
  long qDim = (long)c->nHead * c->headDim, kvDim = (long)c->nHeadKv * c->headDim;
  long big = c->nFF > c->nEmbd ? c->nFF : c->nEmbd;
  if (qDim > big) big = qDim;
  m->maxDim = big;
  m->L = (ps_layer *)calloc(c->nLayer, sizeof(ps_layer));
  int half = c->nRot / 2;
  m->cosT = (float *)malloc(sizeof(float) * (long)c->ctx * half);
  m->sinT = (float *)malloc(sizeof(float) * (long)c->ctx * half);
  orc_rope_tables(c->nRot, c->ropeBase, c->ctx, ropeFreqs, m->cosT, m->sinT);
  m->kt = (uint16_t *)zalloc(2L * c->nLayer * kvDim * m->ctxPad);
  m->vc = (uint16_t *)zalloc(2L * c->nLayer * kvDim * c->ctx);
  long B = PS_MAXB;
  m->x = zalloc(4 * B * c->nEmbd); m->xb = zalloc(4 * B * big); m->q = zalloc(4 * B * qDim);
  m->k = zalloc(4 * B * kvDim); m->v = zalloc(4 * B * kvDim); m->ao = zalloc(4 * B * qDim);
  m->proj = zalloc(4 * B * c->nEmbd); m->gate = zalloc(4 * B * c->nFF); m->up = zalloc(4 * B * c->nFF);
  m->hb = zalloc(4 * B * c->nFF); m->logits = zalloc(4 * B * (long)c->vocab);
  m->scores = zalloc(4L * m->threads * m->ctxPad);
  m->aq = zalloc(B * big); m->ad = zalloc(4 * B * (big / 32)); m->as = zalloc(4 * B * (big / 32));
  m->as16 = zalloc(4 * B * (big / 16));
  return m;
}

void ps_model_set_global(ps_model *m, int typeE, const uint8_t *embd, int typeO, const uint8_t *out, const float *outNorm) {
  m->embType = typeE; m->emb = embd;
  ps_mat_init(&m->out, typeO, m->c.vocab, m->c.nEmbd, out);
  m->outNorm = outNorm;
}

/* types/datas: attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down */
void ps_model_set_layer(ps_model *m, int l, const float *attnNorm, const float *ffnNorm, const float *qNorm,
                        const float *kNorm, const float *bq, const float *bk, const float *bv, const int *types,
                        const uint8_t *const *datas) {
  ps_cfg *c = &m->c; ps_layer *L = &m->L[l];
  long qDim = (long)c->nHead * c->headDim, kvDim = (long)c->nHeadKv * c->headDim;
  L->attnNorm = attnNorm; L->ffnNorm = ffnNorm; L->qNorm = qNorm; L->kNorm = kNorm; L->bq = bq; L->bk = bk; L->bv = bv;
  ps_mat_init(&L->wq, types[0], qDim, c->nEmbd, datas[0]);
  ps_mat_init(&L->wk, types[1], kvDim, c->nEmbd, datas[1]);
  ps_mat_init(&L->wv, types[2], kvDim, c->nEmbd, datas[2]);
  ps_mat_init(&L->wo, types[3], c->nEmbd, qDim, datas[3]);
  ps_mat_init(&L->wg, types[4], c->nFF, c->nEmbd, datas[4]);
  ps_mat_init(&L->wu, types[5], c->nFF, c->nEmbd, datas[5]);
  ps_mat_init(&L->wd, types[6], c->nEmbd, c->nFF, datas[6]);
}

void ps_model_free(ps_model *m) {
  if (!m) return;
  for (int l = 0; l < m->c.nLayer; l++) {
    ps_layer *L = &m->L[l];
    ps_mat_free(&L->wq); ps_mat_free(&L->wk); ps_mat_free(&L->wv); ps_mat_free(&L->wo);
    ps_mat_free(&L->wg); ps_mat_free(&L->wu); ps_mat_free(&L->wd);
  }
  ps_mat_free(&m->out);
  free(m->L); free(m->cosT); free(m->sinT); free(m->kt); free(m->vc);
  free(m->x); free(m->xb); free(m->q); free(m->k); free(m->v); free(m->ao); free(m->proj); free(m->gate); free(m->up);
  free(m->hb); free(m->logits); free(m->scores); free(m->aq); free(m->ad); free(m->as); free(m->as16);
  free(m);
}

int ps_model_pos(ps_model *m) { return m->pos; }
void ps_model_truncate(ps_model *m, int n) { if (n < m->pos) m->pos = n < 0 ? 0 : n; }
const float *ps_model_logits(ps_model *m) { return m->logits; }

/* quantise row b of src (cols values) into the act buffers (the pool's prep(), src/compute/worker.js:288) */
static void prep_row(ps_model *m, const float *src, long ld, int cols, int b) {
  long big = m->maxDim;
  int8_t *q = m->aq + b * big;
  orc_quantize_act(src + b * ld, cols, q, m->ad + b * (big / 32), m->as + b * (big / 32));
  int32_t *s16 = m->as16 + b * (big / 16);
  for (int g = 0; g < cols / 16; g++) {
    int32_t s = 0;
    for (int i = 0; i < 16; i++) s += q[g * 16 + i];
    s16[g] = s;
  }
}

static ps_act act_of(ps_model *m, const float *src, long ld) {
  long big = m->maxDim;
  ps_act a = {src, ld, m->aq, big, m->ad, m->as, big / 32, m->as16, big / 16};
  return a;
}

/* worker w's tile slice of one matrix for B tokens; float / scalar formats run the oracle's rows */
static void mm_part(const ps_mat *W, int B, const ps_act *a, float *y, long ldy, int w, int n) {
  long t0 = W->tiles * w / n, t1 = W->tiles * (w + 1) / n;
  if (t0 >= t1) return;
  if (W->data) { mm_tiles(W, B, a, y, ldy, t0, t1); return; }
  long r0 = t0 * PS_TR, r1 = t1 * PS_TR < W->rows ? t1 * PS_TR : W->rows;
  for (int b = 0; b < B; b++)
    orc_matvec_rows(W->type, W->raw, W->cols, a->x + b * a->ldx, a->q + b * a->ldq, a->d + b * a->ldd,
                    a->s + b * a->ldd, y + b * ldy, r0, r1);
}

static void row_range(const ps_mat *W, int w, int n, long *r0, long *r1) {
  long t0 = W->tiles * w / n, t1 = W->tiles * (w + 1) / n;
  *r0 = t0 * PS_TR;
  *r1 = t1 * PS_TR < W->rows ? t1 * PS_TR : W->rows;
  if (*r0 > *r1) *r0 = *r1;
}

/* One pass over B tokens at positions pos..pos+B-1 (forwardBatch, src/compute/pool.js:145-160). want: 0 no logits,
 * 1 the last token's, 2 every token's (rows b * vocab). Returns 0, -1 context full, -2 token out of range, -3 batch. */
int ps_model_forward(ps_model *m, const int32_t *tokens, int B, int want) {
  ps_cfg *c = &m->c;
  if (B < 1 || B > PS_MAXB) return -3;
  if (m->pos + B > c->ctx) return -1;
  for (int b = 0; b < B; b++) if (tokens[b] < 0 || tokens[b] >= c->vocab) return -2;
  const int nE = c->nEmbd, hd = c->headDim, nH = c->nHead, nKv = c->nHeadKv, group = nH / nKv;
  const long qDim = (long)nH * hd, kvDim = (long)nKv * hd, big = m->maxDim;
  const int pos0 = m->pos;
  const double scale = 1.0 / sqrt((double)hd);
  for (int b = 0; b < B; b++) orc_dequant_row(m->embType, m->emb, nE, tokens[b], m->x + (long)b * nE);

#pragma omp parallel num_threads(m->threads)
  {
    int w = 0, n = 1;
#ifdef _OPENMP
    w = omp_get_thread_num(); n = omp_get_num_threads();
#endif
    float *att = m->scores + (long)w * m->ctxPad;
    for (int l = 0; l < c->nLayer; l++) {
      ps_layer *L = &m->L[l];
      /* P1: norm + quantisation per token, then my rows of q, k, v */
      for (int b = w; b < B; b += n) {
        orc_rmsnorm(m->xb + b * big, m->x + (long)b * nE, L->attnNorm, c->eps, nE);
        prep_row(m, m->xb, big, nE, b);
      }
#pragma omp barrier
      ps_act a = act_of(m, m->xb, big);
      mm_part(&L->wq, B, &a, m->q, qDim, w, n);
      mm_part(&L->wk, B, &a, m->k, kvDim, w, n);
      mm_part(&L->wv, B, &a, m->v, kvDim, w, n);
      long r0, r1;
      if (L->bq) { row_range(&L->wq, w, n, &r0, &r1); for (int b = 0; b < B; b++) for (long i = r0; i < r1; i++) m->q[b * qDim + i] = (float)((double)m->q[b * qDim + i] + (double)L->bq[i]); }
      if (L->bk) { row_range(&L->wk, w, n, &r0, &r1); for (int b = 0; b < B; b++) for (long i = r0; i < r1; i++) m->k[b * kvDim + i] = (float)((double)m->k[b * kvDim + i] + (double)L->bk[i]); }
      if (L->bv) { row_range(&L->wv, w, n, &r0, &r1); for (int b = 0; b < B; b++) for (long i = r0; i < r1; i++) m->v[b * kvDim + i] = (float)((double)m->v[b * kvDim + i] + (double)L->bv[i]); }
#pragma omp barrier
      /* P2a: per (token, KV head): k-norm, RoPE, cache append; the group's query heads: q-norm, RoPE */
      for (int it = w; it < B * nKv; it += n) {
        int b = it / nKv, kh = it % nKv, pos = pos0 + b;
        float *kk = m->k + b * kvDim + (long)kh * hd, *vv = m->v + b * kvDim + (long)kh * hd;
        if (L->kNorm) orc_rmsnorm(kk, kk, L->kNorm, c->eps, hd);
        orc_apply_rope(kk, 1, hd, c->nRot, c->neox, m->cosT, m->sinT, pos);
        uint16_t *kt = m->kt + ((long)l * nKv + kh) * hd * m->ctxPad;
        uint16_t *vc = m->vc + (((long)l * nKv + kh) * c->ctx + pos) * hd;
        for (int i = 0; i < hd; i++) { kt[(long)i * m->ctxPad + pos] = orc_f32_to_f16(kk[i]); vc[i] = orc_f32_to_f16(vv[i]); }
        for (int g = 0; g < group; g++) {
          float *qq = m->q + b * qDim + (long)(kh * group + g) * hd;
          if (L->qNorm) orc_rmsnorm(qq, qq, L->qNorm, c->eps, hd);
          orc_apply_rope(qq, 1, hd, c->nRot, c->neox, m->cosT, m->sinT, pos);
        }
      }
#pragma omp barrier
      /* P2b: per (token, query head): scores, softmax, weighted sum of V */
      for (int it = w; it < B * nH; it += n) {
        int b = it / nH, h = it % nH, kh = h / group, npos = pos0 + b + 1;
        attn_scores_t(m->q + b * qDim + (long)h * hd, m->kt + ((long)l * nKv + kh) * hd * m->ctxPad, m->ctxPad, hd, npos,
                      scale, att);
        orc_softmax(att, npos);
        attn_av_t(att, m->vc + ((long)l * nKv + kh) * c->ctx * hd, hd, npos, m->ao + b * qDim + (long)h * hd);
      }
#pragma omp barrier
      /* P3: output projection and residual for my rows */
      for (int b = w; b < B; b += n) prep_row(m, m->ao, qDim, (int)qDim, b);
#pragma omp barrier
      a = act_of(m, m->ao, qDim);
      mm_part(&L->wo, B, &a, m->proj, nE, w, n);
      row_range(&L->wo, w, n, &r0, &r1);
      for (int b = 0; b < B; b++)
        for (long i = r0; i < r1; i++) m->x[(long)b * nE + i] = (float)((double)m->x[(long)b * nE + i] + (double)m->proj[(long)b * nE + i]);
#pragma omp barrier
      /* P4: FFN norm + quantisation, my rows of gate and up, SwiGLU */
      for (int b = w; b < B; b += n) {
        orc_rmsnorm(m->xb + b * big, m->x + (long)b * nE, L->ffnNorm, c->eps, nE);
        prep_row(m, m->xb, big, nE, b);
      }
#pragma omp barrier
      a = act_of(m, m->xb, big);
      mm_part(&L->wg, B, &a, m->gate, c->nFF, w, n);
      mm_part(&L->wu, B, &a, m->up, c->nFF, w, n);
      row_range(&L->wg, w, n, &r0, &r1);
      for (int b = 0; b < B; b++)
        for (long i = r0; i < r1; i++) {
          long o = (long)b * c->nFF + i;
          m->hb[o] = (float)(orc_silu((double)m->gate[o]) * (double)m->up[o]);
        }
#pragma omp barrier
      /* P5: down projection and residual for my rows */
      for (int b = w; b < B; b += n) prep_row(m, m->hb, c->nFF, c->nFF, b);
#pragma omp barrier
      a = act_of(m, m->hb, c->nFF);
      mm_part(&L->wd, B, &a, m->proj, nE, w, n);
      row_range(&L->wd, w, n, &r0, &r1);
      for (int b = 0; b < B; b++)
        for (long i = r0; i < r1; i++) m->x[(long)b * nE + i] = (float)((double)m->x[(long)b * nE + i] + (double)m->proj[(long)b * nE + i]);
#pragma omp barrier
    }
    if (want) {
      int first = want == 2 ? 0 : B - 1, nb = B - first;
      for (int b = first + w; b < B; b += n) {
        orc_rmsnorm(m->xb + (b - first) * big, m->x + (long)b * nE, m->outNorm, c->eps, nE);
        prep_row(m, m->xb, big, nE, b - first);
      }
#pragma omp barrier
      ps_act a = act_of(m, m->xb, big);
      mm_part(&m->out, nb, &a, m->logits, c->vocab, w, n);
    }
  }
  m->pos = pos0 + B;
  return 0;
}

/* y[b][r] = one matrix over B activation rows (parity tests of the tile kernels against the oracle's rows) */
int ps_matmul(int type, const uint8_t *raw, long rows, long cols, int B, const float *x, float *y, int threads) {
  if (!ps_supported() || B < 1 || B > PS_MAXB || (cols % 256 && type != T_Q8_0)) return -1;
  orc_tables_init();
  ps_mat W;
  ps_mat_init(&W, type, rows, cols, raw);
  long big = cols;
  int8_t *q = zalloc(B * big); float *d = zalloc(4 * B * (big / 32)); int32_t *s = zalloc(4 * B * (big / 32));
  int32_t *s16 = zalloc(4 * B * (big / 16));
  for (int b = 0; b < B; b++) {
    orc_quantize_act(x + b * cols, (int)cols, q + b * big, d + b * (big / 32), s + b * (big / 32));
    for (long g = 0; g < cols / 16; g++) {
      int32_t t = 0;
      for (int i = 0; i < 16; i++) t += q[b * big + g * 16 + i];
      s16[b * (big / 16) + g] = t;
    }
  }
  ps_act a = {x, cols, q, big, d, s, big / 32, s16, big / 16};
#pragma omp parallel num_threads(threads < 1 ? 1 : threads)
  {
    int w = 0, n = 1;
#ifdef _OPENMP
    w = omp_get_thread_num(); n = omp_get_num_threads();
#endif
    mm_part(&W, B, &a, y, rows, w, n);
  }
  ps_mat_free(&W);
  free(q); free(d); free(s); free(s16);
  return 0;
}
