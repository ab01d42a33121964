// Forward-pass kernels for gfx950: weight repack, dequantisation, RMSNorm + int8 activation quantisation, per-head q/k
// RMSNorm + RoPE + KV append, and causal GQA attention (the GEMV family is in zl_gemv.hip).
//
// Numerics follow zerollm's reference path (src/model/forward.js:184-248, src/compute/ref-kernels.js): integer block
// dots are exact; every scale combination, norm, softmax and RoPE step is done in f64 with the reference's rounding
// points (f32 stores); the attention weighted sum accumulates in f32 in position order, one fused multiply-add per
// position, as the reference's `attOut[i] += p * V[i]` does. The only freedom taken is the order of f64 sums (block
// partials across lanes, softmax denominators), which moves results by ~1e-16 relative before the f32 rounding.
// The whole library is built with -ffp-contract=off; fusions are written out explicitly.
#include "zl_kernels.h"

namespace zl {

// ================================================================================================ repack
// Raw ggml blocks of one matrix (rows x rawRowBytes) -> slab planes (see DevMat in zl_common.h).

__device__ inline void q6_value(const uint8_t *blk, int e, int &lo4, int &hi2) {
  int h = e >> 7, e2 = e & 127, qq = e2 >> 5, l = e2 & 31;
  int byte = blk[64 * h + ((qq & 1) ? 32 : 0) + l];
  lo4 = (qq < 2) ? (byte & 15) : (byte >> 4);
  hi2 = (blk[128 + 32 * h + l] >> (2 * qq)) & 3;
}

// One thread per (row, slab): reads the raw ggml blocks of the slab and writes its tiled-plane elements.
__global__ void k_repack(int type, const uint8_t *__restrict__ raw, long rawRowBytes, int rows, int cols, int nslab,
                         uint8_t *qs, uint8_t *qx, uint8_t *sc, uint16_t *dd) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * nslab) return;
  int r = (int)(idx / nslab), s = (int)(idx % nslab);
  const uint8_t *row = raw + (long)r * rawRowBytes;
  uint8_t oq[64];
  if (type == T_Q8_0 || type == T_Q4_0 || type == T_Q5_0) {
    int nb = cols / 32;
    int bsz = type == T_Q8_0 ? 34 : type == T_Q4_0 ? 18 : 22;
    for (int j = 0; j < 32; j++) oq[j] = 0;
    for (int half = 0; half < 2; half++) {
      int b = 2 * s + half;
      const uint8_t *blk = b < nb ? row + (long)b * bsz : nullptr;
      dd[dd_off(type, r, s, nslab, half)] = blk ? (uint16_t)(blk[0] | (blk[1] << 8)) : 0;
      if (type == T_Q8_0) {
        for (int i = 0; i < 32; i++) oq[32 * half + i] = blk ? blk[2 + i] : 0;
      } else {
        const uint8_t *nib = blk ? blk + (type == T_Q4_0 ? 2 : 6) : nullptr;
        // block value j: j < 16 low nibble of byte j, else high nibble of byte j-16; slab byte j holds value j (low
        // nibble, from block 2s) and value j+32 (high nibble, from block 2s+1)
        for (int j = 0; j < 32; j++) {
          int v = nib ? (j < 16 ? (nib[j] & 15) : (nib[j - 16] >> 4)) : 0;
          oq[j] = (uint8_t)(oq[j] | (half == 0 ? v : v << 4));
        }
        if (type == T_Q5_0) {
          uint32_t h = blk ? ((uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24)) : 0u;
          for (int i = 0; i < 4; i++) qx[qx_off(type, r, s, nslab, 4 * half + i)] = (h >> (8 * i)) & 0xff;
        }
      }
    }
    for (int j = 0; j < qs_bytes(type); j++) qs[qs_off(type, r, s, nslab, j)] = oq[j];
    return;
  }
  if (type == T_Q4_K || type == T_Q5_K) {
    int five = type == T_Q5_K;
    int sb = s >> 2, c = s & 3;
    const uint8_t *blk = row + (long)sb * (five ? 176 : 144);
    const uint8_t *src = blk + (five ? 48 : 16) + 32 * c;
    for (int l = 0; l < 32; l++) qs[qs_off(type, r, s, nslab, l)] = src[l];
    const uint8_t *S = blk + 4;
    int scv[8], mnv[8];
    for (int j = 0; j < 4; j++) {
      scv[j] = S[j] & 63; mnv[j] = S[j + 4] & 63;
      scv[j + 4] = (S[j + 8] & 0x0f) | ((S[j] >> 6) << 4);
      mnv[j + 4] = (S[j + 8] >> 4) | ((S[j + 4] >> 6) << 4);
    }
    sc[sc_off(r, s, nslab, 0)] = (uint8_t)scv[2 * c];
    sc[sc_off(r, s, nslab, 1)] = (uint8_t)scv[2 * c + 1];
    sc[sc_off(r, s, nslab, 2)] = (uint8_t)mnv[2 * c];
    sc[sc_off(r, s, nslab, 3)] = (uint8_t)mnv[2 * c + 1];
    if (c == 0) {
      dd[dd_off(type, r, s, nslab, 0)] = (uint16_t)(blk[0] | (blk[1] << 8));
      dd[dd_off(type, r, s, nslab, 1)] = (uint16_t)(blk[2] | (blk[3] << 8));
    }
    if (five) {
      uint32_t w0 = 0, w1 = 0;
      for (int l = 0; l < 32; l++) {
        w0 |= (uint32_t)((blk[16 + l] >> (2 * c)) & 1) << l;
        w1 |= (uint32_t)((blk[16 + l] >> (2 * c + 1)) & 1) << l;
      }
      for (int i = 0; i < 4; i++) {
        qx[qx_off(type, r, s, nslab, i)] = (w0 >> (8 * i)) & 0xff;
        qx[qx_off(type, r, s, nslab, 4 + i)] = (w1 >> (8 * i)) & 0xff;
      }
    }
    return;
  }
  if (type == T_Q6_K) {
    int sb = s >> 2, u = s & 3;
    const uint8_t *blk = row + (long)sb * 210;
    for (int j = 0; j < 32; j++) {
      int lo0, hi0, lo1, hi1;
      q6_value(blk, 64 * u + j, lo0, hi0);
      q6_value(blk, 64 * u + 32 + j, lo1, hi1);
      qs[qs_off(type, r, s, nslab, j)] = (uint8_t)(lo0 | (lo1 << 4));
    }
    for (int j = 0; j < 16; j++) {
      int b = 0;
      for (int i = 0; i < 4; i++) { int lo, hi; q6_value(blk, 64 * u + j + 16 * i, lo, hi); b |= hi << (2 * i); }
      qx[qx_off(type, r, s, nslab, j)] = (uint8_t)b;
    }
    for (int g = 0; g < 4; g++) sc[sc_off(r, s, nslab, g)] = blk[192 + 4 * u + g];
    if (u == 0) dd[dd_off(type, r, s, nslab, 0)] = (uint16_t)(blk[208] | (blk[209] << 8));
    return;
  }
}

// Q4_K 4-bit plane in matrix-core operand order (zl_gemv_mfma.hip): one thread per (row, slab) of the padded tiles. Row
// r = 64 T + 16 j + n, value quarter g (values 16 g + e, e < 16) goes to lane L = n + 16 g of half j / 2 of the
// tile-slab's 2 KB, bytes 8 (j mod 2) .. + 8: byte i of the first word holds values e = i (low nibble) and i + 4 (high),
// byte i of the second word e = 8 + i and 12 + i.
__global__ void k_frag(const uint8_t *__restrict__ qs, uint8_t *__restrict__ fq, int rowsPadded, int nslab) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rowsPadded * nslab) return;
  const int r = (int)(idx / nslab), s = (int)(idx % nslab);
  uint8_t b[32];
  for (int j = 0; j < 32; j++) b[j] = qs[qs_off(T_Q4_K, r, s, nslab, j)];
  auto val = [&](int v) { return v < 32 ? (b[v] & 15) : (b[v - 32] >> 4); };  // value v of the slab (row layout)
  const int rr = r & 63, jg = rr >> 4, n = rr & 15;
  const long ts = tile_slab(r, s, nslab);
  for (int g = 0; g < 4; g++) {
    uint8_t *dst = fq + ((ts * 2 + (jg >> 1)) * 64 + n + 16 * g) * 16 + (jg & 1) * 8;
    for (int i = 0; i < 4; i++) {
      dst[i] = (uint8_t)(val(16 * g + i) | (val(16 * g + i + 4) << 4));
      dst[4 + i] = (uint8_t)(val(16 * g + 8 + i) | (val(16 * g + 12 + i) << 4));
    }
  }
}

// ================================================================================================ dequantisation
// dequantRow (src/compute/ref-kernels.js:80-120, src/compute/quant.js:33-202) for value c of row r of the repacked
// planes, in f64 with one rounding to f32. One element per thread: coalesced stores, no private arrays.
__device__ inline float dequant_value(const MatView &m, int r, int c) {
  const int t = m.type, s = c >> 6, v = c & 63, h = v >> 5, j = v & 31;
  if (t == T_F32 || t == T_F16 || t == T_BF16) {
    if (c >= m.cols) return 0.f;
    const long e = (long)r * m.cols + c;
    if (t == T_F32) return ((const float *)m.qs)[e];
    if (t == T_F16) return h2f(((const uint16_t *)m.qs)[e]);
    return __uint_as_float((uint32_t)((const uint16_t *)m.qs)[e] << 16);
  }
  const int ns = m.nslab;
  if (t == T_Q8_0) {
    const double d = (double)h2f(m.dd[dd_off(t, r, s, ns, h)]);
    return (float)(d * (double)(int8_t)m.qs[qs_off(t, r, s, ns, v)]);
  }
  const uint8_t qb = m.qs[qs_off(t, r, s, ns, j)];
  const int nib = h == 0 ? (qb & 15) : (qb >> 4);
  if (t == T_Q4_0 || t == T_Q5_0) {
    const double d = (double)h2f(m.dd[dd_off(t, r, s, ns, h)]);
    const int hb = t == T_Q5_0 ? (m.qx[qx_off(t, r, s, ns, 4 * h + (j >> 3))] >> (j & 7)) & 1 : 0;
    const int val = t == T_Q4_0 ? nib - 8 : (nib | (hb << 4)) - 16;
    return (float)(d * (double)val);
  }
  if (t == T_Q4_K || t == T_Q5_K) {
    const double d = (double)h2f(m.dd[dd_off(t, r, s, ns, 0)]), dmin = (double)h2f(m.dd[dd_off(t, r, s, ns, 1)]);
    const int sc = m.sc[sc_off(r, s, ns, h)], mn = m.sc[sc_off(r, s, ns, 2 + h)];
    int q = nib;
    if (t == T_Q5_K) q |= ((m.qx[qx_off(t, r, s, ns, 4 * h + (j >> 3))] >> (j & 7)) & 1) << 4;
    return (float)(d * (double)sc * (double)q - dmin * (double)mn);
  }
  // Q6_K
  const double d = (double)h2f(m.dd[dd_off(t, r, s, ns, 0)]);
  const int lo = v < 32 ? (m.qs[qs_off(t, r, s, ns, v)] & 15) : (m.qs[qs_off(t, r, s, ns, v - 32)] >> 4);
  const int hi = (m.qx[qx_off(t, r, s, ns, v & 15)] >> (2 * (v >> 4))) & 3;
  const int val = (lo | (hi << 4)) - 32;
  return (float)(d * (double)(int8_t)m.sc[sc_off(r, s, ns, v >> 4)] * (double)val);
}

__global__ void k_dequant_rows(const MatView m, const int *rowIds, int nrows, float *out, int ldo) {
  const int rr = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
  if (rr >= nrows || c >= m.cols) return;
  out[(long)rr * ldo + c] = dequant_value(m, rowIds[rr], c);
}

// Embedding lookup: x[b] = dequant(token_embd row step.tokens[b]) (src/model/forward.js:195).
__global__ void k_embed(const MatView m, const Step *step, float *x, int ldx) {
  const int b = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= step->B || c >= m.cols) return;
  x[(long)b * ldx + c] = dequant_value(m, step->tokens[b], c);
}

// ================================================================================================ activation quantisation
// RMSNorm (optional) + quantisation of rows x[row0 + blockIdx.y] (length n) into activation row blockIdx.y (length
// npad >= n, zero padded). rmsnorm: s = 1/sqrt(mean(x^2) + eps), xb = x*s*w (src/compute/ref-kernels.js:305-310).
// Block blockIdx.x quantises elements [512*blockIdx.x, +512); every block of a row computes the same sum of squares
// (same order), so they all use the same s.
constexpr int NQ_CHUNK = 512;
__global__ __launch_bounds__(256) void k_norm_quant(const float *__restrict__ x, int ldx, int row0, const float *__restrict__ w,
                                                    double eps, int n, int npad, Act act) {
  __shared__ double red[4];
  const int b = blockIdx.y, tid = threadIdx.x;
  const float *xr = x + (long)(row0 + b) * ldx;
  // the chunk's values and weights are requested before the sum of squares, which does not wait for them
  constexpr int PER = NQ_CHUNK / 256;
  const int c0 = blockIdx.x * NQ_CHUNK, c1 = min(npad, c0 + NQ_CHUNK);
  float xv[PER], wv[PER];
  const float *wr = w ? w : xr;  // (no weights: a second read of x, unused)
  #pragma unroll
  for (int k = 0; k < PER; k++) {  // unconditional loads: a branch around a load makes the compiler wait for it there
    const int i = c0 + tid + 256 * k;
    xv[k] = xr[i < n ? i : 0];
    wv[k] = wr[i < n ? i : 0];
  }
  const double s = w ? rms_scale256(xr, n, eps, tid, red) : 1.0;
  #pragma unroll
  for (int k = 0; k < PER; k++) {
    const int i = c0 + tid + 256 * k;
    // c1 - c0 is a multiple of 64: a wave's 64 values are all in the chunk or all past it (quant_block32 works on
    // 32-lane groups)
    if (i < c1) {
      float v = 0.f;
      if (i < n) v = w ? (float)((double)xv[k] * s * (double)wv[k]) : xv[k];  // (positions past n stay 0)
      if (act.f) act.f[(long)b * act.ld + i] = v;
      quant_block32(v, i, act, b);
    }
  }
}

// ================================================================================================ synthetic weights
// Raw ggml blocks of a synthetic tensor generated in place (zerollm_amd/csrc/synth.h): one thread per block.
__global__ void k_synth(int type, uint64_t seed, double std, uint64_t srcCols, uint64_t col0, int rows, int cols,
                        uint8_t *out) {
  int bv = zl_synth::block_values(type), bb = zl_synth::block_bytes(type);
  long nbr = cols / bv;
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * nbr) return;
  long r = idx / nbr, b = idx % nbr;
  zl_synth::synth_block(type, seed, std, srcCols, col0, (uint64_t)r, (uint64_t)b, out + idx * bb);
}

__global__ void k_fill_f32(float *p, long n, float v) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ================================================================================================ launch helpers
void launch_norm_quant(const float *x, int ldx, int row0, int nrows, const float *w, double eps, int n, int npad,
                       const Act &act, hipStream_t st) {
  hipLaunchKernelGGL(k_norm_quant, dim3((npad + NQ_CHUNK - 1) / NQ_CHUNK, nrows), dim3(256), 0, st, x, ldx, row0, w, eps, n, npad, act);
  ZL_HIP(hipGetLastError());
}


void launch_embed(const MatView &m, const Step *step, int B, float *x, int ldx, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3((m.cols + 255) / 256, B), dim3(256), 0, st, m, step, x, ldx);
  ZL_HIP(hipGetLastError());
}

void launch_dequant_rows(const MatView &m, const int *rowIds, int nrows, float *out, int ldo, hipStream_t st) {
  hipLaunchKernelGGL(k_dequant_rows, dim3((m.cols + 255) / 256, nrows), dim3(256), 0, st, m, rowIds, nrows, out, ldo);
  ZL_HIP(hipGetLastError());
}

void launch_repack(int type, const uint8_t *raw, long rawRowBytes, int rows, int cols, int nslab, DevMat &m, hipStream_t st) {
  long n = (long)rows * nslab;
  hipLaunchKernelGGL(k_repack, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, type, raw, rawRowBytes, rows, cols, nslab,
                     m.qs, m.qx, m.sc, m.dd);
  ZL_HIP(hipGetLastError());
}

void launch_frag(const DevMat &m, hipStream_t st) {
  const int rp = tiles_of(m.rows) * 64;
  const long n = (long)rp * m.nslab;
  hipLaunchKernelGGL(k_frag, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, m.qs, m.fq, rp, m.nslab);
  ZL_HIP(hipGetLastError());
}

void launch_synth(int type, uint64_t seed, double std, uint64_t srcCols, uint64_t col0, int rows, int cols, uint8_t *out,
                  hipStream_t st) {
  long n = (long)rows * (cols / zl_synth::block_values(type));
  hipLaunchKernelGGL(k_synth, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, type, seed, std, srcCols, col0, rows, cols, out);
  ZL_HIP(hipGetLastError());
}

void launch_fill(float *p, long n, float v, hipStream_t st) {
  hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n, v);
  ZL_HIP(hipGetLastError());
}

}  // namespace zl
