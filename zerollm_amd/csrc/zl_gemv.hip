// GEMV dispatch: K-part choice, token chunks, per-format tile kernels (zl_gemv.h, instantiated in zl_gemv_*.hip) and
// the float-weight kernel.
#include "zl_kernels.h"

namespace zl {

// Float weights (F32/F16/BF16) use the f32 activation (src/compute/ref-kernels.js:278-299): one wave per row,
// sequential f64 sum per lane over a strided subset, then a butterfly.
template <int EPI>
__global__ __launch_bounds__(256) void k_gemv_float(const GemvArgs a, int rows_total, const float *__restrict__ xf, int ldx) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  const bool swig = EPI == EPI_SWIGLU;
  if (row >= rows_total) return;
  for (int t = 0; t < a.M; t++) {
    double accs[2] = {0.0, 0.0};
    for (int r = 0; r < (swig ? 2 : 1); r++) {
      int g = row, si = swig ? r : 0, base = 0;
      if (!swig) while (si + 1 < a.nseg && g >= base + a.seg[si].rows) { base += a.seg[si].rows; si++; }
      const MatView &m = a.seg[si].m;
      int lr = g - base;
      double acc = 0;
      for (int c = lane; c < m.cols; c += 64) {
        long e = (long)lr * m.cols + c;
        float wv = m.type == T_F32 ? ((const float *)m.qs)[e] : m.type == T_F16 ? h2f(((const uint16_t *)m.qs)[e])
                                                                                : __uint_as_float((uint32_t)((const uint16_t *)m.qs)[e] << 16);
        acc = acc + (double)wv * (double)xf[(long)t * ldx + c];
      }
      acc = wave_sum_xor(acc, 64);
      accs[r] = acc;
      if (!swig && lane == 0) {
        const GemvSeg &sg = a.seg[si];
        float y = (float)acc;
        if (EPI == EPI_RESID) { float *xp = a.resid + (long)t * a.ldr + lr; *xp = (float)((double)*xp + (double)y); }
        else { if (sg.bias) y = (float)((double)y + (double)sg.bias[lr]); sg.out[(long)t * sg.ldo + lr] = y; }
      }
    }
    if (swig && lane == 0) {
      double g = (double)(float)accs[0], u = (double)(float)accs[1];
      a.hb[(long)t * a.ldh + row] = (float)(g / (1.0 + exp(-g)) * u);
    }
  }
}

// Launch shape, a function of the matrix shape only (so every summation order is independent of the token count):
// - waves per matrix: 4 when there are enough tiles to fill the GPU with workgroups, else 8 (4 for gate/up pairs, whose
//   workgroup runs the gate and the up rows on two halves). Against 16 (8 per gate/up half) each wave holds more slabs,
//   so more of its compute overlaps the loads, and fewer waves meet in the reduction: 5-25 % faster at M = 1, 5, 9 for
//   every 8B and 0.6B projection shape;
// - K parts: 1 (no cross-workgroup sum) unless a part would exceed the staged-activation limit (GT_KR_MAX slabs) or
//   give a wave more than GT_NMAX slabs; for large single-output matrices of fewer tiles than CUs, more parts where that
//   lowers the slabs the busiest CU streams while every wave keeps at least two slabs (attn_output 4096 x 4096: 4 parts,
//   256 workgroups; attn_v 1024 x 4096: 4 parts, so that its launch mixed with attn_q/attn_k's 160 workgroups stays
//   within one round of 256). Not for gate/up pairs: their workgroups hold too many registers to overlap, so rounds of
//   K parts cost more than they save.
void gemv_shape(int ntiles, int nslab, bool swiglu, int *ks, int *nw) {
  const int w = ntiles >= 256 || swiglu ? 4 : 8;  // waves per matrix
  int k = 1;
  while ((nslab + k - 1) / k > 96 || ((nslab + k - 1) / k + w - 1) / w > 16) k *= 2;
  // large matrices of fewer tiles than CUs: more K parts while that lowers the most slabs one CU streams (workgroups
  // run in rounds of 256), keeping at least two slabs per wave
  if (!swiglu && ntiles < 256 && (long)ntiles * nslab >= 1024) {
    auto load = [&](int kk) { return (long)((ntiles * kk + 255) / 256) * ((nslab + kk - 1) / kk); };
    for (int kk = k * 2; kk <= 8 && (nslab + kk - 1) / kk >= 2 * w; kk *= 2)
      if (load(kk) < load(k)) k = kk;
  }
  *ks = k;
  *nw = swiglu ? 2 * w : w;  // a gate/up pair: w waves per matrix
}

// Tokens per GEMM launch (ZEROLLM_GEMM_MAXM, read when a launch is enqueued, so a captured graph keeps the value of its
// capture; below GEMM_MIN_M every launch stays on the GEMV kernels in chunks of at most GEMV_MAX_MT tokens: the same
// bits, more weight passes). Default 64, one launch per prefill chunk: measured against two launches of 32 (whose
// sums fit a wave's registers, where 64 tokens spill a few), 16K-token prefill 6.47 -> 6.21 s (target), 2.69 -> 2.32 s
// (draft).
static int gemm_max_m() {
  const char *e = getenv("ZEROLLM_GEMM_MAXM");
  const int m = e ? atoi(e) : 64;
  return m < GEMM_MIN_M ? 0 : std::min(m, 64);
}

// Launches of at least GEMM_MIN_M tokens (ZEROLLM_GEMM_MINM moves it, for measurements) of the formats the GEMM takes,
// without a fused prologue.
static int gemm_min_m() {
  const char *e = getenv("ZEROLLM_GEMM_MINM");
  return e ? std::max(1, atoi(e)) : GEMM_MIN_M;
}
bool gemm_takes(const GemvArgs &a) {
  const int t = a.seg[0].m.type;
  return gemm_max_m() > 0 && a.M >= gemm_min_m() && !a.xf && (t == T_Q8_0 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K);
}

long gemv_part_need(const GemvArgs &a) {
  if (a.ks == 1) return 0;
  if (gemm_takes(a)) {  // a chunk of at most min(M, cap) tokens in G groups of 16 U (the most for the largest chunk)
    GemvArgs c = a;
    c.M = std::min(a.M, gemm_max_m());
    int U, G;
    gemm_groups(c, U, G);
    return (long)a.ntiles * a.ks * 2 * 16 * U * G * 64;
  }
  return (long)a.ntiles * a.ks * 2 * GEMV_MAX_MT * 64;
}

void launch_gemv(const GemvArgs &a0, int epi, const float *xf, int ldx, hipStream_t st) {
  const int fmt = a0.seg[0].m.type;
  for (int i = 1; i < a0.nseg; i++)
    ZL_REQUIRE(a0.seg[i].m.type == fmt && a0.seg[i].m.nslab == a0.nslab, ZL_ERR_ARG, "gemv: segments differ in type or width");
  if (!is_quant(fmt)) {
    int rows_total = 0;
    for (int i = 0; i < a0.nseg; i++) rows_total += (epi == EPI_SWIGLU && i > 0) ? 0 : a0.seg[i].rows;
    const int blocks = (rows_total + 3) / 4;
    if (epi == EPI_STORE) hipLaunchKernelGGL((k_gemv_float<EPI_STORE>), dim3(blocks), dim3(256), 0, st, a0, rows_total, xf, ldx);
    else if (epi == EPI_RESID) hipLaunchKernelGGL((k_gemv_float<EPI_RESID>), dim3(blocks), dim3(256), 0, st, a0, rows_total, xf, ldx);
    else hipLaunchKernelGGL((k_gemv_float<EPI_SWIGLU>), dim3(blocks), dim3(256), 0, st, a0, rows_total, xf, ldx);
    ZL_HIP(hipGetLastError());
    return;
  }
  ZL_REQUIRE(a0.ks >= 1 && a0.ntiles >= 1, ZL_ERR_ARG, "gemv: bad launch shape");
  ZL_REQUIRE(a0.ks == 1 || (a0.part && a0.cnt && a0.ntiles <= GEMV_CNT_TILES && gemv_part_need(a0) <= GEMV_PART_DOUBLES),
             ZL_ERR_ARG, "gemv: split-K work space missing or too small");
  ZL_REQUIRE(a0.act.q && a0.act.ra && a0.act.rb && a0.act.rc && a0.act.ld % 64 == 0 && a0.act.ld >= a0.nslab * 64,
             ZL_ERR_ARG, "gemv: activation records missing");
  // as few weight passes as chunks of at most 64 (GEMM) or GEMV_MAX_MT tokens allow, with the tokens spread evenly
  // over them; every input and output row is addressed from offset pointers, and the results do not depend on the
  // chunking
  const bool gemm = gemm_takes(a0);
  const int cap = gemm ? gemm_max_m() : GEMV_MAX_MT;
  const int nch = (a0.M + cap - 1) / cap;
  for (int c = 0, t0 = 0; c < nch; c++) {
    GemvArgs b = a0;
    b.M = (a0.M - t0) / (nch - c);  // the remaining tokens over the remaining chunks, the larger chunks last
    ZL_REQUIRE(b.M >= 1 && b.M <= cap, ZL_ERR_ARG, "gemv: bad token chunk");
    if (t0) {
      b.act = act_rows(a0.act, t0);
      for (int i = 0; i < b.nseg; i++) if (b.seg[i].out) b.seg[i].out += (long)t0 * b.seg[i].ldo;
      if (b.resid) b.resid += (long)t0 * b.ldr;
      if (b.hb) b.hb += (long)t0 * b.ldh;
      if (b.qout.q) b.qout = act_rows(a0.qout, t0);
      b.xrow0 += t0;  // fused prologue: the chunk's own input rows
    }
    t0 += b.M;
    if (gemm) {  // every weight read once for all the chunk's tokens, on the matrix cores; same results
      switch (fmt) {
        case T_Q8_0: launch_gemm_fmt<T_Q8_0>(b, epi, st); break;
        case T_Q4_K: launch_gemm_fmt<T_Q4_K>(b, epi, st); break;
        case T_Q5_K: launch_gemm_fmt<T_Q5_K>(b, epi, st); break;
        default: launch_gemm_fmt<T_Q6_K>(b, epi, st); break;
      }
      ZL_HIP(hipGetLastError());
      continue;
    }
    if (gemv_mfma_ok(b)) {  // Q4_K and Q8_0 at 2..8 tokens: the int8 dots on the matrix cores, same results
      launch_gemv_mfma(b, epi, st);
      ZL_HIP(hipGetLastError());
      continue;
    }
    switch (fmt) {
      case T_Q8_0: launch_gemv_fmt<T_Q8_0>(b, epi, st); break;
      case T_Q4_0: launch_gemv_fmt<T_Q4_0>(b, epi, st); break;
      case T_Q5_0: launch_gemv_fmt<T_Q5_0>(b, epi, st); break;
      case T_Q4_K: launch_gemv_fmt<T_Q4_K>(b, epi, st); break;
      case T_Q5_K: launch_gemv_fmt<T_Q5_K>(b, epi, st); break;
      case T_Q6_K: launch_gemv_fmt<T_Q6_K>(b, epi, st); break;
      default: throw Error(ZL_ERR_UNSUPPORTED, "gemv: unsupported weight type");
    }
    ZL_HIP(hipGetLastError());
  }
}

}  // namespace zl
