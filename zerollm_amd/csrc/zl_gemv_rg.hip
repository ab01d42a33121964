// Single-token Q8_0 GEMV in 16-row groups (the draft model's passes: every matrix of a 0.6B-shaped Q8_0 model).
//
// y[r] = sum over the row's 32-value blocks of (s * d) * xd (src/compute/ref-kernels.js:132-152): exact int8 block
// dots, f64 terms. A 256-thread workgroup owns 16 rows (a quarter of a 64-row tile) over the whole K range, so a
// matrix of R rows runs R / 16 workgroups (64 to 384 for the draft's projections) instead of R / 64: a single-token
// GEMV of a few MB is bound by how many CUs stream it and by the critical path of each workgroup, not by arithmetic.
//
// Mapping. Wave w takes the slabs s_j = w + 4 j of K. Every weight load of the wave is issued at kernel entry, right
// behind the wave's activation values (loads complete in order: the RMSNorm and quantisation wait for the activations
// only and run while the weights arrive). The wave quantises the activation values of its own slabs only, so no
// workgroup barrier stands between quantisation and use (one stands before it when the input is RMSNorm'd):
//   - lane l loads x[64 s_j + l], which is x[tid + 256 j] for thread tid = 64 w + l: the element each thread adds in
//     rms_scale256, so the RMSNorm scale is that function's bits;
//   - quantizeAct per 32-value block (src/compute/ref-kernels.js:44-62) as quant32 computes it, except that the
//     block scales' two f64 divisions (d = amax / 127, 1 / d) run once for all of the wave's blocks, one block per
//     lane, instead of once per block on 32 lanes each;
//   - the int8 values go to LDS, where the lanes that multiply them read 16 at a time.
// In a slab, lane l holds row l mod 16 of the group and the 16 values 16 (l / 16) .. + 15 (one 16-byte part of the Q8_0
// plane: the 16 lanes of a part read 256 contiguous bytes). Per slab a lane adds (double)(its 16-value dot) * (d * xd)
// to an f64 sum: d * xd (f16 x f32) and its product with a dot of at most 18 bits are exact in f64, so the two parts'
// terms of a block add up to the block's exact term. The four parts of a row meet by an xor butterfly (16, then 32),
// the four waves in LDS ((w0 + w1) + (w2 + w3)): every order depends on the matrix shape only.
#include "zl_gemv.h"

namespace zl {

constexpr int RG_SPW = 12;  // slabs per wave at most: K <= 4 x 12 x 64 = 3072
constexpr int RG_KMAX = 4 * RG_SPW * 64;

// NSW: slabs per wave the kernel is unrolled for (>= the busiest wave's count).
template <int EPI, int NSW>
__global__ __launch_bounds__(256) void k_gemv_rg_q8(const GemvArgs a) {
  constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;  // gate and up rows of the same group
  __shared__ __align__(16) int8_t xq[RG_KMAX];
  __shared__ float amx[4][2 * RG_SPW];   // per wave: block absolute maxima, then the blocks' f32 scales
  __shared__ double inv[4][2 * RG_SPW];  // per wave: the blocks' f64 inverse scales
  __shared__ double red[NR][4][16];
  __shared__ double ssr[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i16 = lane & 15, p = lane >> 4;  // row of the group, 16-value part of the slab
  const int half = lane >> 5;                // 32-value block of the slab this lane quantises
  const int grp = blockIdx.x, tile = grp >> 2, g = grp & 3;
  const int si = __builtin_amdgcn_readfirstlane(
      EPI != EPI_STORE ? 0 : (a.nseg > 2 && tile >= a.seg[2].tile0) ? 2 : (a.nseg > 1 && tile >= a.seg[1].tile0) ? 1 : 0);
#define ZL_SEG(f) (si == 0 ? a.seg[0].f : si == 1 ? a.seg[1].f : a.seg[2].f)
  const int lt = tile - ZL_SEG(tile0), rows = ZL_SEG(rows);
  const int nslab = a.nslab;
  const int nsw = (nslab - wave + 3) >> 2;  // this wave's slabs: wave + 4 j, j < nsw <= NSW
  __amdgpu_buffer_rsrc_t qs[NR], dd[NR];
  qs[0] = make_rsrc(ZL_SEG(m.qs), ZL_SEG(nqs));
  dd[0] = make_rsrc(ZL_SEG(m.dd), ZL_SEG(ndd));
  if constexpr (NR == 2) {
    qs[1] = make_rsrc(a.seg[1].m.qs, a.seg[1].nqs);
    dd[1] = make_rsrc(a.seg[1].m.dd, a.seg[1].ndd);
  }
  // ---- this wave's activation values x[64 s_j + lane] (= x[tid + 256 j]) and norm weights, requested first: loads
  // complete in order, so the prologue below waits for these alone while the weights are still on their way
  const int n = a.n;
  const float *xr = a.xf + (long)a.xrow0 * a.ldxf;
  const float *wr = a.nw ? a.nw : xr;  // (no weights: a second read of x, unused; unconditional loads)
  float xv[NSW], wn[NSW];
  #pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int i = 64 * (wave + 4 * j) + lane;
    xv[j] = xr[i < n ? i : 0];
    wn[j] = wr[i < n ? i : 0];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the weight loads behind these
  // ---- every weight load of this wave, issued before anything waits (past the wave's slabs: out-of-range offsets,
  // answered with zeros and no memory access)
  const int r64 = 16 * g + i16;
  u32x4 wv[NR][NSW];
  uint32_t dv[NR][NSW];
  #pragma unroll
  for (int j = 0; j < NSW; j++) {
    const bool ok = j < nsw;
    const int ts = ok ? lt * nslab + wave + 4 * j : 0;
    const int oob = ok ? 0 : 0x40000000;
    #pragma unroll
    for (int r = 0; r < NR; r++) {
      wv[r][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qs[r], oob + (p * 64 + r64) * 16, ts * 4096, 0));
      dv[r][j] = __builtin_amdgcn_raw_buffer_load_b16(dd[r], oob + (r64 * 2 + (p >> 1)) * 2, ts * 256, 0);
    }
  }
  // the residual value this workgroup's epilogue adds to (threads 0-15: row 16 g + tid of the tile), requested with the
  // weights rather than after the reduction, where its latency would follow the kernel's last step
  float rres = 0.f;
  if constexpr (EPI == EPI_RESID) rres = a.resid[min(lt * 64 + r64, rows - 1)];
  // ---- the activation values, RMSNorm'd with nw when set
  double sc = 1.0;
  if (a.nw) {  // rms_scale256's order: this thread's squares in j order, the 64-lane butterfly, the four waves
    double ss = 0.0;
    #pragma unroll
    for (int j = 0; j < NSW; j++) {
      const double x = 64 * (wave + 4 * j) + lane < n ? (double)xv[j] : 0.0;
      ss += x * x;
    }
    sc = rms_finish(ss, n, a.eps, tid, ssr);
  }
  float v[NSW];
  #pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int i = 64 * (wave + 4 * j) + lane;
    v[j] = i < n ? (a.nw ? (float)((double)xv[j] * sc * (double)wn[j]) : xv[j]) : 0.f;
    const float am = group_fmax(fabsf(v[j]), 32);
    if ((lane & 31) == 0) amx[wave][2 * j + half] = am;
  }
  // lanes read what other lanes of the same wave wrote to LDS: a wave-scope fence orders the accesses
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  // the scales of the wave's 2 NSW blocks, one block per lane: d = amax / 127 (f64, stored f32), inverse 1 / d
  if (lane < 2 * NSW) {
    const double scale = (double)amx[wave][lane] / 127.0;
    inv[wave][lane] = scale != 0.0 ? 1.0 / scale : 0.0;
    amx[wave][lane] = (float)scale;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  #pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int q = (int)round((double)v[j] * inv[wave][2 * j + half]);
    xq[64 * (wave + 4 * j) + lane] = (int8_t)q;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  // ---- the slab terms (the wave reads back only what it wrote: LDS accesses of a wave complete in order)
  double acc[NR];
  #pragma unroll
  for (int r = 0; r < NR; r++) acc[r] = 0.0;
  uint4 x4[NSW];
  double xd[NSW];
  #pragma unroll
  for (int j = 0; j < NSW; j++) {
    x4[j] = *(const uint4 *)(xq + 64 * (wave + 4 * j) + 16 * p);
    xd[j] = (double)amx[wave][2 * j + (p >> 1)];
  }
  #pragma unroll
  for (int j = 0; j < NSW; j++) {
    if (j < nsw) {
      #pragma unroll
      for (int r = 0; r < NR; r++) {
        int dot = sdot4((int)x4[j].x, (int)wv[r][j].x, 0);
        dot = sdot4((int)x4[j].y, (int)wv[r][j].y, dot);
        dot = sdot4((int)x4[j].z, (int)wv[r][j].z, dot);
        dot = sdot4((int)x4[j].w, (int)wv[r][j].w, dot);
        acc[r] = fma((double)dot, (double)h2f((uint16_t)dv[r][j]) * xd[j], acc[r]);
      }
    }
  }
  // ---- parts of a row (xor 16, then xor 32), then the four waves
  #pragma unroll
  for (int r = 0; r < NR; r++) {
    double s = acc[r] + swizzle_xor16(acc[r]);
    s = s + __shfl_xor(s, 32, 64);
    if (p == 0) red[r][wave][i16] = s;
  }
  __syncthreads();
  if (tid < 16) {
    const int row = lt * 64 + r64;
    double tot[NR];
    #pragma unroll
    for (int r = 0; r < NR; r++) tot[r] = (red[r][0][tid] + red[r][1][tid]) + (red[r][2][tid] + red[r][3][tid]);
    if (row < rows) {
      if constexpr (EPI == EPI_SWIGLU) {
        const double gv = (double)(float)tot[0], uu = (double)(float)tot[1];
        a.hb[row] = (float)(gv / (1.0 + exp(-gv)) * uu);  // src/compute/ref-kernels.js:322
      } else if constexpr (EPI == EPI_RESID) {
        a.resid[row] = (float)((double)rres + (double)(float)tot[0]);
      } else {
        const float y = (float)tot[0];
        const float *bias = ZL_SEG(bias);
        ZL_SEG(out)[row] = bias ? (float)((double)y + (double)bias[row]) : y;
      }
    }
  }
#undef ZL_SEG
}

bool gemv_rg_ok(const GemvArgs &a) {
  if (a.M != 1 || !a.xf || a.nslab > 4 * RG_SPW) return false;
  for (int i = 0; i < a.nseg; i++)
    if (a.seg[i].m.type != T_Q8_0) return false;
  return true;
}

template <int EPI>
static void launch_rg_epi(const GemvArgs &a, hipStream_t st) {
  const dim3 grid((unsigned)a.ntiles * 4), blk(256);
  const int nsw = (a.nslab + 3) / 4;  // slabs of wave 0, the busiest
  if (nsw <= 1) hipLaunchKernelGGL((k_gemv_rg_q8<EPI, 1>), grid, blk, 0, st, a);
  else if (nsw <= 2) hipLaunchKernelGGL((k_gemv_rg_q8<EPI, 2>), grid, blk, 0, st, a);
  else if (nsw <= 4) hipLaunchKernelGGL((k_gemv_rg_q8<EPI, 4>), grid, blk, 0, st, a);
  else if (nsw <= 6) hipLaunchKernelGGL((k_gemv_rg_q8<EPI, 6>), grid, blk, 0, st, a);
  else if (nsw <= 8) hipLaunchKernelGGL((k_gemv_rg_q8<EPI, 8>), grid, blk, 0, st, a);
  else hipLaunchKernelGGL((k_gemv_rg_q8<EPI, 12>), grid, blk, 0, st, a);
}

void launch_gemv_rg(const GemvArgs &a, int epi, hipStream_t st) {
  ZL_REQUIRE(gemv_rg_ok(a) && a.n <= a.nslab * 64 && a.ntiles >= 1, ZL_ERR_ARG, "gemv (16-row groups): bad arguments");
  if (epi == EPI_STORE) launch_rg_epi<EPI_STORE>(a, st);
  else if (epi == EPI_RESID) launch_rg_epi<EPI_RESID>(a, st);
  else launch_rg_epi<EPI_SWIGLU>(a, st);
  ZL_HIP(hipGetLastError());
}

}  // namespace zl
