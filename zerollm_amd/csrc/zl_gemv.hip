// Quantised GEMV for M = 1..64 tokens on gfx950: y[t][r] = sum over the row's blocks of the reference's per-block term
// (src/compute/ref-kernels.js:127-302), exact int8 block dots (v_dot4_i32_i8), f64 scale combination with the
// reference's rounding points.
//
// Mapping. `lpr` lanes share a pair of rows (the gate/up pair for SwiGLU) and take the row's 64-value slabs round robin
// (lane j: slabs j, j+lpr, ...); each lane adds its blocks' f64 terms in slab order, then a DPP butterfly combines the
// lpr lanes. lpr depends only on the matrix shape, so a batched pass gives the same bits as token-by-token passes.
// A block of 512 threads (8 waves) stages the activations of MT tokens in LDS once (int8 values, and per 32-value
// block one 16-byte record of scale and sums pre-converted), then strides over row pairs. The first slabs' weight
// loads are issued before the staging, and each lane keeps the next slab's loads in flight while it computes, across
// row-pair boundaries too. The token loop is unrolled without branches (a short last tile reads its last token again
// and stores nothing for the copies), so the LDS reads of all tokens overlap the integer dots.
#include "zl_kernels.h"

#include <map>

namespace zl {

constexpr int GV_THREADS = 512;
constexpr int GV_WAVES = GV_THREADS / 64;
constexpr size_t GV_LDS_MAX = 150 * 1024;


// ---------------------------------------------------------------------------------------------- staged activations
// LDS layout for a tile of MT tokens over K values (nslab = K/64 slabs, values 64s + 32h + 16p + e):
//   X    [MT][h 2][p 2][nslab] x 16 B int8: lanes that take consecutive slabs read consecutive 16-byte pieces, so the
//        reads of a wave hit distinct banks
//   REC  [MT][h 2][nslab] x 16 B: per 32-value block, f64 scale d, then f64 block sum (Q4_K/Q5_K) | int32 sum
//        (Q4_0/Q5_0) | two int32 16-value sums (Q6_K) | nothing (Q8_0)
struct ActRec {
  double d;
  union {
    double s;
    int32_t i[2];
  };
};
__host__ __device__ inline size_t act_rec_off(int mt, int K) { return (size_t)mt * K; }
size_t gemv_lds_bytes(int fmt, int mt, int K) { (void)fmt; return act_rec_off(mt, K) + (size_t)mt * (K / 32) * 16; }

// X piece (16 values) number i of token t's row, and the record of its 32-value block b, in the layout above
__device__ inline int x_piece(int t, int i, int nslab) { return ((t * 2 + ((i >> 1) & 1)) * 2 + (i & 1)) * nslab + (i >> 2); }
__device__ inline int rec_index(int t, int b, int nslab) { return (t * 2 + (b & 1)) * nslab + (b >> 1); }

template <int FMT>
__device__ inline void put_rec(uint8_t *lds, int mt, int K, int b, double d, int s32, int s16a, int s16b) {
  ActRec r;
  r.d = d;
  if (FMT == T_Q4_K || FMT == T_Q5_K) r.s = (double)s32;
  else if (FMT == T_Q6_K) { r.i[0] = s16a; r.i[1] = s16b; }
  else { r.i[0] = s32; r.i[1] = 0; }
  ((ActRec *)(lds + act_rec_off(mt, K)))[b] = r;
}

// Stage tokens [t0, t0+mt) of the quantised activation. Every load of a batch is issued before its stores.
template <int FMT>
__device__ inline void stage_act(const Act &act, int t0, int mt, int MTL, int K, uint8_t *lds) {
  const int tid = threadIdx.x;
  const int pq = K >> 4;  // 16-byte pieces of int8 values per token
  const int nsb = K >> 5;
  const int np = mt * pq, ns = mt * nsb;
  for (int base = 0; base < np || base < ns; base += 2 * GV_THREADS) {
    uint4 v[2];
    float d[2];
    int sv[2], sa[2], sb[2];
    #pragma unroll
    for (int k = 0; k < 2; k++) {
      const int i = base + k * GV_THREADS + tid;
      v[k] = i < np ? *(const uint4 *)(act.q + (long)(t0 + i / pq) * act.ld + (i % pq) * 16) : make_uint4(0, 0, 0, 0);
      const int t = i / nsb, b = i % nsb;
      const long src = (long)(t0 + t) * (act.ld >> 5) + b;
      const long src16 = (long)(t0 + t) * (act.ld >> 4) + 2 * b;
      const bool live = i < ns;
      d[k] = live ? act.d[src] : 0.f;
      sv[k] = live && FMT != T_Q8_0 && FMT != T_Q6_K ? act.s[src] : 0;
      sa[k] = live && FMT == T_Q6_K ? act.s16[src16] : 0;
      sb[k] = live && FMT == T_Q6_K ? act.s16[src16 + 1] : 0;
    }
    #pragma unroll
    for (int k = 0; k < 2; k++) {
      const int i = base + k * GV_THREADS + tid;
      if (i < np) *(uint4 *)(lds + (size_t)x_piece(i / pq, i % pq, K >> 6) * 16) = v[k];
      if (i < ns) put_rec<FMT>(lds, MTL, K, rec_index(i / nsb, i % nsb, K >> 6), (double)d[k], sv[k], sa[k], sb[k]);
    }
  }
}

// Stage tokens [t0, t0+mt) by quantising f32 rows here, with optional RMSNorm first: the same arithmetic and the same
// reduction order as k_norm_quant (256 strided partial sums of squares, a wave butterfly, then (w0+w1)+(w2+w3)), so
// the staged values equal what k_norm_quant writes. Used where the rows are short, so that the block's redundant work
// costs less than a launch.
template <int FMT, int MT>
__device__ inline void stage_f32(const GemvArgs &a, int t0, int mt, int K, uint8_t *lds) {
  __shared__ double red[MT][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = a.n;
  if (a.nw && wave < 4) {
    #pragma unroll
    for (int t = 0; t < MT; t++) {
      if (t < mt) {
        const float *xr = a.xf + (long)(a.xrow0 + t0 + t) * a.ldxf;
        double ss = 0;
        for (int i = tid; i < n; i += 256) { const double v = (double)xr[i]; ss += v * v; }
        ss = wave_sum_xor(ss, 64);
        if (lane == 0) red[t][wave] = ss;
      }
    }
  }
  __syncthreads();
  for (int base = 0; base < mt * K; base += GV_THREADS) {
    const int idx = base + tid;  // a wave's 64 elements lie in one token's row (K is a multiple of 64)
    const int t = min(idx / K, mt - 1), i = idx % K;
    const bool live = idx < mt * K;
    const float *xr = a.xf + (long)(a.xrow0 + t0 + t) * a.ldxf;
    float v = 0.f;
    if (live && i < n) {
      if (a.nw) {
        const double ss = (red[t][0] + red[t][1]) + (red[t][2] + red[t][3]);
        const double sc = 1.0 / sqrt(ss / (double)n + a.eps);
        v = (float)((double)xr[i] * sc * (double)a.nw[i]);
      } else {
        v = xr[i];
      }
    }
    // quantizeAct of one 32-value block per 32 lanes (src/compute/ref-kernels.js:44-62)
    const float am = group_fmax(fabsf(v), 32);
    const double scale = (double)am / 127.0;
    const double inv = scale != 0.0 ? 1.0 / scale : 0.0;
    const int q = (int)round((double)v * inv);
    const int s16 = wave_sum_xor(q, 16);
    const int s16b = __shfl_down(s16, 16, 32);  // the block's second 16-value sum, at its first lane
    const int s32 = s16 + swizzle_xor16(s16);
    if (live) {
      lds[(size_t)x_piece(t, i >> 4, K >> 6) * 16 + (i & 15)] = (uint8_t)(int8_t)q;
      if ((i & 31) == 0) put_rec<FMT>(lds, MT, K, rec_index(t, i >> 5, K >> 6), (double)(float)scale, s32, s16, s16b);
    }
  }
}

// ---------------------------------------------------------------------------------------------- one slab
// Raw planes of one slab as loaded (unpacked only when used, so the next slab's loads stay in flight meanwhile).
template <int FMT>
struct Slab {
  uint32_t L[FMT == T_Q8_0 ? 16 : 8];                                    // int8 values / packed nibbles
  uint32_t H[FMT == T_Q6_K ? 4 : (FMT == T_Q5_0 || FMT == T_Q5_K) ? 2 : 1];  // high bits
  uint32_t scw;                                                           // scale codes (K-quants)
  uint32_t dw;  // f16 scales: (d0 | d1 << 16) Q8_0/Q4_0/Q5_0; (d | dmin << 16) Q4_K/Q5_K; d Q6_K
};

// Buffer resources of a matrix's planes (rows x nslab slabs): loads then take a 32-bit byte offset and read zeros
// past the end of a plane instead of faulting.
struct Planes {
  __amdgpu_buffer_rsrc_t qs, qx, sc, dd;
};
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *p, long bytes) {
  const uint32_t n = bytes <= 0 ? 0u : bytes > 0xFFFFFFFFl ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)n, 0x00020000);
}
template <int FMT>
__device__ inline Planes planes_of(const MatView &m, int rows) {
  const long ns = (long)rows * m.nslab;
  Planes P;
  P.qs = make_rsrc(m.qs, ns * (FMT == T_Q8_0 ? 64 : 32));
  P.qx = make_rsrc(m.qx, (FMT == T_Q5_0 || FMT == T_Q5_K) ? ns * 8 : FMT == T_Q6_K ? ns * 16 : 0);
  P.sc = make_rsrc(m.sc, (FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q6_K) ? ns * 4 : 0);
  P.dd = make_rsrc(m.dd, (FMT == T_Q4_K || FMT == T_Q5_K) ? (ns / 4) * 4 : FMT == T_Q6_K ? (ns / 4) * 2 : ns * 4);
  return P;
}

// Slab number i (= row * nslab + slab) of the planes.
template <int FMT>
__device__ inline void load_slab(const Planes &P, int i, Slab<FMT> &o) {
  typedef uint32_t v4 __attribute__((ext_vector_type(4)));
  typedef uint32_t v2 __attribute__((ext_vector_type(2)));
  if (FMT == T_Q8_0) {
    #pragma unroll
    for (int k = 0; k < 4; k++) {
      v4 v = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(P.qs, i * 64 + 16 * k, 0, 0));
      o.L[4 * k] = v.x; o.L[4 * k + 1] = v.y; o.L[4 * k + 2] = v.z; o.L[4 * k + 3] = v.w;
    }
    o.dw = __builtin_amdgcn_raw_buffer_load_b32(P.dd, i * 4, 0, 0);
    return;
  }
  v4 a = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(P.qs, i * 32, 0, 0));
  v4 b = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(P.qs, i * 32 + 16, 0, 0));
  o.L[0] = a.x; o.L[1] = a.y; o.L[2] = a.z; o.L[3] = a.w; o.L[4] = b.x; o.L[5] = b.y; o.L[6] = b.z; o.L[7] = b.w;
  if (FMT == T_Q5_0 || FMT == T_Q5_K) {
    v2 h = __builtin_bit_cast(v2, __builtin_amdgcn_raw_buffer_load_b64(P.qx, i * 8, 0, 0));
    o.H[0] = h.x; o.H[1] = h.y;
  }
  if (FMT == T_Q6_K) {
    v4 h = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(P.qx, i * 16, 0, 0));
    o.H[0] = h.x; o.H[1] = h.y; o.H[2] = h.z; o.H[3] = h.w;
  }
  if (FMT == T_Q4_0 || FMT == T_Q5_0) o.dw = __builtin_amdgcn_raw_buffer_load_b32(P.dd, i * 4, 0, 0);
  // K-quants: the row's slab count is a multiple of 4, so slab i lies in super-block i / 4 of the dd plane
  if (FMT == T_Q4_K || FMT == T_Q5_K) {
    o.scw = __builtin_amdgcn_raw_buffer_load_b32(P.sc, i * 4, 0, 0);
    o.dw = __builtin_amdgcn_raw_buffer_load_b32(P.dd, (i >> 2) * 4, 0, 0);
  }
  if (FMT == T_Q6_K) {
    o.scw = __builtin_amdgcn_raw_buffer_load_b32(P.sc, i * 4, 0, 0);
    o.dw = __builtin_amdgcn_raw_buffer_load_b16(P.dd, (i >> 2) * 2, 0, 0);
  }
}

// Values of half h (32 values: 0-31 or 32-63) of the slab as int8 lanes, unsigned codes for the offset formats.
template <int FMT>
__device__ inline void unpack_half(const Slab<FMT> &o, int h, uint32_t *w) {
  if (FMT == T_Q8_0) {
    #pragma unroll
    for (int i = 0; i < 8; i++) w[i] = o.L[8 * h + i];
    return;
  }
  if (FMT == T_Q6_K) {
    // values 0-15 | 16-31 come from the low nibbles of L[0..3] | L[4..7], 32-47 | 48-63 from the high nibbles
    #pragma unroll
    for (int i = 0; i < 4; i++) {
      if (h == 0) {
        w[i] = (o.L[i] & 0x0F0F0F0Fu) | ((o.H[i] & 0x03030303u) << 4);
        w[4 + i] = (o.L[4 + i] & 0x0F0F0F0Fu) | ((o.H[i] & 0x0C0C0C0Cu) << 2);
      } else {
        w[i] = ((o.L[i] >> 4) & 0x0F0F0F0Fu) | (o.H[i] & 0x30303030u);
        w[4 + i] = ((o.L[4 + i] >> 4) & 0x0F0F0F0Fu) | ((o.H[i] & 0xC0C0C0C0u) >> 2);
      }
    }
    return;
  }
  #pragma unroll
  for (int i = 0; i < 8; i++) w[i] = (o.L[i] >> (4 * h)) & 0x0F0F0F0Fu;
  if (FMT == T_Q5_0 || FMT == T_Q5_K) {
    #pragma unroll
    for (int i = 0; i < 8; i++) w[i] |= (((o.H[h] >> (4 * i)) & 15u) * 0x00204081u & 0x01010101u) << 4;
  }
}

// Token-independent factors of half h of a slab (exact products of f16 scales and integer codes):
//   Q8_0/Q4_0/Q5_0: a = d of the 32-block;  Q4_K/Q5_K: a = d*sc, b = dmin*mn;  Q6_K: a, b = d*scale of the two 16-groups
template <int FMT>
__device__ inline void half_scale(const Slab<FMT> &o, int h, double &fa, double &fb) {
  const double d0 = (double)h2f(o.dw & 0xffff), d1 = (double)h2f(o.dw >> 16);
  if (FMT == T_Q4_K || FMT == T_Q5_K) {
    fa = d0 * (double)((o.scw >> (8 * h)) & 0xff);
    fb = d1 * (double)((o.scw >> (16 + 8 * h)) & 0xff);
  } else if (FMT == T_Q6_K) {
    fa = d0 * (double)(int8_t)((o.scw >> (16 * h)) & 0xff);
    fb = d0 * (double)(int8_t)((o.scw >> (16 * h + 8)) & 0xff);
  } else {
    fa = h ? d1 : d0;
    fb = 0.0;
  }
}

// acc + the term of one 32-value block for one token, in the reference's rounding (src/compute/ref-kernels.js:132-277).
// X: the token's 32 int8 values; r: the block's activation scale and sums.
template <int FMT>
__device__ inline double block_term(const uint32_t *w, double fa, double fb, const uint32_t *X, const ActRec &r,
                                    double acc) {
  const double xd = r.d;
  if (FMT == T_Q6_K) {
    int g0 = 0, g1 = 0;
    #pragma unroll
    for (int i = 0; i < 4; i++) g0 = sdot4((int)w[i], (int)X[i], g0);
    #pragma unroll
    for (int i = 4; i < 8; i++) g1 = sdot4((int)w[i], (int)X[i], g1);
    g0 -= 32 * r.i[0];
    g1 -= 32 * r.i[1];
    // ((xd*d)*scale)*gsum: xd*d*scale is exact in any association, so it is (d*scale)*xd
    acc = acc + (fa * xd) * (double)g0;
    acc = acc + (fb * xd) * (double)g1;
    return acc;
  }
  int lo = 0;
  #pragma unroll
  for (int i = 0; i < 8; i++) lo = sdot4((int)w[i], (int)X[i], lo);
  if (FMT == T_Q8_0) return acc + ((double)lo * fa) * xd;
  if (FMT == T_Q4_0) return acc + ((double)(lo - 8 * r.i[0]) * fa) * xd;
  if (FMT == T_Q5_0) return acc + ((double)(lo - 16 * r.i[0]) * fa) * xd;
  // Q4_K / Q5_K: xd * (d*sc*sum(q*xq) - dmin*mn*sum(xq)); both products are exact, so their difference rounds once,
  // which one fma of the first product against the negated second computes
  return acc + xd * fma(fa, (double)lo, -(fb * r.s));
}

// ---------------------------------------------------------------------------------------------- kernel
// Rows of a launch: SwiGLU units are (gate row u, up row u) from segments 0 and 1; otherwise unit u is rows 2u, 2u+1
// of the segments laid end to end, whose planes are contiguous (one allocation), so every row is addressed from
// segment 0's planes.
template <int FMT, int MT, int EPI>
__global__ __launch_bounds__(GV_THREADS) void k_gemv(const GemvArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = a.lpr, slots = 64 / lpr, slot = lane / lpr, j = lane % lpr;
  const int nunits = EPI == EPI_SWIGLU ? a.rows_total : (a.rows_total + 1) / 2;
  const int upb = GV_WAVES * slots;  // row pairs per block per step
  const int nslab = a.nslab, K = nslab * 64, nsb = K >> 5;
  if (blockIdx.x * upb >= nunits) return;
  const Planes P0 = planes_of<FMT>(a.seg[0].m, a.rows_total);
  const Planes P1 = EPI == EPI_SWIGLU ? planes_of<FMT>(a.seg[1].m, a.rows_total) : P0;
  // global row of row r (0, 1) of the unit at ub (clamped: units past the end compute a duplicate and store nothing)
  auto unit_row = [&](int ub, int r) -> int {
    const int u = min(ub + wave * slots + slot, nunits - 1);
    return EPI == EPI_SWIGLU ? u : min(2 * u + r, a.rows_total - 1);
  };
  const uint8_t *X = lds;
  const ActRec *REC = (const ActRec *)(lds + act_rec_off(MT, K));

  // The lane's work is a flat sequence of items (unit step, slab): spl = nslab / lpr slabs of each of the block's
  // unit steps. Loads run two items ahead, across unit boundaries; a unit's butterfly and epilogue follow its last item.
  const int spl = (nslab + lpr - 1) / lpr;  // the last round may leave lanes without a slab (they add nothing)
  const int stride = gridDim.x * upb, ub0 = blockIdx.x * upb;
  const int total = (nunits - ub0 + stride - 1) / stride * spl;
  auto load_item = [&](int step, int m, Slab<FMT> &o0, Slab<FMT> &o1) {
    const int ub = ub0 + step * stride, s = min(j + m * lpr, nslab - 1);
    load_slab<FMT>(P0, unit_row(ub, 0) * nslab + s, o0);
    load_slab<FMT>(P1, unit_row(ub, 1) * nslab + s, o1);
  };
  {
    const int t0 = 0, mt = a.M;  // one tile of M <= MT tokens per launch (the host launches one per tile)
    Slab<FMT> c0, c1, n0, n1, q0, q1;
    // items 0 and 1 are in flight during the staging
    load_item(0, 0, c0, c1);
    if (total > 1) load_item(spl > 1 ? 0 : 1, spl > 1 ? 1 : 0, n0, n1);
    if (a.xf) stage_f32<FMT, MT>(a, t0, mt, K, lds);
    else stage_act<FMT>(a.act, t0, mt, MT, K, lds);
    __syncthreads();
    double acc0[MT], acc1[MT];
    #pragma unroll
    for (int t = 0; t < MT; t++) { acc0[t] = 0.0; acc1[t] = 0.0; }
    int step = 0, m = 0;    // current item
    int step2 = 0, m2 = 2;  // item k + 2
    while (m2 >= spl) { m2 -= spl; step2++; }
    for (int k = 0; k < total; k++) {
      if (k + 2 < total) {
        load_item(step2, m2, q0, q1);
        if (++m2 == spl) { m2 = 0; step2++; }
      }
      const int s = j + m * lpr;
      const bool live = s < nslab;
      #pragma unroll
      for (int h = 0; h < 2; h++) {
        if (!live) break;
        uint32_t w0[8], w1[8];
        double fa0, fb0, fa1, fb1;
        unpack_half<FMT>(c0, h, w0); half_scale<FMT>(c0, h, fa0, fb0);
        unpack_half<FMT>(c1, h, w1); half_scale<FMT>(c1, h, fa1, fb1);
        #pragma unroll
        for (int t = 0; t < MT; t++) {
          const int tt = min(t, mt - 1);  // a short tile repeats its last token; those results are not stored
          uint32_t Xv[8];
          const uint4 *xp = (const uint4 *)X + ((tt * 2 + h) * 2) * nslab + s;
          const uint4 v0 = xp[0], v1 = xp[nslab];
          Xv[0] = v0.x; Xv[1] = v0.y; Xv[2] = v0.z; Xv[3] = v0.w; Xv[4] = v1.x; Xv[5] = v1.y; Xv[6] = v1.z; Xv[7] = v1.w;
          const ActRec r = REC[(tt * 2 + h) * nslab + s];
          acc0[t] = block_term<FMT>(w0, fa0, fb0, Xv, r, acc0[t]);
          acc1[t] = block_term<FMT>(w1, fa1, fb1, Xv, r, acc1[t]);
        }
      }
      c0 = n0; c1 = n1;
      n0 = q0; n1 = q1;
      if (++m < spl) continue;
      // ---- last slab of this unit step: combine the lpr lanes and store
      #pragma unroll
      for (int t = 0; t < MT; t++) { acc0[t] = wave_sum_xor(acc0[t], lpr); acc1[t] = wave_sum_xor(acc1[t], lpr); }
      const int unit = ub0 + step * stride + wave * slots + slot;
      if (j == 0 && unit < nunits) {
        if (EPI == EPI_SWIGLU) {
          float *hb = a.hb + (long)t0 * a.ldh + unit;
          #pragma unroll
          for (int t = 0; t < MT; t++) {
            const double g = (double)(float)acc0[t], uu = (double)(float)acc1[t];
            const double silu = g / (1.0 + exp(-g));  // src/compute/ref-kernels.js:322
            if (t < mt) hb[(long)t * a.ldh] = (float)(silu * uu);
          }
        } else {
          #pragma unroll
          for (int r = 0; r < 2; r++) {
            int g = 2 * unit + r;
            if (g >= a.rows_total) break;
            float *out;
            const float *bias = nullptr;
            long ldo;
            if (EPI == EPI_RESID) {
              out = a.resid + (long)t0 * a.ldr + g;
              ldo = a.ldr;
            } else {
              // segment of the row, selected field by field (no dynamic indexing into the argument block)
              int si = 0;
              if (a.nseg > 1 && g >= a.seg[0].rows) { g -= a.seg[0].rows; si = 1; }
              if (si == 1 && a.nseg > 2 && g >= a.seg[1].rows) { g -= a.seg[1].rows; si = 2; }
              out = si == 0 ? a.seg[0].out : si == 1 ? a.seg[1].out : a.seg[2].out;
              bias = si == 0 ? a.seg[0].bias : si == 1 ? a.seg[1].bias : a.seg[2].bias;
              ldo = si == 0 ? a.seg[0].ldo : si == 1 ? a.seg[1].ldo : a.seg[2].ldo;
              out += (long)t0 * ldo + g;
            }
            const double bv = bias ? (double)bias[g] : 0.0;
            #pragma unroll
            for (int t = 0; t < MT; t++) {
              if (t >= mt) break;
              const float y = (float)(r ? acc1[t] : acc0[t]);
              float *o = out + (long)t * ldo;
              if (EPI == EPI_RESID) *o = (float)((double)*o + (double)y);
              else *o = bias ? (float)((double)y + bv) : y;
            }
          }
        }
      }
      #pragma unroll
      for (int t = 0; t < MT; t++) { acc0[t] = 0.0; acc1[t] = 0.0; }
      m = 0;
      step++;
    }
  }
}

// Float weights (F32/F16/BF16) use the f32 activation (src/compute/ref-kernels.js:278-299): one wave per row,
// sequential f64 sum per lane over a strided subset, then a butterfly.
template <int EPI>
__global__ __launch_bounds__(256) void k_gemv_float(const GemvArgs a, const float *__restrict__ xf, int ldx) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  const bool swig = EPI == EPI_SWIGLU;
  if (row >= a.rows_total) return;
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

// ---------------------------------------------------------------------------------------------- launch
static int g_cus = 0;

// Launch with a persistent grid: at most as many blocks as the GPU holds at once for this kernel and LDS size (the
// occupancy query is cached per LDS size), each block striding over row pairs.
template <int FMT, int MT, int EPI>
static void launch_gemv_k(const GemvArgs &a, int blocks, size_t lds, hipStream_t st) {
  static size_t attr = 64 * 1024;  // dynamic LDS above 64 KB must be requested per kernel
  static std::map<size_t, int> occ;
  const void *fn = (const void *)k_gemv<FMT, MT, EPI>;
  if (lds > attr) {
    ZL_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)GV_LDS_MAX));
    attr = GV_LDS_MAX;
  }
  auto it = occ.find(lds);
  if (it == occ.end()) {
    int n = 0;
    ZL_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, GV_THREADS, lds));
    it = occ.emplace(lds, std::max(1, n)).first;
  }
  blocks = std::min(blocks, g_cus * it->second);
  hipLaunchKernelGGL((k_gemv<FMT, MT, EPI>), dim3(blocks), dim3(GV_THREADS), lds, st, a);
}

template <int FMT, int MT>
static void launch_gemv_fmt(const GemvArgs &a, int epi, int blocks, size_t lds, hipStream_t st) {
  if (epi == EPI_STORE) launch_gemv_k<FMT, MT, EPI_STORE>(a, blocks, lds, st);
  else if (epi == EPI_RESID) launch_gemv_k<FMT, MT, EPI_RESID>(a, blocks, lds, st);
  else launch_gemv_k<FMT, MT, EPI_SWIGLU>(a, blocks, lds, st);
}

template <int MT>
static void launch_gemv_mt(int fmt, const GemvArgs &a, int epi, int blocks, size_t lds, hipStream_t st) {
  switch (fmt) {
    case T_Q8_0: launch_gemv_fmt<T_Q8_0, MT>(a, epi, blocks, lds, st); break;
    case T_Q4_0: launch_gemv_fmt<T_Q4_0, MT>(a, epi, blocks, lds, st); break;
    case T_Q5_0: launch_gemv_fmt<T_Q5_0, MT>(a, epi, blocks, lds, st); break;
    case T_Q4_K: launch_gemv_fmt<T_Q4_K, MT>(a, epi, blocks, lds, st); break;
    case T_Q5_K: launch_gemv_fmt<T_Q5_K, MT>(a, epi, blocks, lds, st); break;
    case T_Q6_K: launch_gemv_fmt<T_Q6_K, MT>(a, epi, blocks, lds, st); break;
    default: throw Error(ZL_ERR_UNSUPPORTED, "gemv: unsupported weight type");
  }
}

// Lanes per row pair: enough lanes in total to keep the GPU's memory pipes full (about 2^19 lanes), at most 64, at
// least 8 where the row has that many slabs, a power of two not above the row's slab count. Depends only on the
// matrix shape (rows of the launch, columns).
int gemv_lpr(int rows, int nslab) {
  int want = 8;
  while (want < 64 && (long)want * rows < (1L << 19)) want <<= 1;
  int cap = 1;  // the largest power of two not above nslab, at most 64
  while (cap < 64 && cap * 2 <= nslab) cap <<= 1;
  return want < cap ? want : cap;
}

void launch_gemv(const GemvArgs &a0, int epi, const float *xf, int ldx, hipStream_t st) {
  GemvArgs a = a0;
  const int fmt = a.seg[0].m.type;
  for (int i = 1; i < a.nseg; i++)
    ZL_REQUIRE(a.seg[i].m.type == fmt && a.seg[i].m.nslab == a.nslab, ZL_ERR_ARG, "gemv: segments differ in type or width");
  if (!is_quant(fmt)) {
    const int blocks = (a.rows_total + 3) / 4;
    if (epi == EPI_STORE) hipLaunchKernelGGL((k_gemv_float<EPI_STORE>), dim3(blocks), dim3(256), 0, st, a, xf, ldx);
    else if (epi == EPI_RESID) hipLaunchKernelGGL((k_gemv_float<EPI_RESID>), dim3(blocks), dim3(256), 0, st, a, xf, ldx);
    else hipLaunchKernelGGL((k_gemv_float<EPI_SWIGLU>), dim3(blocks), dim3(256), 0, st, a, xf, ldx);
    ZL_HIP(hipGetLastError());
    return;
  }
  ZL_REQUIRE(a.lpr >= 1 && a.lpr <= 64 && (a.lpr & (a.lpr - 1)) == 0 && a.lpr <= a.nslab, ZL_ERR_ARG, "gemv: bad lanes per row");
  if (epi != EPI_SWIGLU) {
    // the kernel addresses every row from segment 0's planes: the segments must be one allocation, end to end
    long r0 = 0;
    for (int i = 0; i < a.nseg; i++) {
      const MatView &m = a.seg[i].m, &b = a.seg[0].m;
      const long ns = r0 * a.nslab;
      const long nd = (fmt == T_Q4_K || fmt == T_Q5_K) ? r0 * (a.nslab / 4) * 2 : fmt == T_Q6_K ? r0 * (a.nslab / 4) : ns * 2;
      ZL_REQUIRE(m.qs == b.qs + ns * qs_bytes(fmt) && (!qx_bytes(fmt) || m.qx == b.qx + ns * qx_bytes(fmt)) &&
                 (!sc_bytes(fmt) || m.sc == b.sc + ns * sc_bytes(fmt)) && m.dd == b.dd + nd,
                 ZL_ERR_ARG, "gemv: grouped matrices must be contiguous");
      r0 += a.seg[i].rows;
    }
  }
  if (!g_cus) {
    int dev = 0;
    ZL_HIP(hipGetDevice(&dev));
    ZL_HIP(hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev));
  }
  const int K = a.nslab * 64;
  // token tile: exactly M up to 6, else 8 (a short last tile repeats its last token); smaller if the staged
  // activations would not fit the LDS budget
  int MT = a.M <= 6 ? a.M : 8;
  while (MT > 1 && gemv_lds_bytes(fmt, MT, K) > GV_LDS_MAX) MT = MT > 4 ? 4 : MT > 2 ? 2 : 1;
  const size_t lds = gemv_lds_bytes(fmt, MT, K);
  ZL_REQUIRE(lds <= GV_LDS_MAX, ZL_ERR_UNSUPPORTED, "gemv: row too long for the LDS-staged activations");
  const int slots = 64 / a.lpr;
  const int units = epi == EPI_SWIGLU ? a.rows_total : (a.rows_total + 1) / 2;
  const int upb = GV_WAVES * slots;
  int blocks = (units + upb - 1) / upb;
  a.wk = K;
  // one launch per tile of MT tokens: the tile's rows of every input and output are addressed from offset pointers
  const int M = a0.M;
  for (int t0 = 0; t0 < M; t0 += MT) {
    GemvArgs b = a;
    b.M = std::min(MT, M - t0);
    if (t0) {
      b.act.q += (long)t0 * a.act.ld;
      b.act.d += (long)t0 * (a.act.ld >> 5);
      b.act.s += (long)t0 * (a.act.ld >> 5);
      b.act.s16 += (long)t0 * (a.act.ld >> 4);
      b.xrow0 += t0;
      for (int i = 0; i < b.nseg; i++) if (b.seg[i].out) b.seg[i].out += (long)t0 * b.seg[i].ldo;
      if (b.resid) b.resid += (long)t0 * b.ldr;
      if (b.hb) b.hb += (long)t0 * b.ldh;
    }
    switch (MT) {
      case 1: launch_gemv_mt<1>(fmt, b, epi, blocks, lds, st); break;
      case 2: launch_gemv_mt<2>(fmt, b, epi, blocks, lds, st); break;
      case 3: launch_gemv_mt<3>(fmt, b, epi, blocks, lds, st); break;
      case 4: launch_gemv_mt<4>(fmt, b, epi, blocks, lds, st); break;
      case 5: launch_gemv_mt<5>(fmt, b, epi, blocks, lds, st); break;
      case 6: launch_gemv_mt<6>(fmt, b, epi, blocks, lds, st); break;
      default: launch_gemv_mt<8>(fmt, b, epi, blocks, lds, st); break;
    }
    ZL_HIP(hipGetLastError());
  }
}

}  // namespace zl
