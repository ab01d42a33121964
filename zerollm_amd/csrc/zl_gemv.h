// Quantised GEMV for M = 1..9 tokens on gfx950 (included by the per-format zl_gemv_*.hip files):
// y[t][r] = sum over the row's 32-value blocks of the reference's block term (src/compute/ref-kernels.js:127-277):
// exact int8 block dots (v_dot4_i32_i8), f64 scale combination.
//
// Mapping. A wave owns one 64-row tile, one row per lane, and walks slabs (64 values) of the K range its workgroup
// holds: wave w of the workgroup's W waves takes slabs s0 + w, s0 + w + W, ... The weights' 16-byte planes are
// contiguous per tile-slab, so each vector load of the wave reads 1 KB without gaps. Every lane of the wave needs the
// same activation values: the workgroup stages its slab range of the M tokens' int8 values and block records in LDS
// once (those loads are issued before the weight loads, so they are not queued behind them). Per token and slab the
// loop reads the 64 values as one 4-byte word per lane (word k on lane k of each 16-lane row) and the dots take word k
// from lane k of the row by a DPP broadcast; the block records are broadcast LDS loads. No cross-lane reduction in the
// loop. The waves' f64 sums meet in LDS (added in a fixed tree order); with ks > 1 K parts per tile the parts' sums go
// through `part` and the last part to arrive adds them in part order. Every summation order depends only on the matrix shape, never on M, so a batched
// pass gives the same bits as token-by-token passes. Raw slabs are loaded DEPTH slabs ahead of the one computed.
#pragma once
#include "zl_kernels.h"

namespace zl {

constexpr int GT_NMAX = 16;          // slabs per wave at most (the slab loop is unrolled that far)

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
constexpr int GT_KR_MAX = 96;        // slabs per K part at most (staged activations: M x 96 x 96 bytes of LDS)
constexpr int GT_REC = 96;           // LDS bytes per (token, slab): 64 int8 values, then the two blocks' records

template <int FMT>
struct Fmt {
  static constexpr int QW = FMT == T_Q8_0 ? 16 : 8;                                          // qs words per (row, slab)
  static constexpr int HW = FMT == T_Q6_K ? 4 : (FMT == T_Q5_0 || FMT == T_Q5_K) ? 2 : 0;    // qx words
  static constexpr bool SC = FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q6_K;                // scale-code plane
};

// One (row, slab) as loaded.
template <int FMT>
struct Raw {
  uint32_t q[Fmt<FMT>::QW];
  uint32_t h[Fmt<FMT>::HW > 0 ? Fmt<FMT>::HW : 1];
  uint32_t sc, dw;
};

// Buffer resources of one matrix's planes: loads take the lane's byte offset (VGPR, loop invariant) and the
// tile-slab's (SGPR).
struct Rsrc {
  __amdgpu_buffer_rsrc_t qs, qx, sc, dd;
};
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)bytes, 0x00020000);
}

// Load tile-slab ts (super-block index sbi = tile * nslab / 4 + slab / 4 for the K-quants' dd plane). With valid
// false the lane offsets are moved past every plane (planes are below 1 GB): the buffer range check then returns zeros
// without a memory access, so a pipeline can issue its loads unconditionally.
template <int FMT>
__device__ inline void raw_load(const Rsrc &R, int ts, int sbi, int lane, bool valid, Raw<FMT> &o) {
  constexpr int QP = Fmt<FMT>::QW / 4;
  const int oob = valid ? 0 : 0x40000000;
  ts = valid ? ts : 0;
  sbi = valid ? sbi : 0;
  #pragma unroll
  for (int p = 0; p < QP; p++) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.qs, oob + lane * 16, (ts * QP + p) * 1024, 0));
    o.q[4 * p] = v.x; o.q[4 * p + 1] = v.y; o.q[4 * p + 2] = v.z; o.q[4 * p + 3] = v.w;
  }
  if constexpr (Fmt<FMT>::HW == 2) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(R.qx, oob + lane * 8, ts * 512, 0));
    o.h[0] = v.x; o.h[1] = v.y;
  }
  if constexpr (Fmt<FMT>::HW == 4) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.qx, oob + lane * 16, ts * 1024, 0));
    o.h[0] = v.x; o.h[1] = v.y; o.h[2] = v.z; o.h[3] = v.w;
  }
  if constexpr (Fmt<FMT>::SC) o.sc = __builtin_amdgcn_raw_buffer_load_b32(R.sc, oob + lane * 4, ts * 256, 0);
  if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) o.dw = __builtin_amdgcn_raw_buffer_load_b32(R.dd, oob + lane * 4, sbi * 256, 0);
  else if constexpr (FMT == T_Q6_K) o.dw = __builtin_amdgcn_raw_buffer_load_b16(R.dd, oob + lane * 2, sbi * 128, 0);
  else o.dw = __builtin_amdgcn_raw_buffer_load_b32(R.dd, oob + lane * 4, ts * 256, 0);
}

// Token-independent data of one (row, slab): int8 lanes of the 64 values (words 0-7 block 0 = values 0-31, words
// 8-15 block 1; unsigned codes for the offset formats) and exact f64 factors per 32-value block h:
//   Q8_0/Q4_0/Q5_0: fa = d;  Q4_K/Q5_K: fa = d*sc, fb = dmin*mn;  Q6_K: fa, fb = d*scale of the block's 16-groups
template <int FMT>
struct Unp {
  uint32_t w[16];
  double fa[2], fb[2];
};

template <int FMT>
__device__ inline void unpack(const Raw<FMT> &o, Unp<FMT> &u) {
  if constexpr (FMT == T_Q8_0) {
    #pragma unroll
    for (int i = 0; i < 16; i++) u.w[i] = o.q[i];
  } else if constexpr (FMT == T_Q6_K) {
    // block 0: values 0-15 | 16-31 from the low nibbles of q[0..3] | q[4..7]; block 1 from the high nibbles; the top
    // two bits of value j + 16k are bits 2k..2k+1 of qx byte j
    #pragma unroll
    for (int i = 0; i < 4; i++) {
      u.w[i] = (o.q[i] & 0x0F0F0F0Fu) | ((o.h[i] & 0x03030303u) << 4);
      u.w[4 + i] = (o.q[4 + i] & 0x0F0F0F0Fu) | ((o.h[i] & 0x0C0C0C0Cu) << 2);
      u.w[8 + i] = ((o.q[i] >> 4) & 0x0F0F0F0Fu) | (o.h[i] & 0x30303030u);
      u.w[12 + i] = ((o.q[4 + i] >> 4) & 0x0F0F0F0Fu) | ((o.h[i] & 0xC0C0C0C0u) >> 2);
    }
  } else {
    #pragma unroll
    for (int i = 0; i < 8; i++) {
      u.w[i] = o.q[i] & 0x0F0F0F0Fu;
      u.w[8 + i] = (o.q[i] >> 4) & 0x0F0F0F0Fu;
    }
    if constexpr (FMT == T_Q5_0 || FMT == T_Q5_K) {
      // bit j of h[b] is the fifth bit of value j of block b: spread 4 bits to the 4 bytes of a word
      #pragma unroll
      for (int b = 0; b < 2; b++) {
        #pragma unroll
        for (int i = 0; i < 8; i++) u.w[8 * b + i] |= ((((o.h[b] >> (4 * i)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
      }
    }
  }
  const double d0 = (double)h2f((uint16_t)(o.dw & 0xffff)), d1 = (double)h2f((uint16_t)(o.dw >> 16));
  if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
    #pragma unroll
    for (int h = 0; h < 2; h++) {
      u.fa[h] = d0 * (double)((o.sc >> (8 * h)) & 0xff);
      u.fb[h] = d1 * (double)((o.sc >> (16 + 8 * h)) & 0xff);
    }
  } else if constexpr (FMT == T_Q6_K) {
    #pragma unroll
    for (int h = 0; h < 2; h++) {
      u.fa[h] = d0 * (double)(int8_t)((o.sc >> (16 * h)) & 0xff);
      u.fb[h] = d0 * (double)(int8_t)((o.sc >> (16 * h + 8)) & 0xff);
    }
  } else {
    u.fa[0] = d0; u.fa[1] = d1;
    u.fb[0] = 0.0; u.fb[1] = 0.0;
  }
}

__device__ inline double dbl(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(double, (unsigned long long)lo | ((unsigned long long)hi << 32));
}

// The 16 int8 dots of one token's slab, in accumulation chains (c[j] += dot4(activation word k, w[k]) for the words k
// of chain j, back to back). The activation words are spread over each 16-lane row of the wave (lane k of every row
// holds word k), and each dot takes its word from lane k of the row by a DPP row broadcast, so the wave reads a token's
// slab from LDS once, 4 bytes per lane, instead of every lane reading all 64 bytes. Wait states: a DPP instruction
// needs two after a VALU write of a register it reads (the leading s_nop covers writes before the block), and a VALU
// read of a dot's result needs two after the dot (measured on gfx950: with one, the last dot's sum is not yet there;
// the trailing s_nop). A dot reading the previous dot's sum as its accumulator needs none.
//   ORDER 0 (32-value blocks):           c0 words 0-7, c1 words 8-15 (c2, c3 unused)
//   ORDER 1 (16-value groups, Q6_K):     c0 words 0-3, c1 4-7, c2 8-11, c3 12-15
#define ZL_DOT(c, k) "v_dot4c_i32_i8_dpp %" #c ", %[x], %[w" #k "] row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n\t"
#define ZL_WORDS                                                                                                      \
  [w0] "v"(w[0]), [w1] "v"(w[1]), [w2] "v"(w[2]), [w3] "v"(w[3]), [w4] "v"(w[4]), [w5] "v"(w[5]), [w6] "v"(w[6]), \
      [w7] "v"(w[7]), [w8] "v"(w[8]), [w9] "v"(w[9]), [w10] "v"(w[10]), [w11] "v"(w[11]), [w12] "v"(w[12]),       \
      [w13] "v"(w[13]), [w14] "v"(w[14]), [w15] "v"(w[15]), [x] "v"(xw)
template <int ORDER>
__device__ inline void slab_dots(uint32_t xw, const uint32_t *w, int c[4]) {
  if constexpr (ORDER == 0) {
    asm("s_nop 1\n\t"
        ZL_DOT(0, 0) ZL_DOT(0, 1) ZL_DOT(0, 2) ZL_DOT(0, 3) ZL_DOT(0, 4) ZL_DOT(0, 5) ZL_DOT(0, 6) ZL_DOT(0, 7)
        ZL_DOT(1, 8) ZL_DOT(1, 9) ZL_DOT(1, 10) ZL_DOT(1, 11) ZL_DOT(1, 12) ZL_DOT(1, 13) ZL_DOT(1, 14) ZL_DOT(1, 15)
        "s_nop 1"
        : "+v"(c[0]), "+v"(c[1])
        : ZL_WORDS);
  } else {
    asm("s_nop 1\n\t"
        ZL_DOT(0, 0) ZL_DOT(0, 1) ZL_DOT(0, 2) ZL_DOT(0, 3) ZL_DOT(1, 4) ZL_DOT(1, 5) ZL_DOT(1, 6) ZL_DOT(1, 7)
        ZL_DOT(2, 8) ZL_DOT(2, 9) ZL_DOT(2, 10) ZL_DOT(2, 11) ZL_DOT(3, 12) ZL_DOT(3, 13) ZL_DOT(3, 14) ZL_DOT(3, 15)
        "s_nop 1"
        : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3])
        : ZL_WORDS);
  }
}
#undef ZL_DOT
#undef ZL_WORDS

// acc + the terms of the slab's two 32-value blocks (block 0, then block 1) for one token. xw: the token's 64 int8
// values of the slab, word k on lane k of every 16-lane row; R0, R1: the blocks' records (uniform). In the reference's
// arithmetic up to where f64 rounds:
//   Q8_0 (s*d)*xd;  Q4_0/Q5_0 ((s - 8|16 sum) * d) * xd;  Q4_K/Q5_K xd*(d*sc*s - dmin*mn*sum);
//   Q6_K per 16-group (d*scale*(s - 32 sum)) * xd.  The products before the last one are exact; the last multiply
//   and the accumulation are one fma. The integer dots are exact in any order.
template <int FMT>
__device__ inline double slab_terms(const Unp<FMT> &u, uint32_t xw, const u32x4 &R0, const u32x4 &R1, double acc) {
  const double xd0 = dbl(R0[0], R0[1]), xd1 = dbl(R1[0], R1[1]);
  if constexpr (FMT == T_Q6_K) {
    int c[4] = {-(int)R0[2], -(int)R0[3], -(int)R1[2], -(int)R1[3]};
    slab_dots<1>(xw, u.w, c);
    acc = fma(u.fa[0] * (double)c[0], xd0, acc);
    acc = fma(u.fb[0] * (double)c[1], xd0, acc);
    acc = fma(u.fa[1] * (double)c[2], xd1, acc);
    return fma(u.fb[1] * (double)c[3], xd1, acc);
  } else {
    constexpr int CI = FMT == T_Q4_0 ? 2 : 3;  // Q4_0 / Q5_0: the block starts at -8 | -16 x its activation sum
    const bool off = FMT == T_Q4_0 || FMT == T_Q5_0;
    int c[4] = {off ? -(int)R0[CI] : 0, off ? -(int)R1[CI] : 0, 0, 0};
    slab_dots<0>(xw, u.w, c);
    const int lo0 = c[0], lo1 = c[1];
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
      acc = fma(xd0, fma(u.fa[0], (double)lo0, -(u.fb[0] * dbl(R0[2], R0[3]))), acc);
      return fma(xd1, fma(u.fa[1], (double)lo1, -(u.fb[1] * dbl(R1[2], R1[3]))), acc);
    } else {
      acc = fma((double)lo0 * u.fa[0], xd0, acc);
      return fma((double)lo1 * u.fa[1], xd1, acc);
    }
  }
}

// Record array of the format family.
template <int FMT>
__device__ inline const void *recs_of(const Act &a) {
  if constexpr (FMT == T_Q6_K) return a.rb;
  else if constexpr (FMT == T_Q4_0 || FMT == T_Q5_0) return a.rc;
  else return a.ra;
}

// The workgroup (kp, tile) of a launch: K part kp of 64-row tile `tile`; xl is the launch's dynamic LDS. Written as a
// device function so that one kernel can hold two launches of different formats side by side (k_gemv_mix).
template <int FMT, int MT, int EPI, int DEPTH>
__device__ __forceinline__ void gemv_tiles_body(const GemvArgs a, const int kp, const int tile, uint8_t *xl) {
  constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;  // matrices per output row: gate and up for SwiGLU
  // staged activations, per token: [nsl][64] int8 values, then [nsl][32] records; after the slab loop the same bytes
  // hold the waves' sums for the reduction ([W][MT][64] doubles)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = a.nwave;  // waves of the workgroup (1, 2, 4, 8 or 16)
  // SwiGLU: the first half of the waves computes the gate rows, the second half the up rows, each half walking the
  // slabs as a workgroup of W / 2 waves computing one matrix would (so the sums are the same bits)
  const int WH = NR == 2 ? W >> 1 : W;
  const int grp = NR == 2 ? __builtin_amdgcn_readfirstlane(wave / WH) : 0;
  const int wl = wave - grp * WH;
  const int ks = a.ks;
  // segment of the tile, selected field by field (no dynamic indexing into the argument block)
  const int si = __builtin_amdgcn_readfirstlane(
      EPI != EPI_STORE ? 0 : (a.nseg > 2 && tile >= a.seg[2].tile0) ? 2 : (a.nseg > 1 && tile >= a.seg[1].tile0) ? 1 : 0);
#define ZL_SEG(f) (si == 0 ? a.seg[0].f : si == 1 ? a.seg[1].f : a.seg[2].f)
  const int lt = tile - ZL_SEG(tile0), rows = ZL_SEG(rows);
  const int nslab = a.nslab, nsb = nslab >> 2;
  const Rsrc R0 = {make_rsrc(ZL_SEG(m.qs), ZL_SEG(nqs)), make_rsrc(ZL_SEG(m.qx), ZL_SEG(nqx)), make_rsrc(ZL_SEG(m.sc), ZL_SEG(nsc)),
                   make_rsrc(ZL_SEG(m.dd), ZL_SEG(ndd))};
  const Rsrc R1 = NR == 2 ? Rsrc{make_rsrc(a.seg[1].m.qs, a.seg[1].nqs), make_rsrc(a.seg[1].m.qx, a.seg[1].nqx),
                                 make_rsrc(a.seg[1].m.sc, a.seg[1].nsc), make_rsrc(a.seg[1].m.dd, a.seg[1].ndd)}
                          : R0;
  const int kr = a.kr, s0 = kp * kr, s1 = min(nslab, s0 + kr), nsl = s1 - s0;
  const int n = nsl > wl ? (nsl - wl + WH - 1) / WH : 0;  // this wave's slabs: s0 + wl + WH i, i < n <= GT_NMAX
  const int M = a.M;
  const uint8_t *xq = (const uint8_t *)a.act.q, *xr = (const uint8_t *)recs_of<FMT>(a.act);
  const long ldq = a.act.ld, ldr = (long)(a.act.ld >> 5) * 16;

  const Rsrc R = grp == 0 ? R0 : R1;
  double acc[MT];
  #pragma unroll
  for (int t = 0; t < MT; t++) acc[t] = 0.0;
  Raw<FMT> buf[DEPTH];
  auto load = [&](int i, Raw<FMT> &b) {
    const int s = s0 + wl + WH * i;
    const int ts = lt * nslab + s, sbi = lt * nsb + (s >> 2);
    raw_load<FMT>(R, ts, sbi, lane, i < n, b);
  };
  #pragma unroll
  for (int d = 0; d < DEPTH; d++) load(d, buf[d]);
  if (a.xf) {
    // ---- fused prologue: RMSNorm scale per token (groups of 4 waves, each in k_norm_quant's order), then quantise the
    // slab range of every token into LDS in the staged layout
    __shared__ double ssr[4][4];
    __shared__ double scl[GEMV_MAX_MT];
    const int groups = W >> 2, g = wave >> 2;
    // one token, one K part, rows of at most 1024 values: the values this thread quantises (elements e = tid,
    // tid + 64 W, e < 1024) are among the four it loads for the sum of squares (x[tid mod 256 + 256 k], k = e / 256),
    // and their norm weights are requested with them, so the quantisation waits for no load
    const bool own = M == 1 && s0 == 0 && a.n <= 1024 && a.nw && nsl * 64 <= 2 * W * 64;
    float xo[4], wo[2];
    if (own) {
      const int tt = threadIdx.x & 255;
      const float *xr = a.xf + (long)a.xrow0 * a.ldxf;
      #pragma unroll
      for (int k = 0; k < 4; k++) { const int i = tt + 256 * k; xo[k] = xr[i < a.n ? i : 0]; }
      #pragma unroll
      for (int q = 0; q < 2; q++) { const int e = threadIdx.x + q * W * 64; wo[q] = a.nw[e < a.n ? e : 0]; }
      double ss = 0.0;  // rms_scale256's order
      #pragma unroll
      for (int k = 0; k < 4; k++) { const double x = tt + 256 * k < a.n ? (double)xo[k] : 0.0; ss += x * x; }
      const double sc = rms_finish(ss, a.n, a.eps, tt, ssr[g & 3]);
      if (threadIdx.x == 0) scl[0] = sc;
      __syncthreads();
    } else {
      for (int t0 = 0; t0 < M; t0 += groups) {
        const int t = t0 + g;
        const bool act_ = t < M;
        double sc = 1.0;
        if (a.nw) {
          // rms_scale256 synchronises the block: every thread takes part, idle groups with a dummy row
          const float *xr = a.xf + (long)(a.xrow0 + (act_ ? t : 0)) * a.ldxf;
          sc = rms_scale256(xr, a.n, a.eps, (int)threadIdx.x & 255, ssr[g & 3]);
        }
        if (act_ && (threadIdx.x & 255) == 0) scl[t] = sc;
        __syncthreads();
      }
    }
    const int per = nsl * 64;  // values of one token in the range (a multiple of 64: each wave holds whole blocks)
    for (int e = threadIdx.x; e < M * per; e += W * 64) {
      const int t = e / per, j = e - t * per, col = s0 * 64 + j;
      float v = 0.f;
      if (col < a.n) {
        if (own) {
          v = (float)((double)xo[e >> 8] * scl[0] * (double)wo[e >= W * 64 ? 1 : 0]);
        } else {
          const float xv = a.xf[(long)(a.xrow0 + t) * a.ldxf + col];
          v = a.nw ? (float)((double)xv * scl[t] * (double)a.nw[col]) : xv;
        }
      }
      const QBlock b = quant32(v);
      uint8_t *tb = xl + t * nsl * GT_REC;
      tb[j] = (uint8_t)(int8_t)b.q;
      if ((j & 31) == 0) *(uint4 *)(tb + nsl * 64 + (j >> 5) * 16) = block_record<FMT>(b);
    }
  } else {
    // ---- stage the activations of the workgroup's slab range in LDS, after the first weight loads: per token its
    // nsl * 64 int8 values, then its nsl * 32 record bytes, copied in 1 KB chunks by direct global-to-LDS loads (lane
    // l moves bytes 16l..16l+15 of a chunk), one chunk per wave at a time
    const int xb = nsl * 64, rb = nsl * 32, xc = (xb + 1023) >> 10, rc = (rb + 1023) >> 10, per = xc + rc;
    for (int c = wave; c < M * per; c += W) {
      const int t = c / per, k = c - t * per;
      const bool isx = k < xc;
      const int kk = isx ? k : k - xc, off = kk * 1024 + lane * 16;
      const uint8_t *src = (isx ? xq + t * ldq + s0 * 64 : xr + t * ldr + s0 * 32) + off;
      uint8_t *dst = xl + t * nsl * GT_REC + (isx ? 0 : xb) + kk * 1024;
      if (off < (isx ? xb : rb))
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                         (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
    }
  }
  // the residual value of this lane's row for the wave's first token, requested now rather than after the reduction
  // (and the K parts' hand-off), where its latency would follow the kernel's last step
  float rres = 0.f;
  if constexpr (EPI == EPI_RESID) rres = a.resid[(long)min(wave, M - 1) * a.ldr + min(lt * 64 + lane, rows - 1)];
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged bytes are in LDS
  __syncthreads();
  // fully unrolled over the most slabs a wave can hold (no loop-carried registers: each slot's reload lands in the
  // registers it was loaded into, and the waits count exactly the loads still needed)
  #pragma unroll
  for (int i0 = 0; i0 < GT_NMAX; i0 += DEPTH) {
    if (i0 >= n) break;
    #pragma unroll
    for (int d = 0; d < DEPTH; d++) {
      const int i = i0 + d;
      if (i >= GT_NMAX) break;
      Unp<FMT> u;
      unpack<FMT>(buf[d], u);
      // the slot is reloaded only after it has been unpacked (the reload reuses its registers, no copies)
      __builtin_amdgcn_sched_barrier(0);
      load(i + DEPTH, buf[d]);  // past the wave's last slab: no memory access
      if (i < n) {
        const int sl = wl + WH * i;  // slab within the workgroup's range
        #pragma unroll
        for (int t = 0; t < MT; t++) {
          const int tt = MT == 1 ? 0 : min(t, M - 1);  // a short token tile repeats its last token (not stored)
          const uint8_t *tb = xl + tt * nsl * GT_REC;
          const uint32_t xw = ((const uint32_t *)(tb + sl * 64))[lane & 15];
          const uint4 *rp = (const uint4 *)(tb + nsl * 64 + sl * 32);
          const uint4 r0 = rp[0], r1 = rp[1];
          acc[t] = slab_terms<FMT>(u, xw, u32x4{r0.x, r0.y, r0.z, r0.w}, u32x4{r1.x, r1.y, r1.z, r1.w}, acc[t]);
        }
      }
    }
  }

  // ---- each matrix's sum over its WH waves in the order of a halving tree (at each level wave w + half is added onto
  // wave w): every wave parks its sums in LDS once, then the wave of token t adds that token's sums in that order
  __syncthreads();  // every wave is past its last read of the staged activations, which the sums overwrite
  double *red = (double *)xl;
  #pragma unroll
  for (int t = 0; t < MT; t++) red[(wave * MT + t) * 64 + lane] = acc[t];
  __syncthreads();
  auto tree = [&](int r, int t) {
    double v[16];
    #pragma unroll
    for (int w = 0; w < 16; w++) v[w] = red[((r * WH + min(w, WH - 1)) * MT + t) * 64 + lane];  // all loads issued at once
    #pragma unroll
    for (int half = 8; half >= 1; half >>= 1)
      if (2 * half <= WH) {
        #pragma unroll
        for (int w = 0; w < half; w++) v[w] = v[w] + v[w + half];
      }
    return v[0];
  };

  // ---- K parts: the last part of the tile to arrive adds all parts' sums in part order. Partial sums are written and
  // read with device-scope (agent) atomic accesses, which are coherent across the XCDs' L2 caches without cache-wide
  // fences; each wave waits for its stores to complete before the workgroup counts itself in.
  constexpr int PW = NR * MT * 64;  // doubles per part
  if (ks > 1) {
    __shared__ uint32_t last;
    double *pp = a.part + ((long)tile * ks + kp) * PW;
    for (int t = wave; t < M; t += W) {
      #pragma unroll
      for (int r = 0; r < NR; r++) __hip_atomic_store(pp + (r * MT + t) * 64 + lane, tree(r, t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0) last = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(ks - 1);
    __syncthreads();
    if (!last) return;
    if (threadIdx.x == 0) __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  auto total = [&](int r, int t) {
    if (ks == 1) return tree(r, t);
    const double *pt = a.part + (long)tile * ks * PW + (r * MT + t) * 64 + lane;
    constexpr int KSMAX = 8;  // the parts' loads of one sum are issued together
    double pv[KSMAX];
    #pragma unroll
    for (int k = 0; k < KSMAX; k++) pv[k] = __hip_atomic_load(pt + (long)min(k, ks - 1) * PW, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    double v = pv[0];
    #pragma unroll
    for (int k = 1; k < KSMAX; k++)
      if (k < ks) v += pv[k];
    return v;
  };

  // ---- epilogue of token t on wave t (t, t + W, ...): lane = row of the tile
  const int row = lt * 64 + lane;
  const bool live = row < rows;
  for (int t = wave; t < M; t += W) {
    if constexpr (EPI == EPI_SWIGLU) {
      const double g = (double)(float)total(0, t), uu = (double)(float)total(1, t);
      const float hv = live ? (float)(g / (1.0 + exp(-g)) * uu) : 0.f;  // src/compute/ref-kernels.js:322
      if (live) a.hb[(long)t * a.ldh + row] = hv;
      if (a.qout.q) quant_block32(hv, row, a.qout, t);
    } else if constexpr (EPI == EPI_RESID) {
      const double y = (double)(float)total(0, t);
      if (live) {
        float *o = a.resid + (long)t * a.ldr + row;
        *o = (float)((double)(t == wave ? rres : *o) + y);
      }
    } else {
      const float y = (float)total(0, t);
      if (live) {
        const float *bias = ZL_SEG(bias);
        ZL_SEG(out)[(long)t * ZL_SEG(ldo) + row] = bias ? (float)((double)y + (double)bias[row]) : y;
      }
    }
  }
#undef ZL_SEG
}

template <int FMT, int MT, int EPI, int DEPTH>
__global__ __launch_bounds__(1024) void k_gemv_tiles(const GemvArgs a) {
  extern __shared__ __align__(16) uint8_t xl[];
  gemv_tiles_body<FMT, MT, EPI, DEPTH>(a, blockIdx.x, blockIdx.y, xl);  // grid: (K parts, tiles)
}

template <auto K>
inline void allow_big_lds() {
  static bool done = false;  // dynamic LDS beyond 64 KB must be allowed per kernel (one flag per kernel), once
  if (!done) {
    ZL_HIP(hipFuncSetAttribute((const void *)K, hipFuncAttributeMaxDynamicSharedMemorySize, 112 * 1024));
    done = true;
  }
}

// Launch one chunk of at most GEMV_MAX_MT tokens: token tile MT = M (M = 7 runs as 8).
template <int FMT, int MT>
inline void launch_tiles_mt(const GemvArgs &a, int epi, hipStream_t st) {
  const int wpm = epi == EPI_SWIGLU ? a.nwave / 2 : a.nwave;  // waves per matrix
  ZL_REQUIRE(a.kr <= GT_KR_MAX && a.M <= MT && a.ks <= 8 && wpm >= 1 && a.nwave <= 16 &&
                 (epi != EPI_SWIGLU || (a.nwave % 2 == 0 && wpm <= 8)) && (a.kr + wpm - 1) / wpm <= GT_NMAX &&
                 (!a.xf || (a.nwave >= 4 && a.n <= a.nslab * 64)),
             ZL_ERR_ARG, "gemv: launch shape out of range");
  const dim3 grid((unsigned)a.ks, (unsigned)a.ntiles), blk((unsigned)a.nwave * 64);
  // [M][kr] staged records of 96 bytes, then (same bytes) the waves' sums
  const size_t lds = std::max((size_t)a.M * a.kr * GT_REC, (size_t)a.nwave * MT * 64 * 8);
  if (epi == EPI_STORE) {
    allow_big_lds<k_gemv_tiles<FMT, MT, EPI_STORE, 4>>();
    hipLaunchKernelGGL((k_gemv_tiles<FMT, MT, EPI_STORE, 4>), grid, blk, lds, st, a);
  } else if (epi == EPI_RESID) {
    allow_big_lds<k_gemv_tiles<FMT, MT, EPI_RESID, 4>>();
    hipLaunchKernelGGL((k_gemv_tiles<FMT, MT, EPI_RESID, 4>), grid, blk, lds, st, a);
  } else {
    allow_big_lds<k_gemv_tiles<FMT, MT, EPI_SWIGLU, 4>>();
    hipLaunchKernelGGL((k_gemv_tiles<FMT, MT, EPI_SWIGLU, 4>), grid, blk, lds, st, a);
  }
}

template <int FMT>
void launch_gemv_fmt(const GemvArgs &a, int epi, hipStream_t st) {
  switch (a.M) {
    case 1: launch_tiles_mt<FMT, 1>(a, epi, st); break;
    case 2: launch_tiles_mt<FMT, 2>(a, epi, st); break;
    case 3: launch_tiles_mt<FMT, 3>(a, epi, st); break;
    case 4: launch_tiles_mt<FMT, 4>(a, epi, st); break;
    case 5: launch_tiles_mt<FMT, 5>(a, epi, st); break;
    case 6: launch_tiles_mt<FMT, 6>(a, epi, st); break;
    case 7: case 8: launch_tiles_mt<FMT, 8>(a, epi, st); break;
    case 9: launch_tiles_mt<FMT, 9>(a, epi, st); break;
    default: throw Error(ZL_ERR_ARG, "gemv: bad token count");
  }
}

}  // namespace zl
