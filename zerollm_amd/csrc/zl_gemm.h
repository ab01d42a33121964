// Quantised GEMM for 10..64 tokens (prefill chunks, wide verify passes), included by the per-format zl_gemm_*.hip
// files. Every weight byte is read once per launch for all the launch's tokens, as the reference's batched kernels read
// each weight tile once for every token of a chunk (src/compute/wasm/kernels.js:127-240,
// src/compute/wasm/kquant-kernels.js:337-504); the int8 block dots run on the matrix cores and the f64 block terms are
// the reference's (src/compute/ref-kernels.js:132-277), per (row, token) in exactly the order of k_gemv_tiles
// (zl_gemv.h): the same slabs per wave, slab by slab, block 0 then block 1 (Q6_K: its four 16-value groups in order),
// the same halving tree over the waves and the same K parts. A token therefore gets the same bits whatever the size of
// the pass it is in (1..9 tokens through the GEMV kernels, 10..64 here).
//
// Mapping. The workgroup is the GEMV's (K part, 64-row tile) with its W waves (gate/up pairs: W / 2 per matrix); wave
// wl of a matrix walks slabs s0 + wl + WH i as in k_gemv_tiles, but for every token of the launch at once. One
// v_mfma_i32_16x16x64_i8 multiplies A (16 tokens: lane l supplies token l mod 16's values of the slab's value quarter
// g = l / 16) by B (16 rows of the tile: lane l supplies row l mod 16's values of quarter g) into D[token][row]; lane l
// receives tokens 4 g + v (v = 0..3) of row l mod 16. To keep one 32-value block (Q6_K: one 16-value group) per dot, A
// holds the token's values only in the quarters of that block and zeros elsewhere: two MFMAs per (16 tokens, 16 rows)
// and slab (Q6_K: four). The B operands are built from the row-layout planes (lane l reads row 16 j + l mod 16's
// 16-byte part of quarter g and the scale words), so no second copy of the weights is needed.
//
// Accumulators. Lane l holds acc[j][u][v] = the running f64 sum of row 16 j + l mod 16 (j = 0..3 row groups of the
// tile) and token 16 u + 4 g + v (u = 0..U-1 token groups): 16 U doubles. Its f64 factors (Q4_K/Q5_K d*sc and dmin*mn
// of the two blocks, Q6_K d*scale of the four groups, Q8_0 the two block scales) are formed per slab for its four rows.
//
// Activations. Per round i (slabs s0 + WH i + wl of every wave wl of a matrix) the workgroup stages the int8 values and
// block records of those WH slabs for all tokens in LDS ([wl][token][64 B], then [wl][token][32 B]), double-buffered:
// the next round's bytes are loaded into registers while the current round computes and stored to LDS after it, and
// one barrier per round hands the buffer over. (Direct global-to-LDS loads would make the compiler wait for every
// load in flight, the weights' included, before each LDS read.)
#pragma once
#include "zl_gemv.h"

namespace zl {

constexpr int GEMM_MAX_M = 64;   // tokens per launch at most (four groups of 16)

typedef int gm_i32x4 __attribute__((ext_vector_type(4)));

// One slab of one lane as loaded: for each row group j (row 16 j + lane mod 16 of the tile) the 16 bytes of value
// quarter g's plane part, the extra-bit word(s), the scale-code word and the super-block / block scale word.
template <int FMT>
struct GmRaw {
  static constexpr int HW = FMT == T_Q6_K ? 4 : FMT == T_Q5_K ? 1 : 0;
  uint32_t q[4][4];
  uint32_t h[4][HW > 0 ? HW : 1];
  uint32_t sc[4];
  uint32_t dw[4];
};

template <int FMT>
__device__ __forceinline__ void gm_load(const Rsrc &R, int ts, int sbi, int n16, int g, bool valid, GmRaw<FMT> &o) {
  const int oob = valid ? 0 : 0x40000000;
  ts = valid ? ts : 0;
  sbi = valid ? sbi : 0;
  #pragma unroll
  for (int j = 0; j < 4; j++) {
    const int r = 16 * j + n16;
    u32x4 v;
    if constexpr (FMT == T_Q8_0) {
      // part g (values 16 g .. 16 g + 15) of row r is 16-byte unit 64 g + r of the tile-slab
      v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.qs, oob + (g * 64 + r) * 16, ts * 4096, 0));
    } else {
      // 4-bit planes: part (g & 1) holds the low nibbles of values 16 (g & 1) .. + 15 and the high nibbles 32 later
      v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.qs, oob + ((g & 1) * 64 + r) * 16, ts * 2048, 0));
    }
    o.q[j][0] = v.x; o.q[j][1] = v.y; o.q[j][2] = v.z; o.q[j][3] = v.w;
    if constexpr (FMT == T_Q6_K) {
      const u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.qx, oob + r * 16, ts * 1024, 0));
      o.h[j][0] = x.x; o.h[j][1] = x.y; o.h[j][2] = x.z; o.h[j][3] = x.w;
    } else if constexpr (FMT == T_Q5_K) {
      o.h[j][0] = __builtin_amdgcn_raw_buffer_load_b32(R.qx, oob + r * 8 + 4 * (g >> 1), ts * 512, 0);
    }
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q6_K) o.sc[j] = __builtin_amdgcn_raw_buffer_load_b32(R.sc, oob + r * 4, ts * 256, 0);
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) o.dw[j] = __builtin_amdgcn_raw_buffer_load_b32(R.dd, oob + r * 4, sbi * 256, 0);
    else if constexpr (FMT == T_Q6_K) o.dw[j] = __builtin_amdgcn_raw_buffer_load_b16(R.dd, oob + r * 2, sbi * 128, 0);
    else o.dw[j] = __builtin_amdgcn_raw_buffer_load_b32(R.dd, oob + r * 4, ts * 256, 0);
  }
}

// B operands (the 16 values of quarter g of the lane's four rows, as int8) and the exact f64 factors of the rows:
//   Q8_0 f = {d0, d1};  Q4_K/Q5_K f = {d*sc0, d*sc1, dmin*mn0, dmin*mn1};  Q6_K f = {d*scale of groups 0..3}.
// The products are those k_gemv_tiles forms (zl_gemv.h unpack), so every term below is bit for bit its term.
template <int FMT>
__device__ __forceinline__ void gm_unpack(const GmRaw<FMT> &o, int g, gm_i32x4 B[4], double f[4][4]) {
  #pragma unroll
  for (int j = 0; j < 4; j++) {
    #pragma unroll
    for (int k = 0; k < 4; k++) {
      uint32_t w = o.q[j][k];
      if constexpr (FMT != T_Q8_0) w = (w >> (4 * (g >> 1))) & 0x0F0F0F0Fu;
      if constexpr (FMT == T_Q5_K) {
        // bit 16 (g & 1) + 4 k + i of the word is the fifth bit of byte i of this dword
        w |= ((((o.h[j][0] >> (16 * (g & 1) + 4 * k)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
      }
      if constexpr (FMT == T_Q6_K) w |= ((o.h[j][k] >> (2 * g)) & 0x03030303u) << 4;  // top two bits of value 16 g + byte
      B[j][k] = (int)w;
    }
    const double d0 = (double)h2f((uint16_t)(o.dw[j] & 0xffff)), d1 = (double)h2f((uint16_t)(o.dw[j] >> 16));
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
      f[j][0] = d0 * (double)(o.sc[j] & 0xff);
      f[j][1] = d0 * (double)((o.sc[j] >> 8) & 0xff);
      f[j][2] = d1 * (double)((o.sc[j] >> 16) & 0xff);
      f[j][3] = d1 * (double)((o.sc[j] >> 24) & 0xff);
    } else if constexpr (FMT == T_Q6_K) {
      #pragma unroll
      for (int k = 0; k < 4; k++) f[j][k] = d0 * (double)(int8_t)((o.sc[j] >> (8 * k)) & 0xff);
    } else {
      f[j][0] = d0; f[j][1] = d1; f[j][2] = 0.0; f[j][3] = 0.0;
    }
  }
}

template <int FMT, int EPI, int W, int U>
__global__ __launch_bounds__(W * 64) void k_gemm(const GemvArgs a) {
  extern __shared__ __align__(16) uint8_t xl[];
  constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;
  constexpr int WH = NR == 2 ? W / 2 : W;                 // waves per matrix
  constexpr int DEPTH = U <= 2 ? 2 : 1;                   // slabs of weights in flight beyond the one computed
  constexpr int MP = 16 * U;                               // staged tokens (the last group padded with the last token)
  constexpr int RB = WH * MP * 96;                         // LDS bytes of one round: values, then records
  constexpr int CH = RB / 1024;                            // 1 KB staging chunks per round
  constexpr int SPW = (CH + W - 1) / W;                    // staging loads per wave and round
  constexpr int NG = FMT == T_Q6_K ? 4 : 2;                // dots per slab: 16-value groups or 32-value blocks
  static_assert(RB % 1024 == 0, "whole staging chunks");
  const int kp = blockIdx.x, tile = blockIdx.y;
  // token group z of the launch's G (blockIdx.z): tokens tb .. tb + Ml - 1, staged as rows 0 .. MP - 1. A (row, token)
  // sum does not depend on which workgroup holds the token, so the groups only spread a small matrix over more CUs.
  const int zg = blockIdx.z, G = gridDim.z, tb = zg * MP, Ml = min(MP, a.M - tb);
  const int lane = threadIdx.x & 63, n16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = NR == 2 ? __builtin_amdgcn_readfirstlane(wave / WH) : 0;
  const int wl = wave - grp * WH;
  const int ks = a.ks, M = Ml;  // this group's tokens
  const int si = __builtin_amdgcn_readfirstlane(
      EPI == EPI_SWIGLU ? 0 : (a.nseg > 2 && tile >= a.seg[2].tile0) ? 2 : (a.nseg > 1 && tile >= a.seg[1].tile0) ? 1 : 0);
#define ZL_SEG(f) (si == 0 ? a.seg[0].f : si == 1 ? a.seg[1].f : a.seg[2].f)
  const int lt = tile - ZL_SEG(tile0), rows = ZL_SEG(rows);
  const int nslab = a.nslab, nsb = nslab >> 2;
  const Rsrc R0 = {make_rsrc(ZL_SEG(m.qs), ZL_SEG(nqs)), make_rsrc(ZL_SEG(m.qx), ZL_SEG(nqx)), make_rsrc(ZL_SEG(m.sc), ZL_SEG(nsc)),
                   make_rsrc(ZL_SEG(m.dd), ZL_SEG(ndd))};
  const Rsrc R1 = NR == 2 ? Rsrc{make_rsrc(a.seg[1].m.qs, a.seg[1].nqs), make_rsrc(a.seg[1].m.qx, a.seg[1].nqx),
                                 make_rsrc(a.seg[1].m.sc, a.seg[1].nsc), make_rsrc(a.seg[1].m.dd, a.seg[1].ndd)}
                          : R0;
  const Rsrc R = grp == 0 ? R0 : R1;
  const int kr = a.kr, s0 = kp * kr, s1 = min(nslab, s0 + kr), nsl = s1 - s0;
  const int n = nsl > wl ? (nsl - wl + WH - 1) / WH : 0;  // this wave's slabs: s0 + wl + WH i, i < n
  const int nr = (nsl + WH - 1) / WH;                      // rounds (the most slabs a wave of the workgroup has)
  const uint8_t *xq = (const uint8_t *)a.act.q;
  const uint8_t *xr = (const uint8_t *)(FMT == T_Q6_K ? (const void *)a.act.rb : (const void *)a.act.ra);
  const long ldq = a.act.ld, ldr = (long)(a.act.ld >> 5) * 16;

  // ---- staging of round r into buffer r & 1 (chunk c of the round is LDS bytes [1024 c, 1024 c + 1024) of the
  // buffer), through registers: the loads are issued at the start of the previous round and the LDS stores follow its
  // compute, so the compiler's load counters track them exactly and the weight loads in flight are never waited for
  auto stage_load = [&](int r, u32x4 *sg) {
    #pragma unroll
    for (int k = 0; k < SPW; k++) {
      const int c = min(wave + W * k, CH - 1);  // surplus loads repeat the last chunk (the same bytes)
      const bool isv = c < WH * U;
      const int o = (isv ? c : c - WH * U) * 1024 + lane * 16;
      const int per = isv ? MP * 64 : MP * 32, rb = isv ? 64 : 32;
      const int w_ = o / per, rem = o - w_ * per, t = min(rem / rb, M - 1), e = rem % rb;
      const int s = min(s0 + w_ + WH * r, nslab - 1);  // rounds past the last one read a slab in range (unused)
      sg[k] = *(const u32x4 *)(isv ? xq + (long)(tb + t) * ldq + (long)s * 64 + e : xr + (long)(tb + t) * ldr + (long)s * 32 + e);
    }
  };
  auto stage_store = [&](int r, const u32x4 *sg) {
    uint8_t *buf = xl + (r & 1) * RB;
    #pragma unroll
    for (int k = 0; k < SPW; k++) {
      const int c = min(wave + W * k, CH - 1);
      *(u32x4 *)(buf + c * 1024 + lane * 16) = sg[k];
    }
  };

  double acc[4][U][4];
  #pragma unroll
  for (int j = 0; j < 4; j++)
    #pragma unroll
    for (int u = 0; u < U; u++)
      #pragma unroll
      for (int v = 0; v < 4; v++) acc[j][u][v] = 0.0;

  auto load = [&](int i, GmRaw<FMT> &b) {
    const int s = s0 + wl + WH * i;
    gm_load<FMT>(R, lt * nslab + s, lt * nsb + (s >> 2), n16, g, i < n, b);
  };
  GmRaw<FMT> ring[DEPTH];
  {
    u32x4 sg[SPW];
    stage_load(0, sg);
    #pragma unroll
    for (int d = 0; d < DEPTH; d++) load(d, ring[d]);
    stage_store(0, sg);
    __syncthreads();
  }

  // one round: the wave's slab r (weights in `slot`, activations in buffer r & 1), the next round's activations staged
  auto round = [&](int r, GmRaw<FMT> &slot) {
    gm_i32x4 B[4];
    double f[4][4];
    gm_unpack<FMT>(slot, g, B, f);
    // the operands are formed here, before the slot is reloaded (not sunk to their uses below), so the reload can
    // land in the slot's own registers
    #pragma unroll
    for (int j = 0; j < 4; j++) {
      asm volatile("" : "+v"(B[j]));
      #pragma unroll
      for (int k = 0; k < (FMT == T_Q8_0 ? 2 : 4); k++) asm volatile("" : "+v"(f[j][k]));
    }
    u32x4 sg[SPW];
    __builtin_amdgcn_sched_barrier(0);  // issue order: the staging loads, then the weights (the stores below wait for
    stage_load(r + 1, sg);              // the former only)
    __builtin_amdgcn_sched_barrier(0);
    load(r + DEPTH, slot);  // past the wave's last slab: no memory access
    __builtin_amdgcn_sched_barrier(0);
    if (r < n) {
      const uint8_t *buf = xl + (r & 1) * RB;
      const uint8_t *vals = buf + wl * MP * 64, *recs = buf + WH * MP * 64 + wl * MP * 32;
      #pragma unroll
      for (int u = 0; u < U; u++) {
        const uint4 av = *(const uint4 *)(vals + (16 * u + n16) * 64 + 16 * g);
        #pragma unroll
        for (int b = 0; b < NG; b++) {
          const bool on = (NG == 2 ? (g >> 1) : g) == b;  // this lane's quarter lies in block / group b
          const gm_i32x4 A = on ? gm_i32x4{(int)av.x, (int)av.y, (int)av.z, (int)av.w} : gm_i32x4{0, 0, 0, 0};
          gm_i32x4 D[4];
          #pragma unroll
          for (int j = 0; j < 4; j++) D[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B[j], gm_i32x4{0, 0, 0, 0}, 0, 0, 0);
          const int blk = NG == 2 ? b : b >> 1;
          #pragma unroll
          for (int v = 0; v < 4; v++) {
            const uint4 rc = *(const uint4 *)(recs + (16 * u + 4 * g + v) * 32 + blk * 16);
            const double xd = dbl(rc.x, rc.y);
            #pragma unroll
            for (int j = 0; j < 4; j++) {
              double &s = acc[j][u][v];
              if constexpr (FMT == T_Q6_K) {
                const int c = D[j][v] - (int)((b & 1) ? rc.w : rc.z);  // dot minus 32 x the group's activation sum
                s = fma(f[j][b] * (double)c, xd, s);
              } else if constexpr (FMT == T_Q8_0) {
                s = fma((double)D[j][v] * f[j][b], xd, s);
              } else {
                s = fma(xd, fma(f[j][b], (double)D[j][v], -(f[j][2 + b] * dbl(rc.z, rc.w))), s);
              }
            }
          }
        }
      }
    }
    stage_store(r + 1, sg);  // buffer (r + 1) & 1 was last read in round r - 1, before the previous barrier
    __syncthreads();
  };
  // whole groups of DEPTH rounds (a round past the last only stages and loads unused bytes), so each slot of the ring
  // keeps its registers from one iteration to the next
  for (int r = 0; r < nr; r += DEPTH) {
    round(r, ring[0]);
    if constexpr (DEPTH == 2) round(r + 1, ring[1]);
  }

  // ---- per token group: each wave parks its sums, then the wave of token t adds that token's sums over the waves of
  // each matrix in the order of a halving tree (as k_gemv_tiles) and runs the epilogue (or stores a K part)
  double *red = (double *)xl;  // [W][4 j][4 v][64 lanes] of one token group
  const int PW = NR * MP * 64;  // doubles per K part
  double *pp = a.part + (((long)tile * G + zg) * ks + kp) * PW;
  const int row = lt * 64 + lane;
  const bool live = row < rows;
  auto epilogue = [&](int t, double g0, double u0) {
    if constexpr (EPI == EPI_SWIGLU) {
      const double gv = (double)(float)g0, uu = (double)(float)u0;
      const float hv = live ? (float)(gv / (1.0 + exp(-gv)) * uu) : 0.f;  // src/compute/ref-kernels.js:322
      if (live) a.hb[(long)t * a.ldh + row] = hv;
      if (a.qout.q) quant_block32(hv, row, a.qout, t);
    } else if constexpr (EPI == EPI_RESID) {
      const double y = (double)(float)g0;
      if (live) {
        float *o = a.resid + (long)t * a.ldr + row;
        *o = (float)((double)*o + y);
      }
    } else {
      const float y = (float)g0;
      if (live) {
        const float *bias = ZL_SEG(bias);
        ZL_SEG(out)[(long)t * ZL_SEG(ldo) + row] = bias ? (float)((double)y + (double)bias[row]) : y;
      }
    }
  };
  #pragma unroll
  for (int u = 0; u < U; u++) {
    #pragma unroll
    for (int j = 0; j < 4; j++)
      #pragma unroll
      for (int v = 0; v < 4; v++) red[((wave * 4 + j) * 4 + v) * 64 + lane] = acc[j][u][v];
    __syncthreads();
    for (int tt = wave; tt < 16; tt += W) {
      const int t = 16 * u + tt;
      if (t >= M) break;
      // (row = lane, token t): row group lane / 16 in lane 16 (tt / 4) + lane mod 16, slot v = tt mod 4
      const int src = 16 * (tt >> 2) + n16, jv = (lane >> 4) * 4 + (tt & 3);
      double sums[NR];
      #pragma unroll
      for (int r = 0; r < NR; r++) {
        double vv[8];
        #pragma unroll
        for (int w = 0; w < 8; w++) vv[w] = red[(((r * WH + min(w, WH - 1)) * 16) + jv) * 64 + src];
        #pragma unroll
        for (int half = 4; half >= 1; half >>= 1)
          if (2 * half <= WH) {
            #pragma unroll
            for (int w = 0; w < half; w++) vv[w] = vv[w] + vv[w + half];
          }
        sums[r] = vv[0];
      }
      if (ks == 1) {
        epilogue(tb + t, sums[0], sums[NR - 1]);
      } else {
        #pragma unroll
        for (int r = 0; r < NR; r++) __hip_atomic_store(pp + (r * MP + t) * 64 + lane, sums[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
  }
  if (ks == 1) return;

  // ---- K parts: the last part of the tile to arrive adds all parts' sums in part order (as k_gemv_tiles)
  __shared__ uint32_t last;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  uint32_t *cnt = a.cnt + (long)tile * G + zg;
  if (threadIdx.x == 0) last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(ks - 1);
  __syncthreads();
  if (!last) return;
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int t = wave; t < M; t += W) {
    double sums[NR];
    #pragma unroll
    for (int r = 0; r < NR; r++) {
      const double *pt = a.part + ((long)tile * G + zg) * ks * PW + (r * MP + t) * 64 + lane;
      constexpr int KSMAX = 8;  // the parts' loads of one sum are issued together
      double pv[KSMAX];
      #pragma unroll
      for (int k = 0; k < KSMAX; k++) pv[k] = __hip_atomic_load(pt + (long)min(k, ks - 1) * PW, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      double v = pv[0];
      #pragma unroll
      for (int k = 1; k < KSMAX; k++)
        if (k < ks) v += pv[k];
      sums[r] = v;
    }
    epilogue(tb + t, sums[0], sums[NR - 1]);
  }
#undef ZL_SEG
}

// LDS bytes of a launch: two staging rounds, or the sums of one token group.
template <int W, int U>
constexpr size_t gemm_lds(bool swiglu) {
  return std::max((size_t)2 * (swiglu ? W / 2 : W) * 16 * U * 96, (size_t)W * 16 * 64 * 8);
}

template <int FMT, int EPI, int W, int U>
inline void launch_gemm_k(const GemvArgs &a, int G, hipStream_t st) {
  const size_t lds = gemm_lds<W, U>(EPI == EPI_SWIGLU);
  static bool done = false;
  if (!done) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_gemm<FMT, EPI, W, U>, hipFuncAttributeMaxDynamicSharedMemorySize, 112 * 1024));
    done = true;
  }
  hipLaunchKernelGGL((k_gemm<FMT, EPI, W, U>), dim3((unsigned)a.ks, (unsigned)a.ntiles, (unsigned)G), dim3(W * 64), lds, st, a);
}

template <int FMT, int EPI, int W>
inline void launch_gemm_w(const GemvArgs &a, hipStream_t st) {
  int U, G;
  gemm_groups(a, U, G);
  ZL_REQUIRE(a.ks == 1 || (long)a.ntiles * G <= GEMV_CNT_TILES, ZL_ERR_ARG, "gemm: too many split-K counters");
  switch (U) {
    case 1: launch_gemm_k<FMT, EPI, W, 1>(a, G, st); break;
    case 2: launch_gemm_k<FMT, EPI, W, 2>(a, G, st); break;
    case 3: launch_gemm_k<FMT, EPI, W, 3>(a, G, st); break;
    default: launch_gemm_k<FMT, EPI, W, 4>(a, G, st); break;
  }
}

template <int FMT>
void launch_gemm_fmt(const GemvArgs &a, int epi, hipStream_t st) {
  ZL_REQUIRE(a.M >= 1 && a.M <= GEMM_MAX_M && (a.nwave == 4 || a.nwave == 8) && (epi != EPI_SWIGLU || a.nwave == 8) &&
                 a.ks >= 1 && a.ks <= 8 && !a.xf && a.kr >= 1,
             ZL_ERR_ARG, "gemm: launch shape out of range");
  if (epi == EPI_SWIGLU) {
    launch_gemm_w<FMT, EPI_SWIGLU, 8>(a, st);
  } else if (epi == EPI_RESID) {
    if (a.nwave == 4) launch_gemm_w<FMT, EPI_RESID, 4>(a, st);
    else launch_gemm_w<FMT, EPI_RESID, 8>(a, st);
  } else {
    if (a.nwave == 4) launch_gemm_w<FMT, EPI_STORE, 4>(a, st);
    else launch_gemm_w<FMT, EPI_STORE, 8>(a, st);
  }
}

}  // namespace zl
