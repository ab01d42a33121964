// Q4_K and Q8_0 GEMVs for 2..9 tokens with the int8 block dots on the matrix cores (v_mfma_i32_16x16x64_i8), the same
// results bit for bit as k_gemv_tiles (zl_gemv.h): the same slabs per wave, the same f64 block terms per (row, token)
// in the same order (slab by slab, block 0 then block 1, in the reference's arithmetic, src/compute/ref-kernels.js:
// 132-152, 210-240), the same halving-tree reduction over the waves and the same K parts.
//
// One MFMA multiplies an activation fragment A (16 rows rho: token t's values of the slab's 32-value block b, zero
// elsewhere in the slab) by a weight fragment B (16 rows of the tile, the slab's 64 values) into D[rho][row]: the
// integer dot of every (token, block) with every row at once. Lane l supplies A row l mod 16 and B row l mod 16 for the
// value quarter l / 16 (16 bytes each), and receives D[4 (l / 16) + v][l mod 16], v = 0..3 (measured on gfx950). Row
// rho = 4 g + v holds token g (v = 0, 1) or token 4 + g (v = 2, 3), block v mod 2, so lane group g receives tokens g and
// 4 + g, both blocks. Terms of tokens past M are not formed: at 2..4 tokens elements 2 and 3 are skipped (8 block
// terms per lane and slab, not 16); at 5 tokens token 4 sits in lane group 0 of every row group's MFMA, and two
// v_permlane16_swap and one v_permlane32_swap gather row group j's into lane group j, which then holds its own row
// (10 terms per lane and slab). At 9 tokens a second A fragment carries token 8 in the place of token 4, multiplied by
// the same weight fragments and gathered the same way (18 terms per lane and slab). A tile-slab is four MFMAs (row
// groups j = 0..3; eight at 9 tokens). The weights come
// from a second copy of the matrix's 4-bit plane in that operand order (DevMat::fq: per tile-slab, half h holds row
// groups 2h and 2h + 1; lane L = n + 16 g of a half holds 8 bytes per group: the values 16 g .. 16 g + 15 of row
// 16 j + n, value e and e + 4 in the low and high nibble of byte e of each 4-byte word, so two masks and a shift give
// the operand's 16 bytes in value order). The scale codes and super-block scales are read from the row-layout planes,
// one row per lane as in k_gemv_tiles; each lane forms its row's four f64 factors once per slab and parks them in LDS,
// where the lanes of the other row groups read them. Q8_0 needs no second plane: its row-layout plane holds part p
// (values 16 p .. 16 p + 15) of row r at 16-byte unit 64 p + r of a tile-slab, so lane n + 16 g reads its operand bytes
// for row group j at unit 64 g + 16 j + n; the factors are the two block scales d.
#include "zl_gemv.h"

namespace zl {

// sums per lane: 4 row groups x 2 tokens, and token 8 at 9 tokens
constexpr int mf_slots(int mc) { return mc == 3 ? 9 : 8; }
// LDS bytes between two tokens' staged rows past their nsl * GT_REC bytes: a stride of 16 x an odd number of bytes
// modulo 256 puts the token rows that one A-fragment read takes (up to 8 in a 16-lane group) on disjoint banks, where
// a multiple of 256 (nsl a multiple of 8) put them all on the same four
constexpr int MF_TPAD = 16;

// MC: token class of the launch, 0 = 2..4 tokens, 1 = 5 tokens, 2 = 6..8 tokens, 3 = 9 tokens
template <int FMT, int EPI, int MC>
__device__ __forceinline__ void gemv_mfma_body(const GemvArgs a, const int kp, const int tile, uint8_t *xl) {
  static_assert(FMT == T_Q4_K || FMT == T_Q8_0, "matrix-core formats");
  constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;
  constexpr int DEPTH = FMT == T_Q4_K ? 4 : 3;  // Q8_0 slabs are 64 bytes per lane: three in flight
  constexpr int MF_SLOTS = mf_slots(MC);
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  // staged activations as in k_gemv_tiles; after the slab loop the same bytes hold the waves' sums ([W][8][64])
  __shared__ __align__(16) double fac[16][64][4];  // per wave: the factors of the tile's rows for one slab (Q4_K: fa0,
                                                   // fa1, fb0, fb1; Q8_0: d0, d1)
  const int lane = threadIdx.x & 63, n16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = a.nwave;
  const int WH = NR == 2 ? W >> 1 : W;
  const int grp = NR == 2 ? __builtin_amdgcn_readfirstlane(wave / WH) : 0;
  const int wl = wave - grp * WH;
  const int ks = a.ks;
  const int si = __builtin_amdgcn_readfirstlane(
      EPI != EPI_STORE ? 0 : (a.nseg > 2 && tile >= a.seg[2].tile0) ? 2 : (a.nseg > 1 && tile >= a.seg[1].tile0) ? 1 : 0);
#define ZL_SEG(f) (si == 0 ? a.seg[0].f : si == 1 ? a.seg[1].f : a.seg[2].f)
  const int lt = tile - ZL_SEG(tile0), rows = ZL_SEG(rows);
  const int nslab = a.nslab, nsb = nslab >> 2;
  // Q4_K: the fragment plane takes the place of the row-layout 4-bit plane (same size and per-tile-slab offsets); Q8_0:
  // the row-layout plane is already in operand order (part p of row r at 16-byte unit 64 p + r of the tile-slab)
  const Rsrc R0 = {make_rsrc(FMT == T_Q4_K ? ZL_SEG(m.fq) : ZL_SEG(m.qs), ZL_SEG(nqs)), make_rsrc(nullptr, 0),
                   make_rsrc(ZL_SEG(m.sc), ZL_SEG(nsc)), make_rsrc(ZL_SEG(m.dd), ZL_SEG(ndd))};
  const Rsrc R1 = NR == 2 ? Rsrc{make_rsrc(FMT == T_Q4_K ? a.seg[1].m.fq : a.seg[1].m.qs, a.seg[1].nqs), make_rsrc(nullptr, 0),
                                 make_rsrc(a.seg[1].m.sc, a.seg[1].nsc), make_rsrc(a.seg[1].m.dd, a.seg[1].ndd)}
                          : R0;
  const int kr = a.kr, s0 = kp * kr, s1 = min(nslab, s0 + kr), nsl = s1 - s0;
  const int ts = nsl * GT_REC + MF_TPAD;  // LDS bytes per token of the staged activations
  const int n = nsl > wl ? (nsl - wl + WH - 1) / WH : 0;
  const int M = a.M;
  const uint8_t *xq = (const uint8_t *)a.act.q, *xr = (const uint8_t *)a.act.ra;
  const long ldq = a.act.ld, ldr = (long)(a.act.ld >> 5) * 16;

  const Rsrc R = grp == 0 ? R0 : R1;
  double acc[4][2];
  #pragma unroll
  for (int j = 0; j < 4; j++) acc[j][0] = acc[j][1] = 0.0;
  Raw<FMT> buf[DEPTH];
  auto load = [&](int i, Raw<FMT> &b) {
    const int s = s0 + wl + WH * i;
    const int ts = lt * nslab + s, sbi = lt * nsb + (s >> 2);
    if constexpr (FMT == T_Q4_K) {
      raw_load<FMT>(R, ts, sbi, lane, i < n, b);
    } else {
      // Q8_0: q[4 j .. 4 j + 3] = part g of row 16 j + n16 (the B operand of row group j); dw = the two block scales of
      // row `lane` (its factors); past the wave's last slab the offsets leave the planes (zeros, no memory access)
      const int oob = i < n ? 0 : 0x40000000, tsv = i < n ? ts : 0;
      #pragma unroll
      for (int j = 0; j < 4; j++) {
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.qs, oob + (g * 64 + n16) * 16 + j * 256, tsv * 4096, 0));
        b.q[4 * j] = v.x; b.q[4 * j + 1] = v.y; b.q[4 * j + 2] = v.z; b.q[4 * j + 3] = v.w;
      }
      b.dw = __builtin_amdgcn_raw_buffer_load_b32(R.dd, oob + lane * 4, tsv * 256, 0);
    }
  };
  #pragma unroll
  for (int d = 0; d < DEPTH; d++) load(d, buf[d]);
  {
    // ---- stage the activations of the workgroup's slab range in LDS (as k_gemv_tiles does)
    const int xb = nsl * 64, rb = nsl * 32, xc = (xb + 1023) >> 10, rc = (rb + 1023) >> 10, per = xc + rc;
    for (int c = wave; c < M * per; c += W) {
      const int t = c / per, k = c - t * per;
      const bool isx = k < xc;
      const int kk = isx ? k : k - xc, off = kk * 1024 + lane * 16;
      const uint8_t *src = (isx ? xq + t * ldq + s0 * 64 : xr + t * ldr + s0 * 32) + off;
      uint8_t *dst = xl + t * ts + (isx ? 0 : xb) + kk * 1024;
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
  // A-fragment row rho = n16 of this lane: token n16 / 4 (n16 mod 4 < 2) or 4 + n16 / 4, block n16 & 1; its quarter g
  // holds values of that block
  const int at = (n16 & 2) ? 4 + (n16 >> 2) : (n16 >> 2);
  const bool avalid = at < M && (g >> 1) == (n16 & 1);
  const uint8_t *abase = xl + (avalid ? at : 0) * ts + 16 * g;
  // records of this lane's D elements: tokens g and 4 + g (a token past M repeats the last one; not stored)
  const int t0 = min(g, M - 1), t1 = min(4 + g, M - 1);
  const uint8_t *rb0 = xl + t0 * ts + nsl * 64, *rb1 = xl + t1 * ts + nsl * 64;
  // 9 tokens: the second fragment's row rho = n16 holds token 8 where n16 mod 16 is 2 or 3 (block n16 & 1), else zeros
  const bool avalid8 = MC == 3 && M > 8 && (n16 & 14) == 2 && (g >> 1) == (n16 & 1);
  const uint8_t *abase8 = xl + (avalid8 ? 8 : 0) * ts + 16 * g;
  const uint8_t *rb8 = xl + (MC == 3 && M > 8 ? 8 : 0) * ts + nsl * 64;
  double acc8 = 0.0;  // 9 tokens: (this lane's row 16 g + n16, token 8)
  double *fw = &fac[wave][0][0];
  #pragma unroll
  for (int i0 = 0; i0 < GT_NMAX; i0 += DEPTH) {
    if (i0 >= n) break;
    #pragma unroll
    for (int d = 0; d < DEPTH; d++) {
      const int i = i0 + d;
      if (i >= GT_NMAX) break;
      // this lane's row (16 g + n16 = lane): its factors, as k_gemv_tiles forms them
      const Raw<FMT> &o = buf[d];
      const double d0 = (double)h2f((uint16_t)(o.dw & 0xffff)), d1 = (double)h2f((uint16_t)(o.dw >> 16));
      double f4[4];
      if constexpr (FMT == T_Q4_K) {
        f4[0] = d0 * (double)(o.sc & 0xff); f4[1] = d0 * (double)((o.sc >> 8) & 0xff);
        f4[2] = d1 * (double)((o.sc >> 16) & 0xff); f4[3] = d1 * (double)((o.sc >> 24) & 0xff);
      } else {
        f4[0] = d0; f4[1] = d1; f4[2] = 0.0; f4[3] = 0.0;
      }
      constexpr int QN = FMT == T_Q4_K ? 8 : 16;
      uint32_t q[QN];
      #pragma unroll
      for (int k = 0; k < QN; k++) q[k] = o.q[k];
      __builtin_amdgcn_sched_barrier(0);
      load(i + DEPTH, buf[d]);  // past the wave's last slab: no memory access
      if (i < n) {
        const int sl = wl + WH * i;
        {  // the two 16-byte halves of a lane's 32-byte record swap places where (lane / 8) is odd, so lanes l and l + 8
           // of a 16-lane access meet no bank twice (the readers swizzle by their row the same way)
          double2 *fr = (double2 *)(fw + lane * 4);
          const int sw = (lane >> 3) & 1;
          fr[sw] = make_double2(f4[0], f4[1]);
          fr[sw ^ 1] = make_double2(f4[2], f4[3]);
        }
        const uint4 av = avalid ? *(const uint4 *)(abase + sl * 64) : make_uint4(0, 0, 0, 0);
        const i32x4 A = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
        const uint4 r00 = *(const uint4 *)(rb0 + sl * 32), r01 = *(const uint4 *)(rb0 + sl * 32 + 16);
        const uint4 r10 = *(const uint4 *)(rb1 + sl * 32), r11 = *(const uint4 *)(rb1 + sl * 32 + 16);
        // (xd, xs) of the elements v = 0..3: (token g, block 0), (g, 1), (4 + g, 0), (4 + g, 1)
        const double xd[4] = {dbl(r00.x, r00.y), dbl(r01.x, r01.y), dbl(r10.x, r10.y), dbl(r11.x, r11.y)};
        const double xs[4] = {dbl(r00.z, r00.w), dbl(r01.z, r01.w), dbl(r10.z, r10.w), dbl(r11.z, r11.w)};
        auto term = [&](double &acc1, double fa, double fb, double xdv, double xsv, int dv) {
          if constexpr (FMT == T_Q4_K) acc1 = fma(xdv, fma(fa, (double)dv, -(fb * xsv)), acc1);
          else acc1 = fma((double)dv * fa, xdv, acc1);  // Q8_0: (s * d) * xd
        };
        int d4[2][4];  // 5 tokens: token 4's elements (blocks 0, 1) of row group j, in lane group 0 (9 tokens: token 8's)
        i32x4 A8 = {0, 0, 0, 0};
        double xd8[2] = {0.0, 0.0}, xs8[2] = {0.0, 0.0};
        if constexpr (MC == 3) {
          const uint4 a8 = avalid8 ? *(const uint4 *)(abase8 + sl * 64) : make_uint4(0, 0, 0, 0);
          A8 = (i32x4){(int)a8.x, (int)a8.y, (int)a8.z, (int)a8.w};
          const uint4 r80 = *(const uint4 *)(rb8 + sl * 32), r81 = *(const uint4 *)(rb8 + sl * 32 + 16);
          xd8[0] = dbl(r80.x, r80.y); xd8[1] = dbl(r81.x, r81.y);
          xs8[0] = dbl(r80.z, r80.w); xs8[1] = dbl(r81.z, r81.w);
        }
        #pragma unroll
        for (int j = 0; j < 4; j++) {
          i32x4 B;
          if constexpr (FMT == T_Q4_K) {
            const uint32_t p0 = q[2 * j], p1 = q[2 * j + 1];
            B = (i32x4){(int)(p0 & 0x0F0F0F0Fu), (int)((p0 >> 4) & 0x0F0F0F0Fu), (int)(p1 & 0x0F0F0F0Fu),
                        (int)((p1 >> 4) & 0x0F0F0F0Fu)};
          } else {
            B = (i32x4){(int)q[4 * j], (int)q[4 * j + 1], (int)q[4 * j + 2], (int)q[4 * j + 3]};
          }
          const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, (i32x4){0, 0, 0, 0}, 0, 0, 0);
          const double2 *fr = (const double2 *)(fw + (16 * j + n16) * 4);  // row 16 j + n16: its factors
          const int sw = (n16 >> 3) & 1;                                    // (the writer's swizzle, by row)
          const double2 flo = fr[sw], fhi = fr[sw ^ 1];
          const double4 f = make_double4(flo.x, flo.y, fhi.x, fhi.y);
          #pragma unroll
          for (int v = 0; v < (MC >= 2 ? 4 : 2); v++) {
            const double fa = (v & 1) ? f.y : f.x, fb = (v & 1) ? f.w : f.z;
            term(acc[j][v >> 1], fa, fb, xd[v], xs[v], D[v]);
          }
          if constexpr (MC == 1) {
            d4[0][j] = D[2];
            d4[1][j] = D[3];
          }
          if constexpr (MC == 3) {
            const i32x4 D8 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A8, B, (i32x4){0, 0, 0, 0}, 0, 0, 0);
            d4[0][j] = D8[2];
            d4[1][j] = D8[3];
          }
        }
        if constexpr (MC == 1 || MC == 3) {
          // token 4 (token 8): row group j's from lane group 0 of MFMA j to lane group j, i.e. this lane's own row
          // 16 g + n16, whose factors it formed itself
          #pragma unroll
          for (int bk = 0; bk < 2; bk++) {
            const auto e01 = __builtin_amdgcn_permlane16_swap((unsigned)d4[bk][0], (unsigned)d4[bk][1], false, false);
            const auto e23 = __builtin_amdgcn_permlane16_swap((unsigned)d4[bk][2], (unsigned)d4[bk][3], false, false);
            const int c = (int)__builtin_amdgcn_permlane32_swap(e01[0], e23[0], false, false)[0];
            if constexpr (MC == 1) term(acc[0][1], f4[bk], f4[2 + bk], xd[2 + bk], xs[2 + bk], c);
            else term(acc8, f4[bk], f4[2 + bk], xd8[bk], xs8[bk], c);
          }
        }
      }
    }
  }

  // ---- sums over the WH waves of each matrix in the order of a halving tree; the wave of token t adds that token's
  __syncthreads();  // every wave is past its last read of the staged activations, which the sums overwrite
  double *red = (double *)xl;
  #pragma unroll
  for (int j = 0; j < 4; j++)
    #pragma unroll
    for (int tt = 0; tt < 2; tt++) red[(wave * MF_SLOTS + 2 * j + tt) * 64 + lane] = acc[j][tt];
  if constexpr (MC == 3) red[(wave * MF_SLOTS + 8) * 64 + lane] = acc8;
  __syncthreads();
  // (row = lane, token t) lives in lane 16 t + row mod 16, slot 2 (row / 16) for t < 4; for 4 <= t < 8 in lane
  // 16 (t - 4) + row mod 16, slot 2 (row / 16) + 1 (6..9 tokens), or in lane `row`, slot 1 (5 tokens: token 4); token 8
  // in lane `row`, slot 8
  auto tree = [&](int r, int t) {
    const int src = t < 4 ? 16 * t + n16 : (MC == 1 || t == 8) ? lane : 16 * (t - 4) + n16;
    const int slot = t < 4 ? 2 * (lane >> 4) : MC == 1 ? 1 : t == 8 ? 8 : 2 * (lane >> 4) + 1;
    double v[16];
    #pragma unroll
    for (int w = 0; w < 16; w++) v[w] = red[((r * WH + min(w, WH - 1)) * MF_SLOTS + slot) * 64 + src];
    #pragma unroll
    for (int half = 8; half >= 1; half >>= 1)
      if (2 * half <= WH) {
        #pragma unroll
        for (int w = 0; w < half; w++) v[w] = v[w] + v[w + half];
      }
    return v[0];
  };

  // ---- K parts (as k_gemv_tiles)
  constexpr int PW = NR * GEMV_MAX_MT * 64;
  if (ks > 1) {
    __shared__ uint32_t last;
    double *pp = a.part + ((long)tile * ks + kp) * PW;
    for (int t = wave; t < M; t += W) {
      #pragma unroll
      for (int r = 0; r < NR; r++) __hip_atomic_store(pp + (r * GEMV_MAX_MT + t) * 64 + lane, tree(r, t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    const double *pt = a.part + (long)tile * ks * PW + (r * GEMV_MAX_MT + t) * 64 + lane;
    constexpr int KSMAX = 8;
    double pv[KSMAX];
    #pragma unroll
    for (int k = 0; k < KSMAX; k++) pv[k] = __hip_atomic_load(pt + (long)min(k, ks - 1) * PW, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    double v = pv[0];
    #pragma unroll
    for (int k = 1; k < KSMAX; k++)
      if (k < ks) v += pv[k];
    return v;
  };

  // ---- epilogue of token t on wave t: lane = row of the tile (as k_gemv_tiles)
  const int row = lt * 64 + lane;
  const bool live = row < rows;
  for (int t = wave; t < M; t += W) {
    if constexpr (EPI == EPI_SWIGLU) {
      const double gv = (double)(float)total(0, t), uu = (double)(float)total(1, t);
      const float hv = live ? (float)(gv / (1.0 + exp(-gv)) * uu) : 0.f;  // src/compute/ref-kernels.js:322
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

// (9 tokens: at most 8 waves, so that the second fragment's sums stay in registers)
template <int FMT, int EPI, int MC>
__global__ __launch_bounds__(MC == 3 ? 512 : 1024) void k_gemv_mfma(const GemvArgs a) {
  extern __shared__ __align__(16) uint8_t xl[];
  gemv_mfma_body<FMT, EPI, MC>(a, blockIdx.x, blockIdx.y, xl);
}

// Two store launches reading the same activations in one kernel: a Q4_K launch on the matrix cores (a1) and a launch of
// another format on the VALU tiles (a2, token tile MT2), workgroups 0 .. a1.ks a1.ntiles - 1 for the first, the rest
// for the second, each exactly as its own launch would run it (the verify pass's attn_q + attn_k and attn_v: the v
// launch's workgroups no longer wait for a launch of their own). The launches' split-K work spaces are disjoint.
template <int FMT2, int MT2>
__global__ __launch_bounds__(MT2 == 9 ? 512 : 1024) void k_gemv_mix(const GemvArgs a1, const GemvArgs a2) {
  extern __shared__ __align__(16) uint8_t xl[];
  const int n1 = a1.ks * a1.ntiles, id = blockIdx.x;
  if (id < n1) gemv_mfma_body<T_Q4_K, EPI_STORE, MT2 <= 4 ? 0 : MT2 == 5 ? 1 : MT2 == 9 ? 3 : 2>(a1, id % a1.ks, id / a1.ks, xl);
  else gemv_tiles_body<FMT2, MT2, EPI_STORE, 4>(a2, (id - n1) % a2.ks, (id - n1) / a2.ks, xl);
}

// Q4_K matrices with their fragment plane, and Q8_0 matrices, at 2..9 tokens without a fused prologue.
bool gemv_mfma_ok(const GemvArgs &a) {
  const int t = a.seg[0].m.type;
  if ((t != T_Q4_K && t != T_Q8_0) || a.M < 2 || a.M > 9 || (a.M == 9 && a.nwave > 8) || a.xf) return false;
  for (int i = 0; i < a.nseg; i++)
    if (a.seg[i].m.type != t || (t == T_Q4_K && !a.seg[i].m.fq)) return false;
  return true;
}

template <int FMT, int MC>
static void launch_mfma_mc(const GemvArgs &a, int epi, dim3 grid, dim3 blk, size_t lds, hipStream_t st) {
  if (epi == EPI_STORE) {
    allow_big_lds<k_gemv_mfma<FMT, EPI_STORE, MC>>();
    hipLaunchKernelGGL((k_gemv_mfma<FMT, EPI_STORE, MC>), grid, blk, lds, st, a);
  } else if (epi == EPI_RESID) {
    allow_big_lds<k_gemv_mfma<FMT, EPI_RESID, MC>>();
    hipLaunchKernelGGL((k_gemv_mfma<FMT, EPI_RESID, MC>), grid, blk, lds, st, a);
  } else {
    allow_big_lds<k_gemv_mfma<FMT, EPI_SWIGLU, MC>>();
    hipLaunchKernelGGL((k_gemv_mfma<FMT, EPI_SWIGLU, MC>), grid, blk, lds, st, a);
  }
}

template <int FMT>
static void launch_mfma_fmt(const GemvArgs &a, int epi, dim3 grid, dim3 blk, size_t lds, hipStream_t st) {
  if (a.M <= 4) launch_mfma_mc<FMT, 0>(a, epi, grid, blk, lds, st);
  else if (a.M == 5) launch_mfma_mc<FMT, 1>(a, epi, grid, blk, lds, st);
  else if (a.M <= 8) launch_mfma_mc<FMT, 2>(a, epi, grid, blk, lds, st);
  else launch_mfma_mc<FMT, 3>(a, epi, grid, blk, lds, st);
}

void launch_gemv_mfma(const GemvArgs &a, int epi, hipStream_t st) {
  const int wpm = epi == EPI_SWIGLU ? a.nwave / 2 : a.nwave;
  ZL_REQUIRE(gemv_mfma_ok(a) && a.kr <= GT_KR_MAX && a.ks <= 8 && wpm >= 1 && a.nwave <= 16 &&
                 (epi != EPI_SWIGLU || (a.nwave % 2 == 0 && wpm <= 8)) && (a.kr + wpm - 1) / wpm <= GT_NMAX,
             ZL_ERR_ARG, "gemv (matrix cores): launch shape out of range");
  const dim3 grid((unsigned)a.ks, (unsigned)a.ntiles), blk((unsigned)a.nwave * 64);
  const size_t lds = std::max((size_t)a.M * (a.kr * GT_REC + MF_TPAD), (size_t)a.nwave * mf_slots(a.M == 9 ? 3 : 0) * 64 * 8);
  if (a.seg[0].m.type == T_Q4_K) launch_mfma_fmt<T_Q4_K>(a, epi, grid, blk, lds, st);
  else launch_mfma_fmt<T_Q8_0>(a, epi, grid, blk, lds, st);
}

// Whether launch_gemv_mix takes this pair: a1 on the matrix cores, a2 a Q6_K or Q8_0 store launch of the same tokens
// and workgroup size, neither with a fused prologue, one chunk of tokens.
bool gemv_mix_ok(const GemvArgs &a1, const GemvArgs &a2) {
  const int f2 = a2.seg[0].m.type;
  if (!gemv_mfma_ok(a1) || a1.seg[0].m.type != T_Q4_K || (f2 != T_Q6_K && f2 != T_Q8_0) || a1.xf || a2.xf ||
      a1.M != a2.M || a1.nwave != a2.nwave)
    return false;
  for (int i = 1; i < a2.nseg; i++)
    if (a2.seg[i].m.type != f2) return false;
  return a2.kr <= GT_KR_MAX && a2.ks <= 8 && (a2.kr + a2.nwave - 1) / a2.nwave <= GT_NMAX && a1.kr <= GT_KR_MAX &&
         a1.ks <= 8 && (a1.kr + a1.nwave - 1) / a1.nwave <= GT_NMAX && a1.nwave <= 16;
}

template <int FMT2, int MT2>
static void launch_mix_k(const GemvArgs &a1, const GemvArgs &a2, hipStream_t st) {
  const size_t l1 = std::max((size_t)a1.M * (a1.kr * GT_REC + MF_TPAD), (size_t)a1.nwave * mf_slots(MT2 == 9 ? 3 : 0) * 64 * 8);
  const size_t l2 = std::max((size_t)a2.M * a2.kr * GT_REC, (size_t)a2.nwave * MT2 * 64 * 8);
  allow_big_lds<k_gemv_mix<FMT2, MT2>>();
  const unsigned n = (unsigned)(a1.ks * a1.ntiles + a2.ks * a2.ntiles);
  hipLaunchKernelGGL((k_gemv_mix<FMT2, MT2>), dim3(n), dim3((unsigned)a1.nwave * 64), std::max(l1, l2), st, a1, a2);
}

template <int FMT2>
static void launch_mix_fmt(const GemvArgs &a1, const GemvArgs &a2, hipStream_t st) {
  switch (a1.M) {
    case 2: launch_mix_k<FMT2, 2>(a1, a2, st); break;
    case 3: launch_mix_k<FMT2, 3>(a1, a2, st); break;
    case 4: launch_mix_k<FMT2, 4>(a1, a2, st); break;
    case 5: launch_mix_k<FMT2, 5>(a1, a2, st); break;
    case 6: launch_mix_k<FMT2, 6>(a1, a2, st); break;
    case 9: launch_mix_k<FMT2, 9>(a1, a2, st); break;
    default: launch_mix_k<FMT2, 8>(a1, a2, st); break;  // 7 and 8 tokens (token tile 8, as the tile launch)
  }
}

void launch_gemv_mix(const GemvArgs &a1, const GemvArgs &a2, hipStream_t st) {
  ZL_REQUIRE(gemv_mix_ok(a1, a2), ZL_ERR_ARG, "gemv: launches cannot share a kernel");
  ZL_REQUIRE(a1.act.q && a1.act.ra && a1.act.rb && a1.act.rc && a2.act.q == a1.act.q, ZL_ERR_ARG, "gemv: activation records missing");
  ZL_REQUIRE((a1.ks == 1 || a1.part) && (a2.ks == 1 || a2.part), ZL_ERR_ARG, "gemv: split-K work space missing");
  if (a2.seg[0].m.type == T_Q6_K) launch_mix_fmt<T_Q6_K>(a1, a2, st);
  else launch_mix_fmt<T_Q8_0>(a1, a2, st);
  ZL_HIP(hipGetLastError());
}

}  // namespace zl
