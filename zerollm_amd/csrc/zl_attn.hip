// Causal GQA attention with the reference's arithmetic (src/model/forward.js:115-140; the gated form of
// src/model/forward-qwen35.js:71-105 when a.gate is set), in two launches per layer:
//   k_attn_scores  s_t = f32(sum_i q_i K_t,i (f64, exact products) * 1/sqrt(hd)) for every position t <= pos, one
//                  block per (64-position chunk, KV head, token): all of K streams in parallel.
//   k_attn_av      softmax over the scores (e = exp(s - max) in f64, stored f32; p = f32(e * (1/sum e))), then
//                  out_i = sum_t p_t V_t,i accumulated in f32 in position order, one block per (32-dim slice, query
//                  head, token); the head output is also quantised for the output projection.
// Scores live in a [token][head][ctx] f32 buffer between the two. The weighted sum keeps the reference's f32 rounding
// after every position: a random-weight network turns a 1e-7 change there into a visible logit difference.
#include "zl_kernels.h"
#include <algorithm>
#include <climits>

namespace zl {

// Query heads handled by one score block: the largest divisor of the GQA group that is at most 8.
inline int attn_heads_per_block(int group) {
  for (int c = 8; c > 1; c--)
    if (group % c == 0) return c;
  return 1;
}

// Score dots: every position's dot is split over HD / ATTN_VPL lanes of ATTN_VPL values each (an f64 fma chain per
// lane in value order, then an xor butterfly over the position's lanes); both attention forms use this order.
constexpr int ATTN_VPL = 32;
// Positions per score block chunk: 64, or one load round of 256 threads where that is more (HD = 64).
constexpr int attn_score_chunk(int hd) { return 256 / (hd / ATTN_VPL) > 64 ? 256 / (hd / ATTN_VPL) : 64; }

// Per-head RMSNorm (weights nw, when set) and RoPE at position pos of one head vector v[0..HD) in LDS, by one wave,
// with the arithmetic of src/model/forward.js:203-211 and src/compute/ref-kernels.js:305-310, 344-363 (64-lane strided
// f64 sum of squares and butterfly; f64 rotation of each (i, i + half) or (2i, 2i + 1) pair, stored f32).
template <int HD>
struct RopeVals {
  static constexpr int PR = (HD / 2 + 63) / 64;  // rotation pairs per lane at most
  static constexpr int NW = (HD + 63) / 64;      // norm weights per lane
  float cv[PR], sv[PR], wv[NW];
};

// The lane's norm weights (a read of the table when there is no norm: no branch around the loads) ...
template <int HD>
__device__ inline void rope_load_w(RopeVals<HD> &r, const float *nw, const float *cosT, int lane) {
  const float *nwp = nw ? nw : cosT;
  #pragma unroll
  for (int k = 0; k < RopeVals<HD>::NW; k++) r.wv[k] = nwp[lane + 64 * k < HD ? lane + 64 * k : 0];
}
// ... and its rotation table values at position pos.
template <int HD>
__device__ inline void rope_load_cs(RopeVals<HD> &r, int nRot, const float *cosT, const float *sinT, int pos, int lane) {
  const int half = nRot / 2;
  #pragma unroll
  for (int k = 0; k < RopeVals<HD>::PR; k++) {
    const int i = lane + 64 * k, ic = i < half ? i : 0;
    r.cv[k] = cosT[(long)pos * half + ic];
    r.sv[k] = sinT[(long)pos * half + ic];
  }
}

// Per-head RMSNorm (weights nw, when set) and RoPE of one head vector v[0..HD) in LDS, by one wave, with the
// arithmetic of src/model/forward.js:203-211 and src/compute/ref-kernels.js:305-310, 344-363 (64-lane strided f64 sum
// of squares and butterfly; f64 rotation of each (i, i + half) or (2i, 2i + 1) pair, stored f32), from values loaded by
// rope_load_w / rope_load_cs.
template <int HD>
__device__ inline void norm_rope_apply(float *v, const RopeVals<HD> &r, const float *nw, double eps, int nRot, int neox,
                                       int lane) {
  const int half = nRot / 2;
  if (nw) {
    double ss = 0;
    for (int i = lane; i < HD; i += 64) { const double x = (double)v[i]; ss += x * x; }
    ss = wave_sum_xor(ss, 64);
    const double sc = 1.0 / sqrt(ss / (double)HD + eps);
    #pragma unroll
    for (int k = 0; k < RopeVals<HD>::NW; k++) {
      const int i = lane + 64 * k;
      if (i < HD) v[i] = (float)((double)v[i] * sc * (double)r.wv[k]);
    }
  }
  #pragma unroll
  for (int k = 0; k < RopeVals<HD>::PR; k++) {
    const int i = lane + 64 * k;
    if (i >= half) break;
    const int i0 = neox ? i : 2 * i, i1 = neox ? i + half : 2 * i + 1;
    const double c = (double)r.cv[k], sn = (double)r.sv[k];
    const double x0 = (double)v[i0], x1 = (double)v[i1];
    v[i0] = (float)(x0 * c - x1 * sn);  // pairs are disjoint across lanes
    v[i1] = (float)(x0 * sn + x1 * c);
  }
}

// Both at position pos; the table values and norm weights are requested before the sum of squares, which does not need
// them.
template <int HD>
__device__ inline void norm_rope(float *v, const float *nw, double eps, int nRot, int neox, const float *cosT,
                                 const float *sinT, int pos, int lane) {
  RopeVals<HD> r;
  rope_load_cs<HD>(r, nRot, cosT, sinT, pos, lane);
  rope_load_w<HD>(r, nw, cosT, lane);
  norm_rope_apply<HD>(v, r, nw, eps, nRot, neox, lane);
}

// Contexts from which the long-context launch forms are used (KV cache capacity in positions).
constexpr int AV_BIG_CTX = 4096;

// Scores of one 64-position chunk of one token for hg query heads sharing a KV head. Keys of positions before the
// pass (pos0) come from the cache; the pass's own keys (positions pos0 .. pos0 + b) are normed and rotated here from the
// projection output, rounded as the cache stores them, and the block of token b appends its own key and value to the
// cache (K position-major, V dimension-major), which is where the reference's pass writes them before attending
// (src/model/forward.js:203-214). The query heads are normed and rotated here too.
template <int HD, bool F16KV>
__global__ __launch_bounds__(256) void k_attn_scores(const AttnArgs a) {
  constexpr int VB = F16KV ? 2 : 4;      // bytes per cached value
  constexpr int EPW = 16 / VB;           // K values per 16-byte load
  constexpr int LP = HD / ATTN_VPL;      // lanes per position (ATTN_VPL values each)
  constexpr int NLD = ATTN_VPL / EPW;    // 16-byte loads per lane and position
  constexpr int PPI = 256 / LP;          // positions per load round
  constexpr int P = attn_score_chunk(HD);  // positions per chunk
  constexpr int R = P / PPI;             // load rounds per chunk
  static_assert(R >= 1 && P % PPI == 0, "chunk geometry");
  __shared__ float qs[8 * HD];
  __shared__ float kf[8 * HD];           // rotated keys of the pass, a batch of up to 8 positions at a time (f32)
  extern __shared__ __align__(16) uint8_t kn[];  // the chunk's new keys in cache format, from position n0: [min(P, B)][HD]
  // Workgroups go to the 8 XCDs round robin (linear id mod 8). At long contexts, where a layer's keys outgrow the
  // L2s, the blocks of the pass's tokens that read the same key chunks are given consecutive linear ids of one XCD, so
  // their K reads meet in that XCD's L2 instead of each token streaming the keys from memory again (measured: 16K
  // context, 9 tokens, 0.24 ms less per verify pass; at ~700 positions the keys stay in L2 and the order costs 0.02 ms).
  const int stB = a.step->B, stPos0 = a.step->pos0;  // the pass's step record (scalar loads, read before the pins)
  const int X = gridDim.x, XY = X * gridDim.y, Z = gridDim.z;
  pin_args(Z, a.q, a.ldq, a.qhs, a.k, a.ldkv, a.kcache, a.hpb, a.layer, a.nHead, a.nHeadKv);
  const int L = blockIdx.x + X * (blockIdx.y + gridDim.y * blockIdx.z);
  int xy, b;
  if (a.ctx >= AV_BIG_CTX && XY % 8 == 0) {
    const int q = L >> 3;
    b = q % Z;
    xy = (L & 7) + 8 * (q / Z);
  } else {
    b = L / XY;
    xy = L - b * XY;
  }
  const int bx = xy % X, by = xy / X;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int group = a.nHead / a.nHeadKv, hg = a.hpb;
  const int h0 = by * hg;        // first query head of this block
  const int kvh = h0 / group;
  const bool writer = h0 % group == 0;   // the first head group of a KV head appends the pass's K and V
  const long kvoff = ((long)a.layer * a.nHeadKv + kvh) * a.ctx * HD;
  const uint8_t *kbase = (const uint8_t *)a.kcache + kvoff * VB;
  float *srow = a.scores + ((long)b * a.nHead + h0) * a.sld;
  const int part = tid % LP, sub = tid / LP;
  uint4 u[R][NLD];
  // cached keys (positions of the pass are filled in from kn); the first chunk's keys and the query heads are requested
  // before the pass's step record arrives, so the positions past the cache's valid ones are read too (and unused)
  auto fetch = [&](int c0, int lim) {
    #pragma unroll
    for (int r = 0; r < R; r++) {
      const int t = c0 + r * PPI + sub;
      #pragma unroll
      for (int k = 0; k < NLD; k++)
        u[r][k] = t < lim ? *(const uint4 *)(kbase + ((long)t * HD + part * ATTN_VPL) * VB + 16 * k) : make_uint4(0, 0, 0, 0);
    }
  };
  // the query heads and the pass's keys, then the first chunk of cached keys: loads complete in order, so the query
  // rotation below waits for the query values alone while the keys are on their way
  constexpr int QV = 8 * HD / 256;  // query values per thread (at most 8 heads of HD values per block)
  float qv[QV];
  #pragma unroll
  for (int k = 0; k < QV; k++) {
    const int i = tid + 256 * k;
    qv[k] = i < hg * HD ? a.q[(long)b * a.ldq + (long)(h0 + i / HD) * a.qhs + i % HD] : 0.f;
  }
  // the pass's first 8 key rows of this KV head (row-major [row][HD], element tid + 256 k), for the blocks that norm
  // and rotate the pass's keys; unconditional loads (rows past B read row 0, unused)
  constexpr int KPT = 8 * HD / 256;
  const int nB = Z;
  float kr[KPT];
  #pragma unroll
  for (int k = 0; k < KPT; k++) {
    const int e = tid + 256 * k, row = e / HD < nB ? e / HD : 0;
    kr[k] = a.k[(long)row * a.ldkv + (long)kvh * HD + e % HD];
  }
  __builtin_amdgcn_sched_barrier(0);
  fetch(bx * P, a.ctx);
  __builtin_amdgcn_sched_barrier(0);
  if (b >= stB) return;
  const int pos0 = stPos0, npos = pos0 + b + 1;
  if (bx * P >= npos) return;
  #pragma unroll
  for (int k = 0; k < QV; k++)
    if (tid + 256 * k < hg * HD) qs[tid + 256 * k] = qv[k];
  __syncthreads();
  for (int h = wave; h < hg; h += 4) norm_rope<HD>(qs + h * HD, a.qNorm, a.eps, a.nRot, a.neox, a.cosT, a.sinT, npos - 1, lane);
  __syncthreads();
  for (int c0 = bx * P; c0 < npos; c0 += X * P) {
    if (c0 != bx * P) fetch(c0, pos0);
    // the pass's keys in this chunk: positions [n0, n1), tokens [n0 - pos0, n1 - pos0)
    const int n0 = max(c0, pos0), n1 = min(c0 + P, npos);
    for (int g0 = n0; g0 < n1; g0 += 8) {
      const int g1 = min(n1, g0 + 8);
      if (g0 == pos0) {  // rows 0 .. g1 - g0 - 1: the prefetched ones
        #pragma unroll
        for (int k = 0; k < KPT; k++)
          if (tid + 256 * k < (g1 - g0) * HD) kf[tid + 256 * k] = kr[k];
      } else {
        for (int i = tid; i < (g1 - g0) * HD; i += 256)
          kf[i] = a.k[(long)(g0 - pos0 + i / HD) * a.ldkv + (long)kvh * HD + i % HD];
      }
      __syncthreads();
      for (int p = g0 + wave; p < g1; p += 4)
        norm_rope<HD>(kf + (p - g0) * HD, a.kNorm, a.eps, a.nRot, a.neox, a.cosT, a.sinT, p, lane);
      __syncthreads();
      for (int i = tid; i < (g1 - g0) * HD; i += 256) {
        const int p = g0 + i / HD, d = i % HD;
        const float kv = kf[i];
        const long off = kvoff + (long)p * HD + d;
        if (F16KV) {
          const uint16_t hbits = f2h(kv);
          ((uint16_t *)kn)[(p - n0) * HD + d] = hbits;
          if (writer && p == npos - 1) {
            ((uint16_t *)a.kcache)[off] = hbits;
            ((uint16_t *)a.vcache)[(((long)a.layer * a.nHeadKv + kvh) * HD + d) * a.vstride + p] =
                f2h(a.v[(long)b * a.ldkv + (long)kvh * HD + d]);
          }
        } else {
          ((float *)kn)[(p - n0) * HD + d] = kv;
          if (writer && p == npos - 1) {
            ((float *)a.kcache)[off] = kv;
            ((float *)a.vcache)[(((long)a.layer * a.nHeadKv + kvh) * HD + d) * a.vstride + p] = a.v[(long)b * a.ldkv + (long)kvh * HD + d];
          }
        }
      }
      __syncthreads();
    }
    #pragma unroll
    for (int r = 0; r < R; r++) {
      const int t = c0 + r * PPI + sub;
      if (t >= pos0 && t < npos) {
        #pragma unroll
        for (int k = 0; k < NLD; k++) u[r][k] = *(const uint4 *)(kn + ((t - n0) * HD + part * ATTN_VPL) * VB + 16 * k);
      }
      double kv[ATTN_VPL];
      #pragma unroll
      for (int k = 0; k < NLD; k++) {
        const uint32_t w4[4] = {u[r][k].x, u[r][k].y, u[r][k].z, u[r][k].w};
        #pragma unroll
        for (int e = 0; e < EPW; e++)
          kv[k * EPW + e] = F16KV ? (double)h2f((uint16_t)((w4[e >> 1] >> (16 * (e & 1))) & 0xffff)) : (double)__uint_as_float(w4[e]);
      }
      for (int h = 0; h < hg; h++) {
        const float *qh = qs + h * HD + part * ATTN_VPL;
        double s = 0.0;
        #pragma unroll
        for (int e = 0; e < ATTN_VPL; e++) s = fma((double)qh[e], kv[e], s);
        s = wave_sum_xor(s, LP);
        if (part == (h % LP) && t < npos) srow[(long)h * a.sld + t] = (float)(s * a.scale);
      }
    }
    __syncthreads();  // kn is refilled by the next chunk
  }
}

// ---- scores of passes of several tokens on the matrix cores. v_mfma_f64_16x16x4_f64 adds its four products to the
// accumulator as four fused multiply-adds in k order (measured on gfx950, every element of random wide-range operands),
// so eight of them over dimensions 32 j .. 32 j + 31 in order are exactly the per-lane f64 fma chain of k_attn_scores
// (part j of a position's dot), and the parts are joined in the same butterfly order: the same bits. The pass's query
// rows and keys are normed and rotated first (k_attn_prep, which also appends the pass's K and V to the cache, as
// k_attn_scores' writer blocks do), so the score blocks only read.

// One wave per (token, head): query heads are normed, rotated and stored f32 to qr [B][nHead][HD]; KV heads (blockIdx.y
// >= nHead) have their key normed, rotated and appended to the cache in its format, and their value appended.
template <int HD, bool F16KV>
__global__ __launch_bounds__(64) void k_attn_prep(const AttnArgs a) {
  __shared__ float v[HD];
  const int b = blockIdx.x, hy = blockIdx.y, lane = threadIdx.x;
  const Step *st = a.step;
  if (b >= st->B) return;
  const int pos = st->pos0 + b;
  const bool isq = hy < a.nHead;
  const int h = isq ? hy : hy - a.nHead;
  const float *src = isq ? a.q + (long)b * a.ldq + (long)h * a.qhs : a.k + (long)b * a.ldkv + (long)h * HD;
  for (int i = lane; i < HD; i += 64) v[i] = src[i];
  __syncthreads();
  norm_rope<HD>(v, isq ? a.qNorm : a.kNorm, a.eps, a.nRot, a.neox, a.cosT, a.sinT, pos, lane);
  __syncthreads();
  if (isq) {
    for (int i = lane; i < HD; i += 64) a.qr[((long)b * a.nHead + h) * HD + i] = v[i];
    return;
  }
  const long kvoff = ((long)a.layer * a.nHeadKv + h) * a.ctx * HD + (long)pos * HD;
  const long voff = ((long)a.layer * a.nHeadKv + h) * HD;
  for (int d = lane; d < HD; d += 64) {
    const float vv = a.v[(long)b * a.ldkv + (long)h * HD + d];
    if (F16KV) {
      ((uint16_t *)a.kcache)[kvoff + d] = f2h(v[d]);
      ((uint16_t *)a.vcache)[(voff + d) * a.vstride + pos] = f2h(vv);
    } else {
      ((float *)a.kcache)[kvoff + d] = v[d];
      ((float *)a.vcache)[(voff + d) * a.vstride + pos] = vv;
    }
  }
}

// Block (every X-th 64-position tile of the pass, KV head, group of NWV row tiles); wave w computes row tile NWV z + w: 16
// rows r = b G + g (token b, query head kvh G + g) against every position of its tiles, 16 positions at a time. Lane l
// supplies A = the row l mod 16's dimension 32 j + 4 m + l / 16 (its query values, f64, held for the whole block) and B = key value
// [position l mod 16][dimension 32 j + 4 m + l / 16] from LDS, where the block has staged 64 positions' keys as f64;
// the accumulator of lane l element v is (row 4 v + l / 16, position l mod 16).
constexpr int MM_PT = 64;    // positions staged in LDS at a time
// NWV waves per block, one row tile each: 8 for passes of 128 rows or more per KV head (prefill chunks: every staged key
// tile serves 8 row tiles), else 4
template <int HD, bool F16KV, int NWV>
__global__ __launch_bounds__(NWV * 64) void k_attn_scores_mm(const AttnArgs a, int nrows) {
  constexpr int NP = HD / ATTN_VPL;    // parts (32 dimensions each)
  constexpr int VB = F16KV ? 2 : 4;
  constexpr int NT = NWV * 64;
  constexpr int RAW = MM_PT * HD * VB / 16 / NT;  // 16-byte K pieces per thread per staged tile
  static_assert(RAW >= 1 && RAW * NT * 16 == MM_PT * HD * VB, "staging geometry");
  typedef double d4 __attribute__((ext_vector_type(4)));
  extern __shared__ __align__(16) uint8_t lds[];
  // [MM_PT][HD + 2] keys as f64: with rows 2 doubles (4 banks) apart, the 32 lanes of a half-wave's B read (16
  // positions x 2 k-groups, one double each) fall on 64 distinct banks
  double *kd = (double *)lds;
  constexpr int KP = HD + 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n16 = lane & 15, g = lane >> 4;
  const int kvh = blockIdx.y, tile = blockIdx.z * NWV + wave;
  const int G = a.nHead / a.nHeadKv;
  const Step *st = a.step;
  const int Bd = st->B, pos0 = st->pos0, nmax = pos0 + Bd;
  // the block's MM_PT-position tiles: bx, bx + X, ... of the pass's positions (the grid holds as many blocks per KV
  // head and row group as stay resident at once, so the tiles of a pass of any length spread evenly over them)
  const int X = gridDim.x, bx = blockIdx.x, ntile = (nmax + MM_PT - 1) / MM_PT;
  if (bx >= ntile) return;
  const long kvoff = ((long)a.layer * a.nHeadKv + kvh) * a.ctx * HD;
  const uint8_t *kbase = (const uint8_t *)a.kcache + kvoff * VB;
  // A operands: row n16 of the tile, dimensions 32 j + 4 m + g
  const int ra = tile * 16 + n16, ba = ra / G, ha = kvh * G + ra % G;
  const bool rowok = ra < nrows && ba < Bd;
  double A[NP][8];
  #pragma unroll
  for (int j = 0; j < NP; j++)
    #pragma unroll
    for (int m = 0; m < 8; m++)
      A[j][m] = rowok ? (double)a.qr[((long)ba * a.nHead + ha) * HD + 32 * j + 4 * m + g] : 0.0;
  // the rows whose accumulator elements this lane holds: 4 v + g, v = 0..3
  int rb[4], rh[4], rn[4];
  #pragma unroll
  for (int v = 0; v < 4; v++) {
    const int r = tile * 16 + 4 * v + g, bb = r / G;
    rb[v] = bb; rh[v] = kvh * G + r % G;
    rn[v] = (r < nrows && bb < Bd) ? pos0 + bb + 1 : 0;  // positions of the row (0: no row)
  }
  const bool waveok = tile * 16 < nrows;
  uint4 raw[RAW];
  auto fetch = [&](int t0) {
    #pragma unroll
    for (int k = 0; k < RAW; k++) {
      const int e = (k * NT + tid) * (16 / VB), p = e / HD, d = e % HD, t = t0 + p;
      raw[k] = t < nmax ? *(const uint4 *)(kbase + ((long)t * HD + d) * VB) : make_uint4(0, 0, 0, 0);
    }
  };
  // A thread's 16 fetched bytes become PPL 16-byte pieces of f64 keys, one run of PPL * 16 bytes per lane: the runs of
  // LPW neighbouring lanes fill a 256-byte bank window. Step s writes piece (s + rot) mod PPL, rot = (tid / LPW) mod PPL,
  // so the lanes that share bank offsets write different pieces and each 16-lane group of a write covers 64 banks.
  constexpr int PPL = 8 / VB, LPW = 256 / (PPL * 16);
  const int rot = (tid / LPW) % PPL;
  auto store = [&]() {
    #pragma unroll
    for (int k = 0; k < RAW; k++) {
      const int e = (k * NT + tid) * (16 / VB), p = e / HD, d = e % HD;
      const uint32_t w0 = raw[k].x, w1 = raw[k].y, w2 = raw[k].z, w3 = raw[k].w;
      #pragma unroll
      for (int s = 0; s < PPL; s++) {
        const int pc = (s + rot) % PPL;
        double lo, hi;
        if (F16KV) {  // piece pc = the two f16 keys of word pc
          const uint32_t wd = pc == 0 ? w0 : pc == 1 ? w1 : pc == 2 ? w2 : w3;
          lo = (double)h2f((uint16_t)(wd & 0xffff));
          hi = (double)h2f((uint16_t)(wd >> 16));
        } else {      // piece pc = the f32 keys of words 2 pc, 2 pc + 1
          lo = (double)__uint_as_float(pc == 0 ? w0 : w2);
          hi = (double)__uint_as_float(pc == 0 ? w1 : w3);
        }
        *(double2 *)(kd + p * KP + d + 2 * pc) = make_double2(lo, hi);
      }
    }
  };
  fetch(bx * MM_PT);
  for (int ti = bx; ti < ntile; ti += X) {
    const int t0 = ti * MM_PT, c1 = min(t0 + MM_PT, nmax);
    __syncthreads();  // the previous tile's reads are done
    store();
    __syncthreads();
    if (ti + X < ntile) fetch((ti + X) * MM_PT);
    if (waveok) {
      #pragma unroll 1
      for (int pt = 0; pt < MM_PT && t0 + pt < c1; pt += 16) {
        d4 acc[NP];
        #pragma unroll
        for (int j = 0; j < NP; j++) {
          acc[j] = d4{0.0, 0.0, 0.0, 0.0};
          #pragma unroll
          for (int m = 0; m < 8; m++)
            acc[j] = __builtin_amdgcn_mfma_f64_16x16x4f64(A[j][m], kd[(pt + n16) * KP + 32 * j + 4 * m + g], acc[j], 0, 0, 0);
        }
        const int t = t0 + pt + n16;
        #pragma unroll
        for (int v = 0; v < 4; v++) {
          double sv[NP];
          #pragma unroll
          for (int j = 0; j < NP; j++) sv[j] = acc[j][v];
          // the butterfly of k_attn_scores over the position's NP lanes: pairs, then pairs of pairs
          #pragma unroll
          for (int w = 1; w < NP; w *= 2)
            #pragma unroll
            for (int j = 0; j < NP; j += 2 * w) sv[j] = sv[j] + sv[j + w];
          if (t < rn[v]) a.scores[((long)rb[v] * a.nHead + rh[v]) * a.sld + t] = (float)(sv[0] * a.scale);
        }
      }
    }
  }
}

size_t attention_mm_lds(int hd) { return (size_t)MM_PT * (hd + 2) * 8; }


// One block per (32-dim slice, query head, token). The slice's V rows (dimension-major in the cache) are staged
// through LDS in chunks of ROWB bytes per dimension (1024: 512 f16 or 256 f32 positions, at long contexts where the
// softmax row leaves room; else 512), double buffered, the first chunk during the softmax; fewer chunks, fewer barriers in the
// chain. The
// chain runs on lanes 0-31 of wave 0, one output dimension each, reading 16 bytes of consecutive positions at a time.
constexpr int AV_DIMS = 32;       // output dimensions per block
constexpr int AV_ROW = 512;       // bytes of one dimension's positions per chunk (the smaller chunk)
constexpr int AV_ROW_BIG = 1024;  // the larger chunk
constexpr int AV_PITCH = AV_ROW + 16;   // LDS row pitch (the pad spreads the chain's rows over the banks)
constexpr int AV_CHUNK = AV_DIMS * AV_PITCH;
constexpr int AV_UNIT = 32;       // positions per unrolled step of the weighted sum

template <bool F16KV, int ROWB>
__global__ __launch_bounds__(256) void k_attn_av(const AttnArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int PITCH = ROWB + 16, CHUNKB = AV_DIMS * PITCH;  // LDS row pitch and bytes of one staged chunk
  constexpr int VB = F16KV ? 2 : 4;
  constexpr int CT = ROWB / VB;        // positions per chunk
  constexpr int EPP = 16 / VB;           // positions per 16-byte piece
  constexpr int PPR = ROWB / 16;       // pieces per row
  constexpr int LPT = AV_DIMS * PPR / 256;   // 16-byte loads per thread per chunk
  const int slice = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int stB = a.step->B, stPos0 = a.step->pos0;  // the pass's step record (scalar loads, read before the pins)
  pin_args(a.hd, a.nHead, a.nHeadKv, a.layer, a.vstride, a.vcache, a.scores, a.sld, a.ctx);
  const int hd = a.hd, kvh = h / (a.nHead / a.nHeadKv);
  float *p = (float *)lds;                                // [ctx rounded up to AV_UNIT] probabilities
  uint8_t *vbuf = lds + (size_t)((a.ctx + AV_UNIT - 1) / AV_UNIT * AV_UNIT) * 4;  // [2][AV_DIMS][PITCH] staged V rows
  __shared__ double redd[4];
  __shared__ float redf[4];
  const uint8_t *vbase = (const uint8_t *)a.vcache + (((long)a.layer * a.nHeadKv + kvh) * hd + (long)slice * AV_DIMS) * a.vstride * VB;
  uint4 pre[LPT];
  int npos = 0;
  // V pieces of chunk c below `lim` positions (inside the cache row); the first chunk and the first 1024 scores are
  // requested before the pass's step record arrives, and the pieces at or past the last position are zeroed after it
  auto fetch = [&](int c, int lim) {
    #pragma unroll
    for (int k = 0; k < LPT; k++) {
      const int idx = k * 256 + tid, dim = idx / PPR, t = c * CT + (idx % PPR) * EPP;
      pre[k] = t < lim ? *(const uint4 *)(vbase + ((long)dim * a.vstride + t) * VB) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
    #pragma unroll
    for (int k = 0; k < LPT; k++) {
      const int idx = k * 256 + tid;
      *(uint4 *)(vbuf + buf * CHUNKB + (idx / PPR) * PITCH + (idx % PPR) * 16) = pre[k];
    }
  };
  // the first 1024 scores, then the first V chunk: loads complete in order, so the softmax below waits for the scores
  // alone while the V chunk is on its way
  const float *srow = a.scores + ((long)b * a.nHead + h) * a.sld;
  float v0[4];
  #pragma unroll
  for (int k = 0; k < 4; k++) { const int t = k * 256 + tid; v0[k] = srow[t < a.ctx ? t : 0]; }  // (t >= npos: unused)
  __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
  for (int k = 0; k < LPT; k++) {  // unconditional loads (pieces past the cache's positions read position 0, zeroed
                                   // below with every piece at or past the last position): a load under a branch
                                   // would make the first use of the scores wait for it too
    const int idx = k * 256 + tid, dim = idx / PPR, t = (idx % PPR) * EPP;
    pre[k] = *(const uint4 *)(vbase + ((long)dim * a.vstride + (t < a.ctx ? t : 0)) * VB);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (b >= stB) return;
  npos = stPos0 + b + 1;
  const int nch = (npos + CT - 1) / CT;
  // ---- softmax (src/compute/ref-kernels.js:313-320)
  float mx = -INFINITY;
  #pragma unroll
  for (int k = 0; k < 4; k++) { const int t = k * 256 + tid; if (t < npos) p[t] = v0[k]; else v0[k] = -INFINITY; mx = fmaxf(mx, v0[k]); }
  for (int t0 = 1024; t0 < npos; t0 += 16 * 256) {  // 16 loads per thread in flight at a time
    float v[16];
    #pragma unroll
    for (int k = 0; k < 16; k++) { const int t = t0 + k * 256 + tid; v[k] = srow[t < npos ? t : 0]; }
    #pragma unroll
    for (int k = 0; k < 16; k++) { const int t = t0 + k * 256 + tid; if (t < npos) { p[t] = v[k]; mx = fmaxf(mx, v[k]); } }
  }
  mx = group_fmax(mx, 64);
  if (lane == 0) redf[wave] = mx;
  __syncthreads();
  const double m = (double)fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  // four independent exponentials per step (their f64 chains overlap), added to the sum in position order as before
  double sum = 0.0;
  for (int t0 = tid; t0 < npos; t0 += 4 * 256) {
    double e[4];
    #pragma unroll
    for (int k = 0; k < 4; k++) {
      const int t = t0 + 256 * k;
      e[k] = exp((double)p[t < npos ? t : t0] - m);
    }
    #pragma unroll
    for (int k = 0; k < 4; k++) {
      const int t = t0 + 256 * k;
      if (t < npos) { p[t] = (float)e[k]; sum += e[k]; }
    }
  }
  sum = wave_sum_xor(sum, 64);
  if (lane == 0) redd[wave] = sum;
  __syncthreads();
  const double inv = 1.0 / ((redd[0] + redd[1]) + (redd[2] + redd[3]));
  for (int t = tid; t < npos; t += 256) p[t] = (float)((double)p[t] * inv);
  for (int t = npos + tid; t < (npos + AV_UNIT - 1) / AV_UNIT * AV_UNIT; t += 256) p[t] = 0.f;
  #pragma unroll
  for (int k = 0; k < LPT; k++) {  // the first chunk's pieces from the last position on: zeros, as in later chunks
    const int t = ((k * 256 + tid) % PPR) * EPP;
    if (t >= npos) pre[k] = make_uint4(0, 0, 0, 0);
    else if (t + EPP > npos) {
      uint32_t w[4] = {pre[k].x, pre[k].y, pre[k].z, pre[k].w};
      #pragma unroll
      for (int e = 0; e < EPP; e++)
        if (t + e >= npos) {
          if (F16KV) w[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
          else w[e] = 0u;
        }
      pre[k] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  store(0);
  __syncthreads();
  // ---- weighted sum of V: f32 fma chain in position order, one output dimension per lane (lanes 0-31 of wave 0)
  const bool chainLane = wave == 0 && lane < AV_DIMS;
  float o = 0.f;
  for (int c = 0; c < nch; c++) {
    if (c + 1 < nch) fetch(c + 1, npos);
    if (chainLane) {
      // units of UNIT positions, software pipelined: the LDS reads of unit u + 1 are issued before the fma steps of
      // unit u, so the chain (one dependent fma per position, ~2.2 ns each) does not wait out an LDS latency per unit.
      // p is zero past the last position, so a unit may run past `cnt`: fmaf(0, v, o) == o for the finite cached
      // values read there. The read-ahead index is clamped to the chunk's last unit (a re-read, never past it).
      const int t0 = c * CT, cnt = min(CT, npos - t0), nu = (cnt + AV_UNIT - 1) / AV_UNIT;
      const uint8_t *row = vbuf + (c & 1) * CHUNKB + lane * PITCH;
      const float *pc = p + t0;
      float4 pa[AV_UNIT / 4], pb[AV_UNIT / 4];
      uint4 va[AV_UNIT * VB / 16], vb[AV_UNIT * VB / 16];
      auto read = [&](int u, float4 (&pv)[AV_UNIT / 4], uint4 (&vv)[AV_UNIT * VB / 16]) {
        #pragma unroll
        for (int k = 0; k < AV_UNIT / 4; k++) pv[k] = *(const float4 *)(pc + u * AV_UNIT + 4 * k);
        #pragma unroll
        for (int k = 0; k < AV_UNIT * VB / 16; k++) vv[k] = *(const uint4 *)(row + (u * AV_UNIT + k * EPP) * VB);
      };
      auto steps = [&](const float4 (&pv)[AV_UNIT / 4], const uint4 (&vv)[AV_UNIT * VB / 16]) {
        #pragma unroll
        for (int k = 0; k < AV_UNIT / 4; k++) {
          float v0, v1, v2, v3;
          if (F16KV) {
            const uint4 &w = vv[k >> 1];
            const uint32_t lo = (k & 1) ? w.z : w.x, hi = (k & 1) ? w.w : w.y;
            v0 = h2f((uint16_t)(lo & 0xffff)); v1 = h2f((uint16_t)(lo >> 16));
            v2 = h2f((uint16_t)(hi & 0xffff)); v3 = h2f((uint16_t)(hi >> 16));
          } else {
            const uint4 &w = vv[k];
            v0 = __uint_as_float(w.x); v1 = __uint_as_float(w.y); v2 = __uint_as_float(w.z); v3 = __uint_as_float(w.w);
          }
          o = fmaf(pv[k].x, v0, o); o = fmaf(pv[k].y, v1, o); o = fmaf(pv[k].z, v2, o); o = fmaf(pv[k].w, v3, o);
        }
      };
      // two units per iteration and no branch between a unit's reads and its steps (a branch there lets the compiler
      // sink the reads to their use); an odd last unit is already in (pa, va) after the loop
      read(0, pa, va);
      int u = 0;
      for (; u + 2 <= nu; u += 2) {
        read(u + 1, pb, vb);
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the steps (the scheduler moves them to their use)
        steps(pa, va);
        read(min(u + 2, nu - 1), pa, va);
        __builtin_amdgcn_sched_barrier(0);
        steps(pb, vb);
      }
      if (u < nu) steps(pa, va);
    }
    __syncthreads();
    if (c + 1 < nch) store((c + 1) & 1);
    __syncthreads();
  }
  if (chainLane) {
    const int col = h * hd + slice * AV_DIMS + lane;
    if (a.gate) {  // gated attention output (src/model/forward-qwen35.js:103): o * sigmoid(gate), f64, stored f32
      const double g = (double)a.gate[(long)b * a.ldq + (long)h * a.qhs + slice * AV_DIMS + lane];
      o = (float)((double)o * (1.0 / (1.0 + exp(-g))));
    }
    if (a.out) a.out[(long)b * a.ldo + col] = o;
    if (a.act.q) quant_block32(o, col, a.act, b);  // (unset: the output GEMV quantises the f32 rows itself)
  }
}

// ---- k_attn_av's weighted sum with the chains on the matrix cores: v_mfma_f32_16x16x4_f32 is four sequential fmaf in k
// order (measured), so a chain of MFMAs whose A operand holds the row's probabilities in row 0 (rows 1-15 zero) and
// whose B operand holds V of 16 dimensions computes the position-order f32 chain of every dimension bit for bit. A
// dependent MFMA issues every 32 cycles (8 per position, where a dependent v_fma_mix_f32 takes 9) only while the wave
// issues nothing else but LDS reads between them (a VALU instruction there costs ~12 cycles: measured), so V is staged
// in LDS already converted to f32 and the chain waves only read and multiply.
// One block per (32-dim slice, query head, token), as k_attn_av: the same softmax (the same max, the exponentials
// summed in the same thread order, p = f32(f32(e) * inv)); then waves 0-1 run the chains of dimensions 16 w .. 16 w + 15
// of chunk c while waves 2-3 stage chunk c + 1 (V as f32, and its probabilities, whose exponentials they compute again
// from the scores: the same bits) and request chunk c + 2. One barrier per chunk; LDS does not grow with the context.
// LDS holds V and the probabilities by position mod 4 (section k holds positions 4 m + k, m ascending), so the 16
// lanes of MFMA k-group g read their own positions contiguously, 4 MFMAs' operands per 16-byte read.
constexpr int AVM_CT = 512;                 // positions per chunk
template <bool B> struct Whole { static constexpr bool value = B; };  // a chunk below every row's last position
constexpr int AVM_SF = AVM_CT / 4 + 4;      // floats of one position section (16-byte pad)
constexpr int AVM_RS = 4 * AVM_SF + 4;      // floats of one dimension row (4 x an odd number: the 16 lanes of a chain
                                            // read, rows n16 = 0..15, fall on 64 distinct banks)
constexpr int AVM_UNIT = 32;                // positions per pipelined step of a chain (8 MFMAs)
constexpr int AVM_NK = 72;                  // scores per thread the softmax keeps in registers
constexpr int AVM_MAX_CTX = AVM_NK * 256;   // contexts this form takes (18432 positions)
size_t attention_av_mfma_lds() { return ((size_t)2 * AV_DIMS * AVM_RS + (2 * 4 + 1) * AVM_SF) * 4; }

template <bool F16KV>
__global__ __launch_bounds__(256) void k_attn_av_mfma(const AttnArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int VB = F16KV ? 2 : 4;
  constexpr int CT = AVM_CT, SF = AVM_SF, RS = AVM_RS;
  constexpr int EPP = 16 / VB;                      // positions per 16-byte piece
  constexpr int PPR = CT / EPP;                     // pieces per dimension row of a chunk
  constexpr int PLT = AV_DIMS * PPR / 128;          // pieces per producer thread per chunk (16 f16, 32 f32)
  constexpr int SPT = CT / 128;                     // probabilities per producer thread per chunk
  constexpr int NU = CT / AVM_UNIT;                 // units per chunk
  float *vk = (float *)lds;                         // [2][AV_DIMS][RS]: V of position 4 m + k, dimension j at j RS + k SF + m
  float *pk = vk + 2 * AV_DIMS * RS;                // [2][4][SF]: p of position 4 m + k at [k][m]
  float *zb = pk + 2 * 4 * SF;                      // [SF] zeros: the A operand of rows 1-15
  __shared__ double redd[4];
  __shared__ float redf[4];
  __shared__ float ot[AV_DIMS];
  const int slice = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n16 = lane & 15, g = lane >> 4;
  const int hd = a.hd, kvh = h / (a.nHead / a.nHeadKv);
  const uint8_t *vbase = (const uint8_t *)a.vcache + (((long)a.layer * a.nHeadKv + kvh) * hd + (long)slice * AV_DIMS) * a.vstride * VB;
  const float *srow = a.scores + ((long)b * a.nHead + h) * a.sld;
  const bool producer = wave >= 2;
  const int pt = tid - 128;                         // producer thread 0..127
  uint4 pre[PLT];
  float sp[SPT];
  int npos = 0;
  double m = 0.0, inv = 0.0;
  // chunk c's V pieces and scores, from in-range rows and positions (what lies past the last position is zeroed when
  // the chunk is staged)
  auto fetch_v = [&](int c, int lim) {
    #pragma unroll
    for (int k = 0; k < PLT; k++) {
      const int idx = k * 128 + pt, dim = idx / PPR, t = c * CT + (idx % PPR) * EPP;
      pre[k] = *(const uint4 *)(vbase + ((long)dim * a.vstride + (t < lim ? t : 0)) * VB);
    }
  };
  auto fetch_s = [&](int c, int lim) {
    #pragma unroll
    for (int i = 0; i < SPT; i++) {
      const int t = c * CT + i * 128 + pt;
      sp[i] = srow[t < lim ? t : 0];
    }
  };
  // producers: chunk c into slot c & 1: V as f32 (zeros past the last position) ...
  auto stage_v = [&](int c) {
    float *vs = vk + (c & 1) * AV_DIMS * RS;
    #pragma unroll
    for (int k = 0; k < PLT; k++) {
      const int idx = k * 128 + pt, dim = idx / PPR, pc = idx % PPR, t = c * CT + pc * EPP;
      const uint32_t w[4] = {pre[k].x, pre[k].y, pre[k].z, pre[k].w};
      float f[EPP];
      #pragma unroll
      for (int e = 0; e < EPP; e++) {
        const float x = F16KV ? h2f((uint16_t)((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffff))) : __uint_as_float(w[e]);
        f[e] = t + e < npos ? x : 0.f;
      }
      float *drow = vs + dim * RS;
      #pragma unroll
      for (int q = 0; q < 4; q++) {
        if (F16KV) *(float2 *)(drow + q * SF + 2 * pc) = make_float2(f[q], f[q + 4]);  // positions t + q, t + 4 + q
        else drow[q * SF + pc] = f[q];                                                 // position t + q
      }
    }
  };
  // ... and its probabilities p = f32(f32(e) * inv) (zeros past the last position)
  auto stage_p = [&](int c) {
    float *ps = pk + (c & 1) * 4 * SF;
    #pragma unroll
    for (int i = 0; i < SPT; i++) {
      const int tl = i * 128 + pt, t = c * CT + tl;
      const double e = exp((double)sp[i] - m);
      ps[(tl & 3) * SF + (tl >> 2)] = t < npos ? (float)((double)(float)e * inv) : 0.f;
    }
  };
  if (producer) {
    fetch_v(0, a.ctx);
    fetch_s(0, a.ctx);
  }
  // ---- softmax (src/compute/ref-kernels.js:313-320), k_attn_av's arithmetic: thread tid takes t = tid + 256 k, its
  // exponentials added in k order. The scores stay in registers (-inf past the last position: exp gives +0, which
  // leaves the sum unchanged), so the producers stage chunk 0's V meanwhile; they are requested before the pass's step
  // record arrives (up to the cache's capacity).
  const Step *st = a.step;
  const int sB = st->B, sp0 = st->pos0;
  float sv[AVM_NK];
  #pragma unroll
  for (int k = 0; k < AVM_NK; k++) { const int t = k * 256 + tid; sv[k] = srow[t < a.ctx ? t : 0]; }
  __asm__ volatile("" ::: "memory");  // keeps the loads above the branch (it would otherwise sink them past it)
  if (b >= sB) return;
  npos = sp0 + b + 1;
  const int nch = (npos + CT - 1) / CT;
  const int nend = (npos + AVM_UNIT - 1) / AVM_UNIT * AVM_UNIT;  // positions the chains run
  if (producer) {
    stage_v(0);
    if (nch > 1) fetch_v(1, npos);
  }
  #pragma unroll
  for (int k = 0; k < AVM_NK; k++) sv[k] = k * 256 + tid < npos ? sv[k] : -INFINITY;
  float mx = -INFINITY;
  #pragma unroll
  for (int k = 0; k < AVM_NK; k++) mx = fmaxf(mx, sv[k]);
  mx = group_fmax(mx, 64);
  if (lane == 0) redf[wave] = mx;
  __syncthreads();
  m = (double)fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  double sum = 0.0;
  #pragma unroll
  for (int k0 = 0; k0 < AVM_NK; k0 += 8) {
    if (k0 * 256 < npos) {  // (uniform)
      double e[8];
      #pragma unroll
      for (int k = 0; k < 8; k++) e[k] = exp((double)sv[k0 + k] - m);
      #pragma unroll
      for (int k = 0; k < 8; k++) sum += e[k];
    }
  }
  sum = wave_sum_xor(sum, 64);
  if (lane == 0) redd[wave] = sum;
  __syncthreads();
  inv = 1.0 / ((redd[0] + redd[1]) + (redd[2] + redd[3]));
  if (producer) {
    stage_p(0);
    if (nch > 1) fetch_s(1, npos);
  }
  for (int i = tid; i < SF; i += 256) zb[i] = 0.f;
  __syncthreads();
  // ---- chains (waves 0-1) / staging (waves 2-3)
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  auto mfma8 = [&](const f4 &p0, const f4 &p1, const f4 &v0, const f4 &v1) {
    #pragma unroll
    for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p0[i], v0[i], acc, 0, 0, 0);
    #pragma unroll
    for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p1[i], v1[i], acc, 0, 0, 0);
  };
  // the producers and the chain waves run loops of their own with one barrier per chunk each (the same count), so the
  // chains' accumulator stays in the matrix cores' registers from chunk to chunk
  if (producer) {
    for (int c = 0; c < nch; c++) {
      if (c + 1 < nch) {
        stage_v(c + 1);
        stage_p(c + 1);
        if (c + 2 < nch) {
          fetch_v(c + 2, npos);
          fetch_s(c + 2, npos);
        }
      }
      __syncthreads();
    }
  } else {
    // unit u: the 8 MFMAs of positions c CT + 32 u .. + 31; lane group g supplies positions 4 m + g, m = 8 u .. 8 u + 7
    // (A: lanes of row 0 read the probabilities, the others the zeros). Units two at a time on two operand sets, the
    // next unit's reads ahead of the current unit's MFMAs; a full chunk in straight-line code (constant offsets). The
    // whole chunks run in a loop of their own, so the accumulator keeps one register assignment there.
    auto chunk = [&](int c, auto whole) __attribute__((always_inline)) {
      const float *vr = vk + ((c & 1) * AV_DIMS + wave * 16 + n16) * RS + g * SF;
      const float *pr = n16 == 0 ? pk + ((c & 1) * 4 + g) * SF : zb;
      auto ld = [&](const float *q, int off) { return *(const f4 *)(q + off); };
      if constexpr (decltype(whole)::value) {
        f4 a0 = ld(pr, 0), a1 = ld(pr, 4), a2 = ld(vr, 0), a3 = ld(vr, 4);
        #pragma unroll
        for (int u = 0; u < NU; u += 2) {
          const f4 b0 = ld(pr, 8 * u + 8), b1 = ld(pr, 8 * u + 12), b2 = ld(vr, 8 * u + 8), b3 = ld(vr, 8 * u + 12);
          __builtin_amdgcn_sched_barrier(0);
          mfma8(a0, a1, a2, a3);
          if (u + 2 < NU) { a0 = ld(pr, 8 * u + 16); a1 = ld(pr, 8 * u + 20); a2 = ld(vr, 8 * u + 16); a3 = ld(vr, 8 * u + 20); }
          __builtin_amdgcn_sched_barrier(0);
          mfma8(b0, b1, b2, b3);
        }
      } else {
        const int nu = (nend - c * CT) / AVM_UNIT;
        f4 a0 = ld(pr, 0), a1 = ld(pr, 4), a2 = ld(vr, 0), a3 = ld(vr, 4);
        int u = 0;
        for (; u + 2 <= nu; u += 2) {
          const f4 b0 = ld(pr, 8 * u + 8), b1 = ld(pr, 8 * u + 12), b2 = ld(vr, 8 * u + 8), b3 = ld(vr, 8 * u + 12);
          __builtin_amdgcn_sched_barrier(0);
          mfma8(a0, a1, a2, a3);
          const int un = min(u + 2, nu - 1);  // (a re-read of the last unit when past it)
          a0 = ld(pr, 8 * un); a1 = ld(pr, 8 * un + 4); a2 = ld(vr, 8 * un); a3 = ld(vr, 8 * un + 4);
          __builtin_amdgcn_sched_barrier(0);
          mfma8(b0, b1, b2, b3);
        }
        if (u < nu) mfma8(a0, a1, a2, a3);
      }
      __syncthreads();
    };
    const int nwhole = min(nch, nend / CT);
    int c = 0;
    for (; c < nwhole; c++) chunk(c, Whole<true>{});
    for (; c < nch; c++) chunk(c, Whole<false>{});
  }
  // ---- epilogue: row 0's outputs (element 0 of lanes 0-15 of each chain wave) to lanes 0-31 of wave 0
  if (!producer && g == 0) ot[wave * 16 + n16] = acc[0];
  __syncthreads();
  if (wave == 0 && lane < AV_DIMS) {
    const int col = h * hd + slice * AV_DIMS + lane;
    float o = ot[lane];
    if (a.gate) {  // gated attention output (src/model/forward-qwen35.js:103): o * sigmoid(gate), f64, stored f32
      const double gv = (double)a.gate[(long)b * a.ldq + (long)h * a.qhs + slice * AV_DIMS + lane];
      o = (float)((double)o * (1.0 / (1.0 + exp(-gv))));
    }
    if (a.out) a.out[(long)b * a.ldo + col] = o;
    if (a.act.q) quant_block32(o, col, a.act, b);  // (unset: the output GEMV quantises the f32 rows itself)
  }
}

// ---- the same weighted sum for long contexts, one block per (query head, token) over all HD dimensions. k_attn_av keeps
// the block's softmax row in LDS, which at 16K positions leaves room for one block per CU, and its four slice blocks of
// a head hold four copies. Here the exponentials are written back over the head's scores (one block per row, so no
// other block reads them), and the probabilities p = f32(e * inv) are staged chunk by chunk with V: LDS no longer grows
// with the context, and a head's four slices share one softmax. The arithmetic is k_attn_av's (the same max, the same
// exponentials summed in the same thread order, the same chain per dimension), so the two give the same bits.
constexpr int AVH_CTX = 8192;  // contexts above this take the per-head form (HD <= 128)

template <int HD, bool F16KV>
__global__ __launch_bounds__(256) void k_attn_av_head(const AttnArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int VB = F16KV ? 2 : 4;
  constexpr int CT = AV_ROW / VB;          // positions per chunk
  constexpr int EPP = 16 / VB;             // positions per 16-byte piece
  constexpr int PPR = AV_ROW / 16;         // pieces per row
  constexpr int CHUNK = HD * AV_PITCH;     // bytes of one staged chunk of V rows
  constexpr int LPT = HD * PPR / 256;      // pieces per thread per chunk
  constexpr int PPT = CT / 256 > 0 ? CT / 256 : 1;  // probabilities per thread per chunk
  static_assert(HD * PPR % 256 == 0 && CT % 256 == 0 || CT == 128, "chunk geometry");
  float *pb = (float *)(lds + 2 * CHUNK);  // [2][CT] staged probabilities
  __shared__ double redd[4];
  __shared__ float redf[4];
  const int h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kvh = h / (a.nHead / a.nHeadKv);
  const uint8_t *vbase = (const uint8_t *)a.vcache + ((long)a.layer * a.nHeadKv + kvh) * HD * a.vstride * VB;
  float *srow = a.scores + ((long)b * a.nHead + h) * a.sld;
  uint4 pre[LPT];
  float pp[PPT];
  auto fetch = [&](int c, int lim) {
    #pragma unroll
    for (int k = 0; k < LPT; k++) {
      const int idx = k * 256 + tid, dim = idx / PPR, t = c * CT + (idx % PPR) * EPP;
      pre[k] = t < lim ? *(const uint4 *)(vbase + ((long)dim * a.vstride + t) * VB) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
    #pragma unroll
    for (int k = 0; k < LPT; k++) {
      const int idx = k * 256 + tid;
      *(uint4 *)(lds + buf * CHUNK + (idx / PPR) * AV_PITCH + (idx % PPR) * 16) = pre[k];
    }
  };
  fetch(0, a.ctx);
  const Step *st = a.step;
  if (b >= st->B) return;
  const int npos = st->pos0 + b + 1;
  const int nch = (npos + CT - 1) / CT;
  #pragma unroll
  for (int k = 0; k < LPT; k++) {  // the first chunk's pieces from the last position on: zeros, as in later chunks
    const int t = ((k * 256 + tid) % PPR) * EPP;
    if (t >= npos) pre[k] = make_uint4(0, 0, 0, 0);
    else if (t + EPP > npos) {
      uint32_t w[4] = {pre[k].x, pre[k].y, pre[k].z, pre[k].w};
      #pragma unroll
      for (int e = 0; e < EPP; e++)
        if (t + e >= npos) {
          if (F16KV) w[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
          else w[e] = 0u;
        }
      pre[k] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  // ---- softmax (src/compute/ref-kernels.js:313-320) in k_attn_av's order; the exponentials replace the scores
  float mx = -INFINITY;
  for (int t0 = tid; t0 < npos; t0 += 16 * 256) {  // 16 loads per thread in flight at a time
    float v[16];
    #pragma unroll
    for (int k = 0; k < 16; k++) { const int t = t0 + 256 * k; v[k] = srow[t < npos ? t : t0]; }
    #pragma unroll
    for (int k = 0; k < 16; k++) mx = fmaxf(mx, v[k]);  // (a clamped reload repeats a value already counted)
  }
  mx = group_fmax(mx, 64);
  if (lane == 0) redf[wave] = mx;
  __syncthreads();
  const double m = (double)fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  double sum = 0.0;
  for (int t0 = tid; t0 < npos; t0 += 16 * 256) {  // positions tid + 256 j added in j order, as k_attn_av does
    float v[16];
    #pragma unroll
    for (int k = 0; k < 16; k++) { const int t = t0 + 256 * k; v[k] = srow[t < npos ? t : t0]; }
    #pragma unroll
    for (int q = 0; q < 16; q += 4) {
      double e[4];
      #pragma unroll
      for (int k = 0; k < 4; k++) e[k] = exp((double)v[q + k] - m);
      #pragma unroll
      for (int k = 0; k < 4; k++) {
        const int t = t0 + 256 * (q + k);
        if (t < npos) { srow[t] = (float)e[k]; sum += e[k]; }
      }
    }
  }
  sum = wave_sum_xor(sum, 64);
  if (lane == 0) redd[wave] = sum;
  __syncthreads();  // also orders this block's writes of the exponentials before their reads below
  const double inv = 1.0 / ((redd[0] + redd[1]) + (redd[2] + redd[3]));
  // probabilities of chunk c (zero past the last position, as k_attn_av's row)
  auto pload = [&](int c) {
    #pragma unroll
    for (int k = 0; k < PPT; k++) {
      const int t = c * CT + k * 256 + tid;
      pp[k] = (k * 256 + tid < CT && t < npos) ? srow[t] : 0.f;
    }
  };
  auto pstore = [&](int buf) {
    #pragma unroll
    for (int k = 0; k < PPT; k++)
      if (k * 256 + tid < CT) pb[buf * CT + k * 256 + tid] = (float)((double)pp[k] * inv);
  };
  pload(0);
  store(0);
  pstore(0);
  __syncthreads();
  // ---- weighted sum: output dimension wave * 64 + lane on the first HD / 64 waves, chunk by chunk (double buffered)
  const bool chainLane = wave < HD / 64;
  const int dim = wave * 64 + lane;
  float o = 0.f;
  for (int c = 0; c < nch; c++) {
    if (c + 1 < nch) { fetch(c + 1, npos); pload(c + 1); }
    if (chainLane) {
      const int cnt = min(CT, npos - c * CT), nu = (cnt + AV_UNIT - 1) / AV_UNIT;
      const uint8_t *row = lds + (c & 1) * CHUNK + dim * AV_PITCH;
      const float *pc = pb + (c & 1) * CT;
      float4 pa[AV_UNIT / 4], pbv[AV_UNIT / 4];
      uint4 va[AV_UNIT * VB / 16], vb[AV_UNIT * VB / 16];
      auto read = [&](int u, float4 (&pv)[AV_UNIT / 4], uint4 (&vv)[AV_UNIT * VB / 16]) {
        #pragma unroll
        for (int k = 0; k < AV_UNIT / 4; k++) pv[k] = *(const float4 *)(pc + u * AV_UNIT + 4 * k);
        #pragma unroll
        for (int k = 0; k < AV_UNIT * VB / 16; k++) vv[k] = *(const uint4 *)(row + (u * AV_UNIT + k * EPP) * VB);
      };
      auto steps = [&](const float4 (&pv)[AV_UNIT / 4], const uint4 (&vv)[AV_UNIT * VB / 16]) {
        #pragma unroll
        for (int k = 0; k < AV_UNIT / 4; k++) {
          float v0, v1, v2, v3;
          if (F16KV) {
            const uint4 &w = vv[k >> 1];
            const uint32_t lo = (k & 1) ? w.z : w.x, hi = (k & 1) ? w.w : w.y;
            v0 = h2f((uint16_t)(lo & 0xffff)); v1 = h2f((uint16_t)(lo >> 16));
            v2 = h2f((uint16_t)(hi & 0xffff)); v3 = h2f((uint16_t)(hi >> 16));
          } else {
            const uint4 &w = vv[k];
            v0 = __uint_as_float(w.x); v1 = __uint_as_float(w.y); v2 = __uint_as_float(w.z); v3 = __uint_as_float(w.w);
          }
          o = fmaf(pv[k].x, v0, o); o = fmaf(pv[k].y, v1, o); o = fmaf(pv[k].z, v2, o); o = fmaf(pv[k].w, v3, o);
        }
      };
      read(0, pa, va);
      int u = 0;
      for (; u + 2 <= nu; u += 2) {
        read(u + 1, pbv, vb);
        __builtin_amdgcn_sched_barrier(0);
        steps(pa, va);
        read(min(u + 2, nu - 1), pa, va);
        __builtin_amdgcn_sched_barrier(0);
        steps(pbv, vb);
      }
      if (u < nu) steps(pa, va);
    }
    __syncthreads();
    if (c + 1 < nch) { store((c + 1) & 1); pstore((c + 1) & 1); }
    __syncthreads();
  }
  if (chainLane) {
    const int col = h * HD + dim;
    if (a.gate) {  // gated attention output (src/model/forward-qwen35.js:103): o * sigmoid(gate), f64, stored f32
      const double g = (double)a.gate[(long)b * a.ldq + (long)h * a.qhs + dim];
      o = (float)((double)o * (1.0 / (1.0 + exp(-g))));
    }
    if (a.out) a.out[(long)b * a.ldo + col] = o;
    if (a.act.q) quant_block32(o, col, a.act, b);  // (unset: the output GEMV quantises the f32 rows itself)
  }
}

size_t attention_head_lds(int hd) { return (size_t)2 * hd * AV_PITCH + 2 * 256 * 4; }

// ---- the weighted sum of multi-token passes at long contexts, grouped by KV head. The per-head form above stages its
// KV head's V once per (query head, token) row: at 16K positions, 4 query heads per KV head and 9 tokens that is 36
// reads of 4 MB per KV head, 1.2 GB per layer, and the launch runs at the speed of those reads. Here the softmax runs
// first, one block per row (k_attn_softmax_rows: the per-head form's code; the exponentials replace the scores and
// 1 / sum goes to pinv), then one block per (32-dimension slice, KV head, group of AVG_ROWS rows) stages each V chunk
// once for the chains of all its rows: lanes 0-31 of wave w run row 2w's 32 dimensions, lanes 32-63 row 2w + 1's. Every
// chain is the same position-order f32 chain as in the per-head form, with the same probabilities f32(e * inv); past
// a row's last position its probabilities are 0 (fmaf(0, v, o) leaves o as it is, V staged there being finite cache
// values or zeros), so the bits are the per-head form's.
constexpr int AVG_ROWS = 8;   // rows (query head, token) per block of the grouped weighted sum
constexpr int AVG_DIMS = 32;  // dimensions per block

constexpr int SMR_T = 512;     // threads of k_attn_softmax_rows
constexpr int SMR_RP = 4096;   // positions per round of its sum
constexpr int SMR_NK = 40;     // positions per thread kept in registers (20480 per row)
template <bool NORM>
__global__ __launch_bounds__(SMR_T) void k_attn_softmax_rows(const AttnArgs a) {
  // SMR_T threads: the exponentials on two waves per SIMD. The sum keeps k_attn_av's order (slot s = t mod 256 adds
  // its positions s, s + 256, ... in order, then the 64-lane butterfly and (w0 + w1) + (w2 + w3)): each round of
  // SMR_RP positions parks its exponentials in LDS by slot, and the 256 slot threads add them in position order.
  constexpr int KR = SMR_RP / SMR_T;          // positions per thread per round (8)
  constexpr int NQ = SMR_NK / KR;             // rounds kept in registers
  __shared__ double ex[SMR_RP];               // a round's exponentials at [k][s], t = r0 + 256 k + s
  __shared__ double redd[4];
  __shared__ float redf[SMR_T / 64];
  const int h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const Step *st = a.step;
  if (b >= st->B) return;
  const int npos = st->pos0 + b + 1;
  float *srow = a.scores + ((long)b * a.nHead + h) * a.sld;
  // thread tid holds positions tid + SMR_T k (a clamped load reads position 0, which leaves the maximum unchanged); the
  // loads wait for the step record: the rows of a prefill chunk are far shorter than the cache
  float v[SMR_NK];
  #pragma unroll
  for (int k = 0; k < SMR_NK; k++) { const int t = tid + SMR_T * k; v[k] = srow[t < npos ? t : 0]; }
  float mx = -INFINITY;
  #pragma unroll
  for (int k = 0; k < SMR_NK; k++) mx = fmaxf(mx, v[k]);
  for (int t = SMR_NK * SMR_T + tid; t < npos; t += SMR_T) mx = fmaxf(mx, srow[t]);
  mx = group_fmax(mx, 64);
  if (lane == 0) redf[wave] = mx;
  __syncthreads();
  float mf = redf[0];
  #pragma unroll
  for (int w = 1; w < SMR_T / 64; w++) mf = fmaxf(mf, redf[w]);
  const double m = (double)mf;
  // round q: thread tid computes t = q SMR_RP + tid + SMR_T i (slot tid mod 256, k = 2 i + tid / 256)
  double sum = 0.0;
  auto slot_add = [&]() {
    __syncthreads();
    if (tid < 256) {
      #pragma unroll
      for (int k = 0; k < SMR_RP / 256; k++) sum += ex[k * 256 + tid];  // +0 past the last position: no change
    }
    __syncthreads();
  };
  #pragma unroll
  for (int q = 0; q < NQ; q++) {
    if (q * SMR_RP < npos) {  // (uniform)
      #pragma unroll
      for (int i = 0; i < KR; i++) {
        const int k = q * KR + i, t = tid + SMR_T * k;
        const double e = exp((double)v[k] - m);
        ex[(2 * i + (tid >> 8)) * 256 + (tid & 255)] = t < npos ? e : 0.0;
        v[k] = (float)e;
        if (!NORM && t < npos) srow[t] = v[k];
      }
      slot_add();
    }
  }
  for (int r0 = SMR_NK * SMR_T; r0 < npos; r0 += SMR_RP) {  // positions past the registers
    #pragma unroll
    for (int i = 0; i < KR; i++) {
      const int t = r0 + tid + SMR_T * i;
      const double e = t < npos ? exp((double)srow[t] - m) : 0.0;
      ex[(2 * i + (tid >> 8)) * 256 + (tid & 255)] = e;
      if (t < npos) srow[t] = (float)e;
    }
    slot_add();
  }
  if (tid < 256) {
    sum = wave_sum_xor(sum, 64);
    if (lane == 0) redd[wave] = sum;
  }
  __syncthreads();
  const double inv = 1.0 / ((redd[0] + redd[1]) + (redd[2] + redd[3]));
  if (!NORM) {
    if (tid == 0) a.pinv[(long)b * a.nHead + h] = inv;
    return;
  }
  // the probabilities themselves, p = f32(f32(e) * inv)
  #pragma unroll
  for (int k = 0; k < SMR_NK; k++) {
    const int t = tid + SMR_T * k;
    if (t < npos) srow[t] = (float)((double)v[k] * inv);
  }
  for (int t = SMR_NK * SMR_T + tid; t < npos; t += SMR_T) srow[t] = (float)((double)srow[t] * inv);
}

// ---- weighted sum of passes of several tokens on the matrix cores. v_mfma_f32_16x16x4_f32 adds its four products to
// the accumulator as four fused multiply-adds in k order (measured on gfx950, every element of random wide-range
// operands), so a chain of them over positions t, t + 1, ... in order is the reference's f32 chain out += p_t v_t
// (one rounding per position, src/model/forward.js:131-134) for 16 rows x 16 dimensions at once: the bits of k_attn_av.
// Block: a 32-dimension slice of a KV head for RB = 16 or 32 rows r = b G + g (token b, query head kvh G + g), one or two
// 16-row tiles. Waves 0 .. 2 RB / 16 - 1 run the chains of (row tile w / 2, dimensions 16 (w mod 2) .. + 15) (lane l
// supplies A = p[row l mod 16][position 4 m + l / 16] and B = V[dimension l mod 16][4 m + l / 16] and holds (row
// 4 (l / 16) + v, dimension l mod 16)) while as many waves more stage chunk c + 1 (the probabilities, already normalised
// by k_attn_softmax_rows<true>,
// zero past each row's last position; V as f32, zero past the pass's last position) and request chunk c + 3: each
// producer unit is 16 consecutive positions of one row or dimension (16-byte loads, one 16-byte LDS store per position
// section), two register sets in turn. As in k_attn_av_mfma the chain waves issue only MFMAs and LDS reads, one barrier
// per chunk, operands by position mod 4 (section k holds positions 4 m + k). 32-row blocks stage V once for two tiles
// (prefill chunks); 16-row blocks keep the chain waves on SIMDs of their own (one block per CU), for passes of few rows.
constexpr int MMV_CT = 256;                 // positions per chunk
constexpr int MMV_SF = MMV_CT / 4 + 4;      // floats of one position section (16-byte pad)
constexpr int MMV_RS = 4 * MMV_SF + 4;      // floats of one dimension or row (4 x an odd number: conflict-free chain reads)
template <bool F16KV, int RB>
__global__ __launch_bounds__(RB * 16) void k_attn_av_mm(const AttnArgs a, int nrows) {
  extern __shared__ __align__(16) uint8_t lds[];
  typedef float f4 __attribute__((ext_vector_type(4)));
  typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));  // a row of scores starts at any float
  constexpr int VB = F16KV ? 2 : 4;
  constexpr int CT = MMV_CT, SF = MMV_SF, RS = MMV_RS, NCW = RB / 8, NPT = NCW * 64;  // chain waves, producer threads
  constexpr int EPP = 16 / VB;                      // positions per 16-byte V piece
  constexpr int UL = 16 / EPP;                      // V pieces per unit of 16 positions (2 f16, 4 f32)
  constexpr int UPR = CT / 16;                      // units per dimension or probability row of a chunk
  constexpr int VU = AV_DIMS * UPR / NPT;           // V units per producer thread per chunk
  constexpr int PU = RB * UPR / NPT;                // probability units per producer thread per chunk
  constexpr int NU = CT / AVM_UNIT;                 // units (8 MFMAs) per chunk
  static_assert((RB == 16 || RB == 32) && VU * NPT == AV_DIMS * UPR && PU * NPT == RB * UPR, "producer units");
  float *vk = (float *)lds;                         // [2][AV_DIMS][RS]: V of position 4 m + k, dimension j at j RS + k SF + m
  float *pk = vk + 2 * AV_DIMS * RS;                // [2][RB][RS]: p of row i, position 4 m + k at i RS + k SF + m
  __shared__ float ot[RB][AV_DIMS + 1];             // the block's outputs [row][dimension] for the epilogue
  __shared__ long roff[RB];
  __shared__ int rnp[RB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n16 = lane & 15, g = lane >> 4;
  // XCD-aware block order: workgroup i of the 1-D grid (a multiple of 8 long) goes to XCD i mod 8, and logical block
  // L = (i mod 8) (grid / 8) + i / 8 gives each XCD a contiguous run of L, ordered slice fastest, then row block, then
  // KV head, so the blocks that read the same probability rows (a row block's slices) and the same V (a KV head's row
  // blocks) share one L2 instead of fetching them from HBM once per XCD
  const int NS = a.hd / AV_DIMS, NZ = (nrows + RB - 1) / RB;
  const int L = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  if (L >= NS * NZ * a.nHeadKv) return;
  const int kvh = L / (NS * NZ), rbk = (L / NS) % NZ, d0 = (L % NS) * AV_DIMS;
  const int G = a.nHead / a.nHeadKv;
  const Step *st = a.step;
  const int Bd = st->B, pos0 = st->pos0, nmax = pos0 + Bd;
  // the block's rows: scores row offsets and positions (0: no row)
  if (tid < RB) {
    const int r = rbk * RB + tid, b = r / G, h = kvh * G + r % G;
    const bool live = r < nrows && b < Bd;
    roff[tid] = live ? ((long)b * a.nHead + h) * a.sld : 0;
    rnp[tid] = live ? pos0 + b + 1 : 0;
  }
  __syncthreads();
  int nrmax = 0;
  #pragma unroll
  for (int i = 0; i < RB; i++) nrmax = max(nrmax, rnp[i]);
  if (nrmax == 0) return;  // (uniform)
  const int nch = (nrmax + CT - 1) / CT;
  const int nend = (nrmax + AVM_UNIT - 1) / AVM_UNIT * AVM_UNIT;  // positions the chains run
  const uint8_t *vbase = (const uint8_t *)a.vcache + (((long)a.layer * a.nHeadKv + kvh) * a.hd + d0) * a.vstride * VB;
  const bool producer = wave >= NCW;
  const int pt = tid - NPT;                         // producer thread 0 .. NPT - 1
  const int tr = RB == 32 ? (wave >> 1) & 1 : 0, dg = wave & 1;  // a chain wave's row tile and dimension group
  bool tlive = false;                               // the chain wave's tile holds a row
  #pragma unroll
  for (int i = 0; i < 16; i++) tlive |= rnp[16 * tr + i] > 0;
  struct Pre {
    uint4 v[VU][UL];
    f4 p[PU][4];
  };
  // a chunk that ends at or before every live row's last position (all chunks but the last one or two) needs no load
  // clamped and no value zeroed: fetch and stage take it in a form without those checks (rows without a live query read
  // row 0 of the scores there; their outputs are never stored, and row i of an MFMA result depends on row i of A only)
  int nrmin = INT_MAX;
  #pragma unroll
  for (int i = 0; i < RB; i++) nrmin = rnp[i] > 0 ? min(nrmin, rnp[i]) : nrmin;
  // chunk c's V pieces and probabilities (loads stay inside the cache row and the scores row; what lies past a row's or
  // the pass's last position is zeroed when the chunk is staged)
  auto fetch_f = [&](auto whole, int c, Pre &s) {
    constexpr bool W = decltype(whole)::value;
    #pragma unroll
    for (int k = 0; k < VU; k++) {
      const int u = k * NPT + pt, dim = u / UPR, t0 = c * CT + (u % UPR) * 16;
      #pragma unroll
      for (int l = 0; l < UL; l++) {
        const int t = t0 + l * EPP;
        s.v[k][l] = *(const uint4 *)(vbase + ((long)dim * a.vstride + (W || t < nmax ? t : 0)) * VB);
      }
    }
    #pragma unroll
    for (int k = 0; k < PU; k++) {
      const int u = k * NPT + pt, r = u / UPR, t0 = c * CT + (u % UPR) * 16;
      const float *src = a.scores + roff[r];
      #pragma unroll
      for (int j = 0; j < 4; j++) {
        const int tq = t0 + 4 * j;
        s.p[k][j] = *(const f4u *)(src + (W || tq + 4 <= a.ctx ? tq : 0));
      }
    }
  };
  auto stage_f = [&](auto whole, int c, const Pre &s) {
    constexpr bool W = decltype(whole)::value;
    float *vs = vk + (c & 1) * AV_DIMS * RS;
    #pragma unroll
    for (int k = 0; k < VU; k++) {
      const int u = k * NPT + pt, dim = u / UPR, uu = u % UPR, t0 = c * CT + uu * 16;
      float f[16];
      #pragma unroll
      for (int e = 0; e < 16; e++) {
        const uint4 &pc = s.v[k][e / EPP];
        const int w = e % EPP;
        const uint32_t wd = (F16KV ? w >> 1 : w) == 0 ? pc.x : (F16KV ? w >> 1 : w) == 1 ? pc.y : (F16KV ? w >> 1 : w) == 2 ? pc.z : pc.w;
        const float x = F16KV ? h2f((uint16_t)((w & 1) ? (wd >> 16) : (wd & 0xffff))) : __uint_as_float(wd);
        f[e] = W || t0 + e < nmax ? x : 0.f;
      }
      float *drow = vs + dim * RS + uu * 4;
      #pragma unroll
      for (int q = 0; q < 4; q++) *(f4 *)(drow + q * SF) = (f4){f[q], f[q + 4], f[q + 8], f[q + 12]};
    }
    float *ps = pk + (c & 1) * RB * RS;
    #pragma unroll
    for (int k = 0; k < PU; k++) {
      const int u = k * NPT + pt, r = u / UPR, uu = u % UPR, t0 = c * CT + uu * 16;
      float *prow = ps + r * RS + uu * 4;
      if (W) {
        #pragma unroll
        for (int e = 0; e < 4; e++) *(f4 *)(prow + e * SF) = (f4){s.p[k][0][e], s.p[k][1][e], s.p[k][2][e], s.p[k][3][e]};
      } else {
        const int np = rnp[r];
        #pragma unroll
        for (int e = 0; e < 4; e++) {
          f4 w;
          #pragma unroll
          for (int j = 0; j < 4; j++) w[j] = t0 + 4 * j + e < np ? s.p[k][j][e] : 0.f;
          *(f4 *)(prow + e * SF) = w;
        }
      }
    }
  };
  // (f16 V only: with f32 V both forms do not fit the registers together)
  auto fetch = [&](int c, Pre &s) {
    if (F16KV && (c + 1) * CT <= nrmin) fetch_f(Whole<F16KV>{}, c, s);
    else fetch_f(Whole<false>{}, c, s);
  };
  auto stage = [&](int c, const Pre &s) {
    if (F16KV && (c + 1) * CT <= nrmin) stage_f(Whole<F16KV>{}, c, s);
    else stage_f(Whole<false>{}, c, s);
  };
  Pre s0, s1;
  if (producer) {
    fetch(0, s0);
    if (nch > 1) fetch(1, s1);
    stage(0, s0);
    if (nch > 2) fetch(2, s0);
  }
  __syncthreads();
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  auto mfma8 = [&](const f4 &p0, const f4 &p1, const f4 &v0, const f4 &v1) {
    #pragma unroll
    for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p0[i], v0[i], acc, 0, 0, 0);
    #pragma unroll
    for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p1[i], v1[i], acc, 0, 0, 0);
  };
  auto chains = [&](int c) {
    // unit u: the 8 MFMAs of positions c CT + 32 u .. + 31 (lane group g: positions 4 m + g, m = 8 u .. 8 u + 7); two
    // operand sets, the next unit's reads ahead of the current unit's MFMAs, a full chunk in straight-line code
    const float *vr = vk + ((c & 1) * AV_DIMS + dg * 16 + n16) * RS + g * SF;
    const float *pr = pk + ((c & 1) * RB + tr * 16 + n16) * RS + g * SF;
    auto ld = [&](const float *q, int off) { return *(const f4 *)(q + off); };
    if (c * CT + CT <= nend) {
      f4 a0 = ld(pr, 0), a1 = ld(pr, 4), a2 = ld(vr, 0), a3 = ld(vr, 4);
      #pragma unroll
      for (int u = 0; u < NU; u += 2) {
        const f4 b0 = ld(pr, 8 * u + 8), b1 = ld(pr, 8 * u + 12), b2 = ld(vr, 8 * u + 8), b3 = ld(vr, 8 * u + 12);
        __builtin_amdgcn_sched_barrier(0);
        mfma8(a0, a1, a2, a3);
        if (u + 2 < NU) { a0 = ld(pr, 8 * u + 16); a1 = ld(pr, 8 * u + 20); a2 = ld(vr, 8 * u + 16); a3 = ld(vr, 8 * u + 20); }
        __builtin_amdgcn_sched_barrier(0);
        mfma8(b0, b1, b2, b3);
      }
    } else {
      const int nu = (nend - c * CT) / AVM_UNIT;
      f4 a0 = ld(pr, 0), a1 = ld(pr, 4), a2 = ld(vr, 0), a3 = ld(vr, 4);
      int u = 0;
      for (; u + 2 <= nu; u += 2) {
        const f4 b0 = ld(pr, 8 * u + 8), b1 = ld(pr, 8 * u + 12), b2 = ld(vr, 8 * u + 8), b3 = ld(vr, 8 * u + 12);
        __builtin_amdgcn_sched_barrier(0);
        mfma8(a0, a1, a2, a3);
        const int un = min(u + 2, nu - 1);  // (a re-read of the last unit when past it)
        a0 = ld(pr, 8 * un); a1 = ld(pr, 8 * un + 4); a2 = ld(vr, 8 * un); a3 = ld(vr, 8 * un + 4);
        __builtin_amdgcn_sched_barrier(0);
        mfma8(b0, b1, b2, b3);
      }
      if (u < nu) mfma8(a0, a1, a2, a3);
    }
  };
  // the producers and the chain waves run loops of their own with one barrier per chunk each (the same count), so the
  // chains' accumulator stays in the matrix cores' registers from chunk to chunk; chunk c + 1 sits in register set
  // (c + 1) mod 2, which then requests chunk c + 3
  if (producer) {
    for (int c = 0; c < nch; c += 2) {
      if (c + 1 < nch) {
        stage(c + 1, s1);
        if (c + 3 < nch) fetch(c + 3, s1);
      }
      __syncthreads();
      if (c + 1 < nch) {
        if (c + 2 < nch) {
          stage(c + 2, s0);
          if (c + 4 < nch) fetch(c + 4, s0);
        }
        __syncthreads();
      }
    }
  } else {
    for (int c = 0; c < nch; c++) {
      if (tlive) chains(c);
      __syncthreads();
    }
  }
  // ---- epilogue: the outputs through LDS, then two rows per wave, a row's 32 dimensions on 32 consecutive lanes (one
  // quantizeAct block)
  if (!producer) {
    #pragma unroll
    for (int v = 0; v < 4; v++) ot[16 * tr + 4 * g + v][16 * dg + n16] = acc[v];
  }
  __syncthreads();
  #pragma unroll
  for (int j = 0; j < 2; j++) {
    const int i = j * (RB / 2) + wave * 2 + (lane >> 5);  // (2 NCW waves: RB / 2 rows per pass)
    if (rnp[i] == 0) continue;
    const int r = rbk * RB + i, b = r / G, h = kvh * G + r % G, dim = d0 + (lane & 31), col = h * a.hd + dim;
    float o = ot[i][lane & 31];
    if (a.gate) {  // gated attention output (src/model/forward-qwen35.js:103): o * sigmoid(gate), f64, stored f32
      const double gv = (double)a.gate[(long)b * a.ldq + (long)h * a.qhs + dim];
      o = (float)((double)o * (1.0 / (1.0 + exp(-gv))));
    }
    if (a.out) a.out[(long)b * a.ldo + col] = o;
    if (a.act.q) quant_block32(o, col, a.act, b);  // (unset: the output GEMV quantises the f32 rows itself)
  }
}

size_t attention_av_mm_lds(int rb) { return (size_t)2 * (AV_DIMS + rb) * MMV_RS * 4; }

// nrows: query heads per KV head x the launch's tokens (rows r = b G + g: token b, query head kvh G + g).
// 512 threads: waves 0-3 run the chains of chunk c while waves 4-7 store chunk c + 1 (V and probabilities) into the
// other buffer and request chunk c + 2, so the staging never stands between two chunks' chains (one barrier per chunk).
constexpr int AVG_THREADS = 512;
template <bool F16KV, int ROWB>
__global__ __launch_bounds__(AVG_THREADS) void k_attn_av_group(const AttnArgs a, int nrows) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int VB = F16KV ? 2 : 4;
  constexpr int CT = ROWB / VB;                       // positions per chunk
  constexpr int EPP = 16 / VB;                        // positions per 16-byte piece
  constexpr int PPR = ROWB / 16;                      // pieces per row
  constexpr int PITCH = ROWB + 16;                    // LDS pitch of a staged V row
  constexpr int CHUNK = AVG_DIMS * PITCH;             // bytes of one staged chunk of V rows
  constexpr int LPT = AVG_DIMS * PPR / 256;           // V pieces per staging thread per chunk
  constexpr int PPT = AVG_ROWS * CT / 256;            // probabilities per staging thread per chunk
  static_assert(AVG_DIMS * PPR % 256 == 0 && AVG_ROWS * CT % 256 == 0 && AVG_ROWS == 8, "chunk geometry");
  constexpr int CTP = CT + 4;                         // row pitch of the staged probabilities (the two rows a wave
                                                      // reads at once fall on different banks)
  float *pb = (float *)(lds + 2 * CHUNK);             // [2][AVG_ROWS][CTP] staged probabilities
  __shared__ int rnpos[AVG_ROWS];
  __shared__ long roff[AVG_ROWS];
  __shared__ double rinv[AVG_ROWS];
  const int slice = blockIdx.x, kvh = blockIdx.y, r0 = blockIdx.z * AVG_ROWS, tid = threadIdx.x, wave = tid >> 6,
            lane = tid & 63;
  const bool stager = tid >= 256;
  const int sid = tid - 256;                          // staging thread index (stagers only)
  const int G = a.nHead / a.nHeadKv;
  const uint8_t *vbase = (const uint8_t *)a.vcache +
                         (((long)a.layer * a.nHeadKv + kvh) * a.hd + (long)slice * AVG_DIMS) * a.vstride * VB;
  uint4 pre[LPT];
  float pp[PPT];
  auto fetch = [&](int c, int lim) {
    #pragma unroll
    for (int k = 0; k < LPT; k++) {
      const int idx = k * 256 + sid, dim = idx / PPR, t = c * CT + (idx % PPR) * EPP;
      pre[k] = t < lim ? *(const uint4 *)(vbase + ((long)dim * a.vstride + t) * VB) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
    #pragma unroll
    for (int k = 0; k < LPT; k++) {
      const int idx = k * 256 + sid;
      *(uint4 *)(lds + buf * CHUNK + (idx / PPR) * PITCH + (idx % PPR) * 16) = pre[k];
    }
  };
  if (stager) fetch(0, a.ctx);
  const Step *st = a.step;
  const int Bd = st->B, pos0 = st->pos0;
  // the group's rows: their scores rows, last positions (0: no row) and 1 / sum
  if (tid < AVG_ROWS) {
    const int r = r0 + tid, b = r / G, h = kvh * G + r % G;
    const bool live = r < nrows && b < Bd;
    rnpos[tid] = live ? pos0 + b + 1 : 0;
    roff[tid] = live ? ((long)b * a.nHead + h) * a.sld : 0;
    rinv[tid] = live ? a.pinv[(long)b * a.nHead + h] : 0.0;
  }
  __syncthreads();
  int nmax = 0;
  #pragma unroll
  for (int i = 0; i < AVG_ROWS; i++) nmax = max(nmax, rnpos[i]);
  if (nmax == 0) return;  // (uniform over the block)
  const int nch = (nmax + CT - 1) / CT;
  // probabilities of chunk c for the group's rows (zero past each row's last position)
  auto pload = [&](int c) {
    #pragma unroll
    for (int k = 0; k < PPT; k++) {
      const int idx = k * 256 + sid, rr = idx / CT, t = c * CT + idx % CT;
      pp[k] = t < rnpos[rr] ? a.scores[roff[rr] + t] : 0.f;
    }
  };
  auto pstore = [&](int buf) {
    #pragma unroll
    for (int k = 0; k < PPT; k++) {
      const int idx = k * 256 + sid, rr = idx / CT;
      pb[(buf * AVG_ROWS + rr) * CTP + idx % CT] = (float)((double)pp[k] * rinv[rr]);
    }
  };
  if (stager) {
    #pragma unroll
    for (int k = 0; k < LPT; k++) {  // the first chunk's pieces from the group's last position on: zeros
      const int t = ((k * 256 + sid) % PPR) * EPP;
      if (t >= nmax) pre[k] = make_uint4(0, 0, 0, 0);
      else if (t + EPP > nmax) {
        uint32_t w[4] = {pre[k].x, pre[k].y, pre[k].z, pre[k].w};
        #pragma unroll
        for (int e = 0; e < EPP; e++)
          if (t + e >= nmax) {
            if (F16KV) w[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
            else w[e] = 0u;
          }
        pre[k] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    pload(0);
    store(0);
    pstore(0);
    if (nch > 1) { fetch(1, nmax); pload(1); }
  }
  __syncthreads();
  // ---- weighted sum: row rl = 2 wave + lane / 32, dimension d = lane mod 32 of the slice, chunk by chunk (waves 0-3)
  const int rl = 2 * (wave & 3) + (lane >> 5), d = lane & 31;
  float o = 0.f;
  for (int c = 0; c < nch; c++) {
    if (stager) {
      // chunk c + 1 into the buffer the chains left at the last barrier, then the loads of chunk c + 2
      if (c + 1 < nch) {
        store((c + 1) & 1);
        pstore((c + 1) & 1);
        if (c + 2 < nch) { fetch(c + 2, nmax); pload(c + 2); }
      }
    } else {
      const int cnt = min(CT, nmax - c * CT), nu = (cnt + AV_UNIT - 1) / AV_UNIT;
      const uint8_t *row = lds + (c & 1) * CHUNK + d * PITCH;
      const float *pc = pb + ((c & 1) * AVG_ROWS + rl) * CTP;
      float4 pa[AV_UNIT / 4], pbv[AV_UNIT / 4];
      uint4 va[AV_UNIT * VB / 16], vb[AV_UNIT * VB / 16];
      auto read = [&](int u, float4 (&pv)[AV_UNIT / 4], uint4 (&vv)[AV_UNIT * VB / 16]) {
        #pragma unroll
        for (int k = 0; k < AV_UNIT / 4; k++) pv[k] = *(const float4 *)(pc + u * AV_UNIT + 4 * k);
        #pragma unroll
        for (int k = 0; k < AV_UNIT * VB / 16; k++) vv[k] = *(const uint4 *)(row + (u * AV_UNIT + k * EPP) * VB);
      };
      auto steps = [&](const float4 (&pv)[AV_UNIT / 4], const uint4 (&vv)[AV_UNIT * VB / 16]) {
        #pragma unroll
        for (int k = 0; k < AV_UNIT / 4; k++) {
          float v0, v1, v2, v3;
          if (F16KV) {
            const uint4 &w = vv[k >> 1];
            const uint32_t lo = (k & 1) ? w.z : w.x, hi = (k & 1) ? w.w : w.y;
            v0 = h2f((uint16_t)(lo & 0xffff)); v1 = h2f((uint16_t)(lo >> 16));
            v2 = h2f((uint16_t)(hi & 0xffff)); v3 = h2f((uint16_t)(hi >> 16));
          } else {
            const uint4 &w = vv[k];
            v0 = __uint_as_float(w.x); v1 = __uint_as_float(w.y); v2 = __uint_as_float(w.z); v3 = __uint_as_float(w.w);
          }
          o = fmaf(pv[k].x, v0, o); o = fmaf(pv[k].y, v1, o); o = fmaf(pv[k].z, v2, o); o = fmaf(pv[k].w, v3, o);
        }
      };
      read(0, pa, va);
      int u = 0;
      for (; u + 2 <= nu; u += 2) {
        read(u + 1, pbv, vb);
        __builtin_amdgcn_sched_barrier(0);
        steps(pa, va);
        read(min(u + 2, nu - 1), pa, va);
        __builtin_amdgcn_sched_barrier(0);
        steps(pbv, vb);
      }
      if (u < nu) steps(pa, va);
    }
    __syncthreads();
  }
  if (!stager && rnpos[rl] > 0) {  // (the same for the 32 lanes of the row)
    const int r = r0 + rl, b = r / G, h = kvh * G + r % G, dim = slice * AVG_DIMS + d, col = h * a.hd + dim;
    if (a.gate) {  // gated attention output (src/model/forward-qwen35.js:103): o * sigmoid(gate), f64, stored f32
      const double g = (double)a.gate[(long)b * a.ldq + (long)h * a.qhs + dim];
      o = (float)((double)o * (1.0 / (1.0 + exp(-g))));
    }
    if (a.out) a.out[(long)b * a.ldo + col] = o;
    if (a.act.q) quant_block32(o, col, a.act, b);  // (unset: the output GEMV quantises the f32 rows itself)
  }
}

// LDS of a grouped block with chunks of rowb bytes per dimension: two staged V chunks and two chunks of probabilities
size_t attention_group_lds(int kvF16, int rowb) {
  return (size_t)2 * AVG_DIMS * (rowb + 16) + (size_t)2 * AVG_ROWS * (rowb / (kvF16 ? 2 : 4) + 4) * 4;
}

template <bool F16KV, int ROWB>
static void launch_av_group_k(const AttnArgs &a, dim3 grid, int nrows, hipStream_t st) {
  static size_t attr = 64 * 1024;  // dynamic LDS above 64 KB must be requested per kernel
  const size_t lds = attention_group_lds(F16KV, ROWB);
  if (lds > attr) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_attn_av_group<F16KV, ROWB>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr = lds;
  }
  hipLaunchKernelGGL((k_attn_av_group<F16KV, ROWB>), grid, dim3(AVG_THREADS), lds, st, a, nrows);
}

template <int HD, bool F16KV>
static void launch_av_head_k(const AttnArgs &a, int B, hipStream_t st) {
  static size_t attr = 64 * 1024;
  const size_t lds = attention_head_lds(HD);
  if (lds > attr) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_attn_av_head<HD, F16KV>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr = lds;
  }
  hipLaunchKernelGGL((k_attn_av_head<HD, F16KV>), dim3(1, a.nHead, B), dim3(256), lds, st, a);
}

// ---- position-split weighted sum (long contexts). The exact chain above runs one dependent f32 step per position, so
// at 16K positions it is ~40 us per output element. Here one block per (256-position chunk, query head, token) takes
// the chunk's scores, its max m_c, e_t = exp(s_t - m_c) and l_c = sum e_t in f64, and o_c[i] = sum e_t V_t,i in f64
// (V staged through LDS with coalesced loads); k_attn_merge then forms out_i = f32(sum_c w_c o_c[i] / sum_c w_c l_c),
// w_c = exp(m_c - max_c m_c), adding the chunks in chunk order. Every order is a function of the position count only,
// so batched and single-token passes agree bit for bit. The result is the softmax-weighted sum in f64, rounded once:
// it differs from the reference's f32 chain (src/model/forward.js:134-139) by that chain's own rounding error.
template <bool F16KV>
__global__ __launch_bounds__(256) void k_attn_av_split(const AttnArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int VB = F16KV ? 2 : 4, C = ATTN_SPLIT_C, EPP = 16 / VB;
  __shared__ double e[C];
  __shared__ double redd[4];
  __shared__ float redf[4];
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hd = a.hd, kvh = h / (a.nHead / a.nHeadKv), t0 = c * C;
  const Step *st = a.step;
  if (b >= st->B) return;
  const int npos = st->pos0 + b + 1;
  if (t0 >= npos) return;
  const int cnt = min(C, npos - t0);
  // V rows of the chunk [hd][C] (dimension-major cache rows), 16 bytes per load, consecutive threads along a row
  const uint8_t *vbase = (const uint8_t *)a.vcache + ((long)a.layer * a.nHeadKv + kvh) * hd * a.vstride * VB;
  // LDS row pitch of C * VB + 4 bytes (an odd number of words): the lanes of a wave, one dimension each, read the same
  // position of consecutive rows from distinct banks
  const int ppr = C / EPP, pitch = C * VB + 4;  // 16-byte pieces per row
  for (int idx = tid; idx < hd * ppr; idx += 256) {
    const int dim = idx / ppr, t = t0 + (idx % ppr) * EPP;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (t < npos) v = *(const uint4 *)(vbase + ((long)dim * a.vstride + t) * VB);
    uint32_t *d = (uint32_t *)(lds + (long)dim * pitch + (idx % ppr) * 16);
    d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
  }
  const float *srow = a.scores + ((long)b * a.nHead + h) * a.sld + t0;
  const float s = tid < cnt ? srow[tid] : -INFINITY;
  float mx = group_fmax(s, 64);
  if (lane == 0) redf[wave] = mx;
  __syncthreads();
  const float m = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  const double ev = tid < cnt ? exp((double)s - (double)m) : 0.0;
  e[tid] = ev;
  double l = wave_sum_xor(ev, 64);
  if (lane == 0) redd[wave] = l;
  __syncthreads();
  l = (redd[0] + redd[1]) + (redd[2] + redd[3]);
  // o_c[i]: thread (i = tid mod hd, q = tid / hd) adds positions q, q + R, ... (R = 256 / hd), then the R partial sums
  // meet in LDS in q order
  const int R = 256 / hd, i = tid % hd, q = tid / hd;
  double o = 0.0;
  const uint8_t *row = lds + (long)i * pitch;
  for (int t = q; t < cnt; t += R) {
    const float v = F16KV ? h2f(((const uint16_t *)row)[t]) : ((const float *)row)[t];
    o = fma(e[t], (double)v, o);
  }
  __syncthreads();  // the staged V is no longer read: its LDS holds the partial sums
  double *po = (double *)lds;
  po[tid] = o;
  __syncthreads();
  if (tid < hd) {
    double tot = po[tid];
    for (int k = 1; k < R; k++) tot += po[k * hd + tid];
    double *dst = a.part + (((long)b * a.nHead + h) * a.nch + c) * (hd + 2);
    dst[2 + tid] = tot;
    if (tid == 0) { dst[0] = (double)m; dst[1] = l; }
  }
}

__global__ __launch_bounds__(256) void k_attn_merge(const AttnArgs a) {
  const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x, hd = a.hd;
  const Step *st = a.step;
  if (b >= st->B || i >= hd) return;
  const int npos = st->pos0 + b + 1, nch = (npos + ATTN_SPLIT_C - 1) / ATTN_SPLIT_C;
  const double *pr = a.part + ((long)b * a.nHead + h) * a.nch * (hd + 2);
  double M = -INFINITY;
  for (int c = 0; c < nch; c++) M = fmax(M, pr[(long)c * (hd + 2)]);
  double L = 0.0, O = 0.0;
  for (int c = 0; c < nch; c++) {
    const double *pc = pr + (long)c * (hd + 2);
    const double w = exp(pc[0] - M);
    L += w * pc[1];
    O += w * pc[2 + i];
  }
  float o = (float)(O / L);
  const int col = h * hd + i;
  if (a.gate) {  // gated attention output (src/model/forward-qwen35.js:103): o * sigmoid(gate), f64, stored f32
    const double g = (double)a.gate[(long)b * a.ldq + (long)h * a.qhs + i];
    o = (float)((double)o * (1.0 / (1.0 + exp(-g))));
  }
  if (a.out) a.out[(long)b * a.ldo + col] = o;
  if (a.act.q) quant_block32(o, col, a.act, b);  // (unset: the output GEMV quantises the f32 rows itself)
}

size_t attention_split_lds(int hd, int kvF16) { return (size_t)hd * (ATTN_SPLIT_C * (kvF16 ? 2 : 4) + 4); }

// Dynamic LDS of one k_attn_av block: the probabilities of ctx positions and two staged V chunks (of AV_ROW or rowb
// bytes per dimension).
size_t attention_lds(int ctx, int rowb) {
  return (size_t)((ctx + AV_UNIT - 1) / AV_UNIT * AV_UNIT) * 4 + 2 * (size_t)AV_DIMS * (rowb + 16);
}
size_t attention_lds(int ctx) { return attention_lds(ctx, AV_ROW); }
constexpr size_t ATTN_LDS_MAX = 150 * 1024;

// Contexts above AVH_CTX positions take the per-head weighted sum (heads of at most 128 dimensions), whose LDS does not
// depend on the context, for passes of several tokens; single-token passes keep the slice form wherever its softmax
// row fits LDS. ZEROLLM_ATTN_HEAD_CTX / ZEROLLM_ATTN_HEAD1_CTX override the two thresholds (tests). Read once per model.
AttnForm attention_form(int ctx, int hd) {
  const char *e = getenv("ZEROLLM_ATTN_HEAD_CTX"), *e1 = getenv("ZEROLLM_ATTN_HEAD1_CTX");
  AttnForm f;
  f.headCtx = hd > 128 ? INT_MAX : e ? atoi(e) : AVH_CTX;
  // single-token passes: the per-head form once the slice form's LDS no longer holds the row
  int fit = 0;
  while (fit < ctx && attention_lds(fit + AV_UNIT) <= ATTN_LDS_MAX) fit += AV_UNIT;
  f.head1Ctx = hd > 128 ? INT_MAX : e1 ? atoi(e1) : std::max(f.headCtx, fit);
  f.split = ctx > f.headCtx ? false : attention_lds(ctx) > ATTN_LDS_MAX;
  // matrix-core score dots for passes of 16 tokens or more (prefill chunks), and of 2 or more where the context is long
  // (verify passes at long contexts); ZEROLLM_ATTN_MM_B overrides the token count (tests)
  const char *em = getenv("ZEROLLM_ATTN_MM_B");
  f.mmMinB = em ? atoi(em) : ctx >= AVH_CTX ? 2 : 16;
  // their weighted sums on the matrix cores likewise: from 16 tokens on (32-row blocks), and from 2 where the context
  // is long (16-row blocks: 9-token verify passes at 16K positions 10.77 -> 10.52 ms against the grouped lane chains)
  const char *ea = getenv("ZEROLLM_ATTN_MMAV_B");
  f.mmAvMinB = ea ? atoi(ea) : em ? f.mmMinB : ctx >= AVH_CTX ? 2 : 16;
  // where the slice form's softmax row would not fit LDS (256-dimension heads beyond ~29,900 positions) every pass
  // takes the matrix-core weighted sum, whose staging does not grow with the context: the exact chain at any context
  if (f.split) {
    f.split = false;
    f.mmAvMinB = 1;
  }
  // the slice form's chains on the matrix cores from AV_BIG_CTX positions, where the lane-chain form's LDS already
  // holds a CU to one block (ZEROLLM_ATTN_AVMF=1 / 0: at any context / never; the same bits)
  const char *ev = getenv("ZEROLLM_ATTN_AVMF");
  f.avmf = ctx <= AVM_MAX_CTX && (ev ? ev[0] == '1' : ctx >= AV_BIG_CTX);
  return f;
}

template <bool F16KV, int RB>
static void launch_av_mm_k(const AttnArgs &a, int nrows, hipStream_t st) {
  static bool attr = false;  // dynamic LDS above 64 KB must be requested per kernel
  if (!attr) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_attn_av_mm<F16KV, RB>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)attention_av_mm_lds(RB)));
    attr = true;
  }
  const int nb = a.hd / AV_DIMS * a.nHeadKv * ((nrows + RB - 1) / RB);  // (slice, KV head, row block) blocks
  const dim3 grid((nb + 7) / 8 * 8);
  hipLaunchKernelGGL((k_attn_av_mm<F16KV, RB>), grid, dim3(RB * 16), attention_av_mm_lds(RB), st, a, nrows);
}

template <int HD, bool F16KV>
static void launch_scores_mm(const AttnArgs &a, dim3 gp, int nrows, hipStream_t st) {
  constexpr bool canWide = HD <= 128;  // (256-dimension rows in 8-wave blocks would spill)
  static bool attr = false;  // dynamic LDS above 64 KB must be requested per kernel
  if (!attr) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_attn_scores_mm<HD, F16KV, 4>, hipFuncAttributeMaxDynamicSharedMemorySize, 140 * 1024));
    if constexpr (canWide)
      ZL_HIP(hipFuncSetAttribute((const void *)k_attn_scores_mm<HD, F16KV, 8>, hipFuncAttributeMaxDynamicSharedMemorySize, 140 * 1024));
    attr = true;
  }
  hipLaunchKernelGGL((k_attn_prep<HD, F16KV>), gp, dim3(64), 0, st, a);
  // as many position blocks per (KV head, row group) as stay resident together (LDS bounds the blocks per CU, and the
  // registers of 8-wave blocks one per CU), at most one per tile of the cache: a pass's tiles then spread over them in
  // one round
  const bool wide = canWide && nrows >= 128;
  const int nwv = wide ? 8 : 4, zg = (nrows + 16 * nwv - 1) / (16 * nwv), ntc = (a.ctx + MM_PT - 1) / MM_PT;
  const size_t lds = attention_mm_lds(HD);
  const int slots = 256 * (wide ? 1 : std::max(1, (int)(160 * 1024 / lds)));
  const dim3 gm((unsigned)std::max(1, std::min(ntc, slots / (a.nHeadKv * zg))), a.nHeadKv, zg);
  if constexpr (canWide) {
    if (wide) {
      hipLaunchKernelGGL((k_attn_scores_mm<HD, F16KV, 8>), gm, dim3(512), lds, st, a, nrows);
      return;
    }
  }
  hipLaunchKernelGGL((k_attn_scores_mm<HD, F16KV, 4>), gm, dim3(256), lds, st, a, nrows);
}

template <int HD, bool F16KV>
static void launch_scores_k(const AttnArgs &a, dim3 grid, int B, hipStream_t st) {
  const size_t kn = (size_t)std::min(64, B) * HD * (F16KV ? 2 : 4);
  hipLaunchKernelGGL((k_attn_scores<HD, F16KV>), grid, dim3(256), kn, st, a);
}

template <bool F16KV, int ROWB>
static void launch_av_rows(const AttnArgs &a, dim3 grid, size_t lds, hipStream_t st) {
  static size_t attr = 64 * 1024;  // dynamic LDS above 64 KB must be requested per kernel
  if (lds > attr) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_attn_av<F16KV, ROWB>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr = lds;
  }
  hipLaunchKernelGGL((k_attn_av<F16KV, ROWB>), grid, dim3(256), lds, st, a);
}

// the larger chunk for long contexts where it fits (the same bits: only the staging changes); at short contexts its
// LDS would halve the blocks a CU holds (measured: 5-token verify pass 3.11 -> 3.32 ms at 1024 positions)
template <bool F16KV>
static void launch_av_k(const AttnArgs &a, dim3 grid, size_t lds, hipStream_t st) {
  const size_t big = attention_lds(a.ctx, AV_ROW_BIG);
  if (a.ctx >= AV_BIG_CTX && big <= ATTN_LDS_MAX) launch_av_rows<F16KV, AV_ROW_BIG>(a, grid, big, st);
  else launch_av_rows<F16KV, AV_ROW>(a, grid, lds, st);
}

template <bool F16KV>
static void launch_av_mfma_k(const AttnArgs &a, dim3 grid, size_t lds, hipStream_t st) {
  static size_t attr = 64 * 1024;  // dynamic LDS above 64 KB must be requested per kernel
  if (lds > attr) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_attn_av_mfma<F16KV>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr = lds;
  }
  hipLaunchKernelGGL((k_attn_av_mfma<F16KV>), grid, dim3(256), lds, st, a);
}

template <bool F16KV>
static void launch_av_split_k(const AttnArgs &a, dim3 grid, size_t lds, hipStream_t st) {
  static size_t attr = 64 * 1024;
  if (lds > attr) {
    ZL_HIP(hipFuncSetAttribute((const void *)k_attn_av_split<F16KV>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr = lds;
  }
  hipLaunchKernelGGL((k_attn_av_split<F16KV>), grid, dim3(256), lds, st, a);
}

void launch_attention(const AttnArgs &a0, int B, hipStream_t st) {
  AttnArgs a = a0;
  // the per-head form for passes of several tokens at long contexts (single-token passes keep the four slice blocks
  // per head, which stage a quarter of the rows each, wherever their softmax row fits LDS); both give the same bits
  const bool head = !a.part && a.ctx > (B > 1 ? a.headCtx : a.head1Ctx);
  // the weighted-sum form: split, the matrix cores, or the lane chains (grouped, per-head or slice form); only the
  // slice form's LDS grows with the context
  const bool avmm = !a.part && a.qr && a.mmAvMinB > 0 && B >= a.mmAvMinB;
  const size_t lds = a.part ? attention_split_lds(a.hd, a.kvF16) : avmm ? 0 : head ? attention_head_lds(a.hd) : attention_lds(a.ctx);
  ZL_REQUIRE(lds <= ATTN_LDS_MAX, ZL_ERR_UNSUPPORTED, "context too long for the attention kernel");
  ZL_REQUIRE(!a.part || a.nch * ATTN_SPLIT_C >= a.ctx, ZL_ERR_ARG, "attention: split partials below the context");
  ZL_REQUIRE(a.hd == 64 || a.hd == 128 || a.hd == 256, ZL_ERR_UNSUPPORTED, "attention: head_dim must be 64, 128 or 256");
  ZL_REQUIRE(a.sld >= a.ctx, ZL_ERR_ARG, "attention: score stride below the context");
  ZL_REQUIRE(a.qhs >= a.hd && a.ldq >= a.nHead * a.qhs, ZL_ERR_ARG, "attention: query head stride below the head size");
  const int group = a.nHead / a.nHeadKv;
  a.hpb = attn_heads_per_block(group);
  const int chunks = (a.ctx + attn_score_chunk(a.hd) - 1) / attn_score_chunk(a.hd);
  if (a.qr && a.mmMinB > 0 && B >= a.mmMinB) {
    const dim3 gp(B, a.nHead + a.nHeadKv);
    const int nrows = B * group;
    switch (a.hd * 2 + a.kvF16) {
      case 128: launch_scores_mm<64, false>(a, gp, nrows, st); break;
      case 129: launch_scores_mm<64, true>(a, gp, nrows, st); break;
      case 256: launch_scores_mm<128, false>(a, gp, nrows, st); break;
      case 257: launch_scores_mm<128, true>(a, gp, nrows, st); break;
      case 512: launch_scores_mm<256, false>(a, gp, nrows, st); break;
      case 513: launch_scores_mm<256, true>(a, gp, nrows, st); break;
    }
  } else {
    dim3 gs(chunks < 64 ? chunks : 64, a.nHead / a.hpb, B);
    switch (a.hd * 2 + a.kvF16) {
      case 128: launch_scores_k<64, false>(a, gs, B, st); break;
      case 129: launch_scores_k<64, true>(a, gs, B, st); break;
      case 256: launch_scores_k<128, false>(a, gs, B, st); break;
      case 257: launch_scores_k<128, true>(a, gs, B, st); break;
      case 512: launch_scores_k<256, false>(a, gs, B, st); break;
      case 513: launch_scores_k<256, true>(a, gs, B, st); break;
    }
  }
  ZL_HIP(hipGetLastError());
  if (a.part) {
    const dim3 gv(a.nch, a.nHead, B);
    if (a.kvF16) launch_av_split_k<true>(a, gv, lds, st);
    else launch_av_split_k<false>(a, gv, lds, st);
    ZL_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_attn_merge, dim3(a.nHead, B), dim3(std::max(64, a.hd)), 0, st, a);
    ZL_HIP(hipGetLastError());
    return;
  }
  if (avmm) {
    // the probabilities of every row, then the weighted sums on the matrix cores, 16 or 32 rows x 32 dimensions per block
    hipLaunchKernelGGL(k_attn_softmax_rows<true>, dim3(1, a.nHead, B), dim3(SMR_T), 0, st, a);
    const int nrows = group * B;
    // 32-row blocks (V staged once for two tiles) where they still give every CU a block (prefill chunks of the 8B
    // shapes), 16-row blocks otherwise (verify passes, the 0.6B shapes' chunks: 128 rows per KV head)
    const bool rb32 = (nrows + 31) / 32 * (a.hd / AV_DIMS) * a.nHeadKv >= 256;
    if (a.kvF16) {
      if (rb32) launch_av_mm_k<true, 32>(a, nrows, st);
      else launch_av_mm_k<true, 16>(a, nrows, st);
    } else {
      if (rb32) launch_av_mm_k<false, 32>(a, nrows, st);
      else launch_av_mm_k<false, 16>(a, nrows, st);
    }
    ZL_HIP(hipGetLastError());
    return;
  }
  if (head && B > 1 && a.pinv) {
    // grouped by KV head: the softmax rows, then each V chunk staged once for a group's rows
    hipLaunchKernelGGL(k_attn_softmax_rows<false>, dim3(1, a.nHead, B), dim3(SMR_T), 0, st, a);
    const int nrows = (a.nHead / a.nHeadKv) * B;
    const dim3 gg(a.hd / AVG_DIMS, a.nHeadKv, (nrows + AVG_ROWS - 1) / AVG_ROWS);
    // 1024-byte chunks (512 f16 / 256 f32 positions): each chunk's chain is long enough to cover the next chunk's loads
    if (a.kvF16) launch_av_group_k<true, AV_ROW_BIG>(a, gg, nrows, st);
    else launch_av_group_k<false, AV_ROW_BIG>(a, gg, nrows, st);
    ZL_HIP(hipGetLastError());
    return;
  }
  if (head) {
    switch (a.hd * 2 + a.kvF16) {
      case 128: launch_av_head_k<64, false>(a, B, st); break;
      case 129: launch_av_head_k<64, true>(a, B, st); break;
      case 256: launch_av_head_k<128, false>(a, B, st); break;
      case 257: launch_av_head_k<128, true>(a, B, st); break;
    }
    ZL_HIP(hipGetLastError());
    return;
  }
  dim3 ga(a.hd / AV_DIMS, a.nHead, B);
  if (a.avmf) {
    ZL_REQUIRE(a.ctx <= AVM_MAX_CTX, ZL_ERR_ARG, "attention: matrix-core slice form beyond its context");
    const size_t lm = attention_av_mfma_lds();
    if (a.kvF16) launch_av_mfma_k<true>(a, ga, lm, st);
    else launch_av_mfma_k<false>(a, ga, lm, st);
  } else if (a.kvF16) {
    launch_av_k<true>(a, ga, lds, st);
  } else {
    launch_av_k<false>(a, ga, lds, st);
  }
  ZL_HIP(hipGetLastError());
}

}  // namespace zl
