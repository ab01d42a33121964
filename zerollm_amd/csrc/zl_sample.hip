// On-device sampling for the speculative step: the sampler's distribution() and draw(), the draft's proposal draws,
// and the acceptance test with residual / bonus draws, so that only accepted token ids leave the GPU.
//
// Semantics follow zerollm's createSampler (src/sampling/sampler.js:81-155), generateSpeculative's accept block
// (src/model/speculative.js:192-209), probOf (:64-67) and drawResidual (:75-87). The f64 arithmetic after the
// candidate selection is sequential in one lane, in the reference's order, so a seeded run consumes the same uniforms
// and takes the same decisions as the reference given the same logits.
#include "zl_kernels.h"

#include <algorithm>

namespace zl {

// mulberry32 (src/util/rng.js:4-13)
__device__ inline double rng_next(uint32_t &a) {
  a = a + 0x6d2b79f5u;
  uint32_t t = a;
  t = (t ^ (t >> 15)) * (t | 1u);
  t ^= t + (t ^ (t >> 7)) * (t | 61u);
  return (double)(t ^ (t >> 14)) / 4294967296.0;
}

// Exact zerollm heap (src/sampling/sampler.js:21-43) for the rare case of ties at the k-th value: which of the tied
// candidates survive depends on the heap's history, so it is replayed literally. One thread; out holds k entries.
__device__ int heap_topk(const float *l, int n, int k, int *ids, double *vals) {
  int size = 0;
  for (int i = 0; i < n; i++) {
    double v = (double)l[i];
    if (size < k) {
      ids[size] = i; vals[size] = v; size++;
      int j = size - 1;
      while (j > 0) {
        int p = (j - 1) >> 1;
        if (vals[j] >= vals[p]) break;
        int ti = ids[j]; ids[j] = ids[p]; ids[p] = ti; double tv = vals[j]; vals[j] = vals[p]; vals[p] = tv;
        j = p;
      }
    } else if (v > vals[0]) {
      ids[0] = i; vals[0] = v;
      int j = 0;
      for (;;) {
        int le = 2 * j + 1, ri = le + 1, m = j;
        if (le < size && vals[le] < vals[m]) m = le;
        if (ri < size && vals[ri] < vals[m]) m = ri;
        if (m == j) break;
        int ti = ids[j]; ids[j] = ids[m]; ids[m] = ti; double tv = vals[j]; vals[j] = vals[m]; vals[m] = tv;
        j = m;
      }
    }
  }
  return size;
}

constexpr int DT = 1024;  // threads of the distribution kernel

// The digit step of the radix select, on the 64 lanes of one wave: d = the largest digit whose keys, with those of all
// larger digits, number at least rem (0 if there is none), which a scan from digit 255 down finds first; above = the
// number of keys of the digits above d. Lane L holds digits 4L .. 4L + 3; the suffix counts are integer sums, so the
// result is the scan's.
__device__ inline void radix_digit(const uint32_t *hc, uint32_t rem, int lane, int &d, uint32_t &above) {
  const uint32_t h0 = hc[4 * lane], h1 = hc[4 * lane + 1], h2 = hc[4 * lane + 2], h3 = hc[4 * lane + 3];
  const uint32_t loc = h0 + h1 + h2 + h3;
  uint32_t suf = loc;  // keys of the digits of lanes L' >= L
  #pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_down(suf, o, 64);
    if (lane + o < 64) suf += t;
  }
  const uint32_t s3 = suf - loc + h3, s2 = s3 + h2, s1 = s2 + h1, s0 = s1 + h0;  // keys of digits >= 4L + 3 .. >= 4L
  int c = (s0 >= rem) + (s1 >= rem) + (s2 >= rem) + (s3 >= rem);  // the digits that qualify are 0 .. d
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
  d = c > 0 ? c - 1 : 0;
  uint32_t a = (4 * lane > d ? h0 : 0u) + (4 * lane + 1 > d ? h1 : 0u) + (4 * lane + 2 > d ? h2 : 0u) +
               (4 * lane + 3 > d ? h3 : 0u);
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
  above = a;
}

// First stage of the two-stage selection: block (c, r) radix-selects the K-th largest key among logits
// [c CAND_CHUNK, (c + 1) CAND_CHUNK) of row r and lists every logit at or above it (all of them when the block holds at
// most K). Every logit of the row's top K is in its block's list (fewer than K logits of the row, hence of the block, lie
// above it), and so is every logit equal to the row's K-th largest: the row's selection over the lists finds the same
// K-th key, the same count of keys equal to it and the same candidates as over the whole row. A list longer than cmax
// is reported by its count, and the row then selects over the whole row.
constexpr int CT_T = 256;                   // threads of the candidate kernel (one per digit)
constexpr int CT_PER = CAND_CHUNK / CT_T;   // logits per thread
__global__ __launch_bounds__(CT_T) void k_topk_cand(const float *__restrict__ logits, int ldl, int vocab, int K,
                                                  int cmax, CandWork cw) {
  __shared__ uint32_t hc[256];
  __shared__ uint32_t s_prefix, s_mask, s_rem;
  __shared__ int s_n;
  const int c = blockIdx.x, r = blockIdx.y, nb = gridDim.x, tid = threadIdx.x;
  const int i0 = c * CAND_CHUNK, n = min(vocab - i0, CAND_CHUNK);
  const float *l = logits + (long)r * ldl + i0;
  float v[CT_PER];
  uint32_t k[CT_PER];
  #pragma unroll
  for (int j = 0; j < CT_PER; j++) {
    const int i = j * CT_T + tid;
    v[j] = l[i < n ? i : 0];
    k[j] = fkey(v[j]);
  }
  if (tid == 0) { s_prefix = 0; s_mask = 0; s_rem = (uint32_t)K; s_n = 0; }
  __syncthreads();
  if (n > K) {  // (uniform over the block)
    for (int shift = 24; shift >= 0; shift -= 8) {
      hc[tid] = 0;
      __syncthreads();
      const uint32_t prefix = s_prefix, mask = s_mask;
      #pragma unroll
      for (int j = 0; j < CT_PER; j++)
        if (j * CT_T + tid < n && (k[j] & mask) == prefix) atomicAdd(&hc[(k[j] >> shift) & 255u], 1u);
      __syncthreads();
      if (tid < 64) {
        int d;
        uint32_t above;
        radix_digit(hc, s_rem, tid, d, above);
        if (tid == 0) {
          s_rem -= above;
          s_prefix = prefix | ((uint32_t)d << shift);
          s_mask = mask | (255u << shift);
        }
      }
      __syncthreads();
    }
  }
  const uint32_t T = n > K ? s_prefix : 0u;
  const long base = ((long)r * nb + c) * cmax;
  #pragma unroll
  for (int j = 0; j < CT_PER; j++) {
    const int i = j * CT_T + tid;
    if (i < n && k[j] >= T) {
      const int p = atomicAdd(&s_n, 1);
      if (p < cmax) { cw.ids[base + p] = i0 + i; cw.vals[base + p] = v[j]; }
    }
  }
  __syncthreads();
  if (tid == 0) cw.cnt[r * nb + c] = s_n;
}

// Candidates of a row the distribution kernel gathers into LDS (more: it selects over the whole row).
constexpr int CAND_LDS = 6144;

// The row's logits copied to cp with the repetition / presence / frequency penalties of the last repeatLastN history ids
// applied (src/sampling/sampler.js:96-110), in the reference's order (distinct ids in first-occurrence order). Every
// thread of the block calls it.
__device__ void penalized_copy(const float *l, float *cp, int vocab, const SamplerParams &sp, const int *hist, int hl,
                               bool penalize) {
  const int tid = threadIdx.x;
  for (int i = tid; i < vocab; i += blockDim.x) cp[i] = l[i];
  __syncthreads();
  if (penalize && tid == 0) {
    int start = hl - sp.repeatLastN;
    if (start < 0) start = 0;
    for (int i = start; i < hl; i++) {
      int t = hist[i];
      bool seen = false;
      for (int j = start; j < i; j++) if (hist[j] == t) { seen = true; break; }
      if (seen) continue;
      int c = 0;
      for (int j = i; j < hl; j++) c += hist[j] == t;
      double lv = (double)cp[t];
      double v = sp.repeatPenalty != 1.0 ? (lv > 0 ? lv / sp.repeatPenalty : lv * sp.repeatPenalty) : lv;
      v -= (double)c * sp.frequency + sp.presence;
      cp[t] = (float)v;
    }
  }
  __syncthreads();
  __threadfence_block();
}

// distribution(logits row, history) for nrows rows (src/sampling/sampler.js:94-142).
// cw.ids set: the first stage's lists of nb blocks per row (cmax entries each) to select from.
__global__ __launch_bounds__(DT) void k_dist_rows(const float *__restrict__ logits, int ldl, int vocab, SamplerParams sp,
                                                 const int *hist, int histLen0, int histInc, float *scratch, CandWork cw,
                                                 int nb, int cmax, DevDist *out) {
  __shared__ uint32_t hcount[256];
  __shared__ int s_ids[KCAP];
  __shared__ double s_vals[KCAP];
  __shared__ int o_ids[KCAP];
  __shared__ double o_vals[KCAP];
  __shared__ uint32_t s_prefix, s_mask, s_remaining, s_eqcount;
  __shared__ int s_ncand;
  __shared__ float s_bestv[DT / 64];
  __shared__ int s_besti[DT / 64];
  const int r = blockIdx.x, tid = threadIdx.x;
  const float *l = logits + (long)r * ldl;
  DevDist *D = out + r;
  // ---- penalties on a private copy (the reference modifies and restores the caller's buffer)
  const int hl = hist ? histLen0 + r * histInc : 0;
  if (sp.penalized && hl > 0) {
    float *cp = scratch + (long)r * vocab;
    penalized_copy(l, cp, vocab, sp, hist, hl, true);
    l = cp;
  }
  // ---- greedy: first maximum (src/sampling/sampler.js:46-50)
  if (sp.temperature <= 0.0 || sp.greedyArgmax) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = tid; i < vocab; i += DT) {
      float v = l[i];
      if (v > bv) { bv = v; bi = i; }
    }
    for (int o = 1; o < 64; o <<= 1) {
      float ov = __shfl_xor(bv, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((tid & 63) == 0) { s_bestv[tid >> 6] = bv; s_besti[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
      float b = s_bestv[0];
      int id = s_besti[0];
      for (int w = 1; w < DT / 64; w++)
        if (s_bestv[w] > b || (s_bestv[w] == b && s_besti[w] < id)) { b = s_bestv[w]; id = s_besti[w]; }
      if (id == 0x7fffffff) id = 0;  // every logit NaN: the reference's argmax also returns 0
      D->n = 1; D->greedy = 1; D->total = 1.0; D->ids[0] = id; D->probs[0] = 1.0;
    }
    return;
  }
  const int K = sp.topK;
  // ---- the first stage's candidates of this row into LDS, unless a list overflowed or they are too many
  __shared__ float c_val[CAND_LDS];
  __shared__ int c_id[CAND_LDS];
  __shared__ int s_off[CAND_MAXB + 1];
  __shared__ int s_cand;
  bool cand = cw.ids != nullptr;
  if (cand) {
    if (tid < 64) {  // exclusive prefix of the blocks' counts, two blocks per lane
      const int b0 = 2 * tid, b1 = 2 * tid + 1;
      const int n0 = b0 < nb ? cw.cnt[r * nb + b0] : 0, n1 = b1 < nb ? cw.cnt[r * nb + b1] : 0;
      int ovf = n0 > cmax || n1 > cmax;
      const int loc = n0 + n1;
      int inc = loc;
      #pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (tid >= o) inc += t;
      }
      if (b0 < nb) s_off[b0] = inc - loc;
      if (b1 < nb) s_off[b1] = inc - loc + n0;
      #pragma unroll
      for (int o = 32; o > 0; o >>= 1) ovf |= __shfl_xor(ovf, o, 64);
      const int total = __shfl(inc, 63, 64);
      if (tid == 0) { s_off[nb] = total; s_cand = !ovf && total <= CAND_LDS; }
    }
    __syncthreads();
    cand = s_cand;
    if (cand) {
      const int b = tid >> 3, q = tid & 7;  // eight threads per block's list, eight entries each in flight
      if (b < nb) {
        const int cn = s_off[b + 1] - s_off[b], dst = s_off[b];
        const long src = ((long)r * nb + b) * cmax;
        for (int j0 = q; j0 < cn; j0 += 64) {
          float vv[8];
          int ii[8];
          #pragma unroll
          for (int m = 0; m < 8; m++) {
            const int j = j0 + 8 * m;
            vv[m] = j < cn ? cw.vals[src + j] : 0.f;
            ii[m] = j < cn ? cw.ids[src + j] : 0;
          }
          #pragma unroll
          for (int m = 0; m < 8; m++) {
            const int j = j0 + 8 * m;
            if (j < cn) { c_val[dst + j] = vv[m]; c_id[dst + j] = ii[m]; }
          }
        }
      }
    }
  }
  const int NC = cand ? s_off[nb] : 0;
  // ---- radix select of the K-th largest key
  if (tid == 0) { s_prefix = 0; s_mask = 0; s_remaining = (uint32_t)K; }
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += DT) hcount[i] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    if (cand) {
      for (int i = tid; i < NC; i += DT) {
        const uint32_t kv = fkey(c_val[i]);
        if ((kv & mask) == prefix) atomicAdd(&hcount[(kv >> shift) & 255u], 1u);
      }
    } else {
      // 8 keys per thread requested at a time
      for (int i0 = 0; i0 < vocab; i0 += 8 * DT) {
        uint32_t kv[8];
        #pragma unroll
        for (int j = 0; j < 8; j++) { const int i = i0 + j * DT + tid; kv[j] = i < vocab ? fkey(l[i]) : 0u; }
        #pragma unroll
        for (int j = 0; j < 8; j++)
          if (i0 + j * DT + tid < vocab && (kv[j] & mask) == prefix) atomicAdd(&hcount[(kv[j] >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (tid < 64) {
      int d;
      uint32_t above;
      radix_digit(hcount, s_remaining, tid, d, above);
      if (tid == 0) {
        s_remaining -= above;
        s_eqcount = hcount[d];
        s_prefix = prefix | ((uint32_t)d << shift);
        s_mask = mask | (255u << shift);
      }
    }
    __syncthreads();
  }
  const uint32_t T = s_prefix;
  const bool tie = s_eqcount != s_remaining;
  if (tid == 0) s_ncand = 0;
  __syncthreads();
  if (!tie && cand) {
    for (int i = tid; i < NC; i += DT) {
      const float v = c_val[i];
      if (fkey(v) >= T) {
        const int p = atomicAdd(&s_ncand, 1);
        if (p < KCAP) { s_ids[p] = c_id[i]; s_vals[p] = (double)v; }
      }
    }
  } else if (!tie) {
    for (int i0 = 0; i0 < vocab; i0 += 8 * DT) {
      float v[8];
      #pragma unroll
      for (int j = 0; j < 8; j++) { const int i = i0 + j * DT + tid; v[j] = l[i < vocab ? i : 0]; }
      #pragma unroll
      for (int j = 0; j < 8; j++) {
        const int i = i0 + j * DT + tid;
        if (i < vocab && fkey(v[j]) >= T) {
          int p = atomicAdd(&s_ncand, 1);
          if (p < KCAP) { s_ids[p] = i; s_vals[p] = (double)v[j]; }
        }
      }
    }
  } else if (tid == 0) {
    s_ncand = heap_topk(l, vocab, K, s_ids, s_vals);
  }
  __syncthreads();
  const int m = min(s_ncand, K);
  // ---- sort by value desc, id asc (rank sort)
  for (int i = tid; i < m; i += DT) {
    double vi = s_vals[i];
    int ii = s_ids[i], rank = 0;
    for (int j = 0; j < m; j++) {
      double vj = s_vals[j];
      rank += (vj > vi) || (vj == vi && s_ids[j] < ii);
    }
    o_ids[rank] = ii; o_vals[rank] = vi;
  }
  __syncthreads();
  // ---- softmax with temperature, min-p, top-p (one lane, the reference's order, on LDS; s_vals is free again), then the
  // kept entries written out by all threads
  __shared__ int s_keep;
  double *pr = s_vals;
  if (tid == 0) {
    double mx = o_vals[0], sum = 0;
    for (int i = 0; i < m; i++) { const double e = exp((o_vals[i] - mx) / sp.temperature); pr[i] = e; sum += e; }
    for (int i = 0; i < m; i++) pr[i] = pr[i] / sum;
    int keep = m;
    if (sp.minP > 0) {
      double thr = sp.minP * pr[0];
      keep = 1;
      while (keep < m && pr[keep] >= thr) keep++;
    }
    if (sp.topP < 1) {
      double c = 0;
      int i = 0;
      while (i < keep) { c += pr[i]; i++; if (c >= sp.topP) break; }
      keep = i > 1 ? i : 1;
    }
    double total = 0;
    for (int i = 0; i < keep; i++) total += pr[i];
    s_keep = keep;
    D->n = keep; D->greedy = 0; D->total = total;
  }
  __syncthreads();
  for (int i = tid; i < s_keep; i += DT) { D->ids[i] = o_ids[i]; D->probs[i] = pr[i]; }
}

// Entry i of a distribution, from its fixed list or its full-list storage.
__device__ inline int dist_id(const DevDist &d, int i) { return d.wids ? d.wids[i] : d.ids[i]; }
__device__ inline double dist_p(const DevDist &d, int i) { return d.wprobs ? d.wprobs[i] : d.probs[i]; }

// draw(dist) (src/sampling/sampler.js:145-151)
__device__ inline int draw_dist(const DevDist &d, uint32_t &rng) {
  if (d.greedy) return dist_id(d, 0);
  double r = rng_next(rng) * d.total;
  for (int i = 0; i < d.n; i++) {
    r -= dist_p(d, i);
    if (r <= 0) return dist_id(d, i);
  }
  return dist_id(d, d.n - 1);
}

// probOf (src/model/speculative.js:64-67); a full list finds the id's rank in wpos
__device__ inline double prob_of(const DevDist &d, int id) {
  if (d.wpos) {
    const int k = d.wpos[id];
    return k ? d.wprobs[k - 1] / d.total : 0.0;
  }
  for (int i = 0; i < d.n; i++) if (d.ids[i] == id) return d.probs[i] / d.total;
  return 0.0;
}

// drawResidual (src/model/speculative.js:75-87); the dense scratch of the reference is a lookup into q's support
__device__ int draw_residual(const DevDist &p, const DevDist &q, uint32_t &rng) {
  double resl[KCAP];
  double *res = p.wres ? p.wres : resl;
  double sum = 0;
  for (int i = 0; i < p.n; i++) {
    const double v = dist_p(p, i) / p.total - prob_of(q, dist_id(p, i));
    res[i] = 0.0;
    if (v > 0) { res[i] = v; sum += v; }
  }
  if (!(sum > 0)) return draw_dist(p, rng);
  double r = rng_next(rng) * sum;
  int last = 0;
  for (int i = 0; i < p.n; i++) {
    if (res[i] > 0) {
      last = i;
      r -= res[i];
      if (r <= 0) return dist_id(p, i);
    }
  }
  return dist_id(p, last);
}

// Draft proposal j (src/model/speculative.js:169-177): draw x_j from the draft's distribution, record it, stop after a
// stop token (later calls in the same cycle do nothing, as the reference's loop has ended), and make x_j the next
// draft input and the (j+1)-th verify token.
__global__ void k_draft_draw(const DevDist *dist, SpecState *ss, int j, const int *stopIds, int nStop, Step *draftStep,
                             int advance, Step *targetStep, int *hist, int histLen0) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  if (ss->stopped) return;
  uint32_t rng = ss->rng;
  int x = draw_dist(*dist, rng);
  ss->rng = rng;
  ss->drafted[j] = x;
  ss->kk = j + 1;
  for (int i = 0; i < nStop; i++) if (stopIds[i] == x) ss->stopped = 1;
  draftStep->tokens[0] = x;
  draftStep->pos0 += advance;
  draftStep->B = 1;
  targetStep->tokens[1 + j] = x;
  if (hist) hist[histLen0 + j] = x;
}

// Acceptance (src/model/speculative.js:192-209): greedy compare, or accept with probability min(1, p/q) and on the first
// rejection draw from the residual; when every draft is accepted the bonus token comes from the last row.
// The fixed-list form of the acceptance (distributions of at most KCAP entries): the wave copies each distribution it
// needs into LDS and finds q's probability of every entry of p in parallel; lane 0 then takes the same decisions in
// the same order, with the same arithmetic, as the one-lane form below (prob_of, draw_residual, draw_dist).
__device__ void accept_lists(const DevDist *pdist, const DevDist *qdist, SpecState *ss) {
  __shared__ int pid[KCAP], qid[KCAP];
  __shared__ double ppr[KCAP], qpr[KCAP], qat[KCAP];
  __shared__ double s_px, s_qx;
  const int lane = threadIdx.x;
  auto stage = [&](const DevDist &d, int *ids, double *pr) {
    for (int i = lane; i < d.n; i += 64) { ids[i] = d.ids[i]; pr[i] = d.probs[i]; }
  };
  uint32_t rng = ss->rng;  // every lane steps its own copy of the stream the same way
  const int kk = ss->kk;
  int a = 0, tok = -1;
  for (int j = 0; j < kk; j++) {
    const DevDist &P = pdist[j], &Q = qdist[j];
    const int x = ss->drafted[j], pn = P.n, qn = Q.n;
    stage(P, pid, ppr);
    stage(Q, qid, qpr);
    if (lane == 0) { s_px = 0.0; s_qx = 0.0; }
    __syncthreads();
    for (int i = lane; i < pn; i += 64) if (pid[i] == x) s_px = ppr[i] / P.total;  // ids of a list are distinct
    for (int i = lane; i < qn; i += 64) if (qid[i] == x) s_qx = qpr[i] / Q.total;
    __syncthreads();
    if (rng_next(rng) * s_qx < s_px) { a++; __syncthreads(); continue; }
    // rejected: the residual max(0, p - q) over p's entries
    for (int i = lane; i < pn; i += 64) {
      double v = 0.0;
      for (int k = 0; k < qn; k++) if (qid[k] == pid[i]) { v = qpr[k] / Q.total; break; }
      qat[i] = v;
    }
    __syncthreads();
    if (lane == 0) {
      double *res = ppr;  // each entry's residual replaces its probability once read
      double sum = 0;
      for (int i = 0; i < pn; i++) {
        const double v = ppr[i] / P.total - qat[i];
        res[i] = 0.0;
        if (v > 0) { res[i] = v; sum += v; }
      }
      if (!(sum > 0)) {
        tok = draw_dist(P, rng);
      } else {
        double r = rng_next(rng) * sum;
        int last = 0;
        tok = -1;
        for (int i = 0; i < pn; i++) {
          if (res[i] > 0) {
            last = i;
            r -= res[i];
            if (r <= 0) { tok = pid[i]; break; }
          }
        }
        if (tok < 0) tok = pid[last];
      }
    }
    break;
  }
  if (a == kk) {  // (a is the same in every lane) the bonus draw from the last row, as draw_dist takes it
    const DevDist &P = pdist[kk];
    const int pn = P.n;
    stage(P, pid, ppr);
    __syncthreads();
    if (lane == 0) {
      if (P.greedy) {
        tok = pid[0];
      } else {
        double r = rng_next(rng) * P.total;
        tok = pid[pn - 1];
        for (int i = 0; i < pn; i++) {
          r -= ppr[i];
          if (r <= 0) { tok = pid[i]; break; }
        }
      }
    }
  }
  if (lane != 0) return;
  ss->a = a;
  ss->tok = tok;
  ss->rng = rng;
}

__global__ void k_accept(const DevDist *pdist, const DevDist *qdist, SpecState *ss, int greedy) {
  if (blockIdx.x != 0) return;
  if (!greedy && !pdist[0].wids) { accept_lists(pdist, qdist, ss); return; }
  if (threadIdx.x != 0) return;
  uint32_t rng = ss->rng;
  const int kk = ss->kk;
  int a = 0, tok = -1;
  for (int j = 0; j < kk; j++) {
    const DevDist &P = pdist[j];
    const int x = ss->drafted[j];
    if (greedy) {
      int t = dist_id(P, 0);
      if (t == x) { a++; continue; }
      tok = t;
      break;
    }
    double px = prob_of(P, x), qx = prob_of(qdist[j], x);
    if (rng_next(rng) * qx < px) { a++; continue; }
    tok = draw_residual(P, qdist[j], rng);
    break;
  }
  if (a == kk) tok = draw_dist(pdist[kk], rng);
  ss->a = a;
  ss->tok = tok;
  ss->rng = rng;
}

__global__ void k_draw_one(const DevDist *dist, uint32_t *rng, int *out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  uint32_t s = *rng;
  *out = draw_dist(*dist, s);
  *rng = s;
}

// Greedy rows without penalties: first-maximum argmax of each row split over many blocks. Each block reduces its
// chunk to one key (order-preserving value bits, then the complement of the index, so the larger key is the larger
// value and, among equal values, the smaller index), stores it, and the last block of the row to arrive (counted with a
// device-scope atomic that it resets for the next launch) reduces the row's keys in one pass. NaN logits are never
// selected, as in the single-block path.
constexpr int AM_THREADS = 512;
constexpr int AM_CHUNK = AM_THREADS * 8;  // logits per block

__global__ __launch_bounds__(AM_THREADS) void k_argmax_rows(const float *__restrict__ logits, int ldl, int vocab,
                                                            unsigned long long *keys, uint32_t *count, DevDist *out) {
  __shared__ unsigned long long wk[AM_THREADS / 64];
  __shared__ uint32_t prev;
  const int r = blockIdx.y, nb = gridDim.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float *l = logits + (long)r * ldl;
  const int base = blockIdx.x * AM_CHUNK + tid * 8;
  float v[8];
  if (base + 8 <= vocab && ((((uintptr_t)(l + base)) & 15) == 0)) {
    const float4 a = *(const float4 *)(l + base), b = *(const float4 *)(l + base + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    #pragma unroll
    for (int k = 0; k < 8; k++) v[k] = base + k < vocab ? l[base + k] : -INFINITY;
  }
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  #pragma unroll
  for (int k = 0; k < 8; k++)
    if (v[k] > bv) { bv = v[k]; bi = base + k; }
  unsigned long long key = ((unsigned long long)fkey(bv) << 32) | (uint32_t)~(uint32_t)bi;
  key = group_reduce(key, 64, [](unsigned long long x, unsigned long long y) { return x > y ? x : y; });
  if (lane == 0) wk[wave] = key;
  __syncthreads();
  if (tid == 0) {
    unsigned long long k = wk[0];
    for (int w = 1; w < AM_THREADS / 64; w++) k = wk[w] > k ? wk[w] : k;
    keys[(long)r * nb + blockIdx.x] = k;
    __threadfence();
    prev = atomicAdd(&count[r], 1u);
  }
  __syncthreads();
  if (prev != (uint32_t)(nb - 1)) return;
  // last block of the row: every other block's key is visible after its fence and atomic
  __threadfence();
  if (tid < 64) {
    unsigned long long k = 0;
    for (int b = tid; b < nb; b += 64) {
      const unsigned long long kb = __atomic_load_n(&keys[(long)r * nb + b], __ATOMIC_RELAXED);
      k = kb > k ? kb : k;
    }
    k = group_reduce(k, 64, [](unsigned long long x, unsigned long long y) { return x > y ? x : y; });
    if (tid == 0) {
      int id = (int)~(uint32_t)(k & 0xffffffffu);
      if (id == 0x7fffffff || id < 0 || id >= vocab) id = 0;  // no finite maximum: the reference's argmax returns 0
      DevDist *D = out + r;
      D->n = 1; D->greedy = 1; D->total = 1.0; D->ids[0] = id; D->probs[0] = 1.0;
      count[r] = 0;
    }
  }
}

// ---- full candidate lists (topK 0 or at least the vocabulary: every id, sorted by logit descending, then id ascending,
// src/sampling/sampler.js:115-118; topK above KCAP: the K best, src/sampling/sampler.js:21-43). The order is an LSD radix
// sort of (~key of the penalised logit) with the ids as payload, four 8-bit passes, each stable, over ids taken in
// ascending order, so equal logits stay in id order. The softmax, min-p, top-p and total then follow the reference's
// order in one lane, as the fixed lists do.
constexpr int WT = 256;                          // threads of the sort kernels
constexpr int WPT = WIDE_CHUNK / WT;             // keys per thread and chunk

// the penalised logits of each row (scratch) and the first sort buffers: key ~fkey(logit), payload the id
__global__ __launch_bounds__(DT) void k_wide_prep(const float *__restrict__ logits, int ldl, int vocab, SamplerParams sp,
                                                  const int *hist, int histLen0, int histInc, float *scratch, WideWork ww) {
  const int r = blockIdx.x;
  const int hl = hist ? histLen0 + r * histInc : 0;
  float *cp = scratch + (long)r * vocab;
  penalized_copy(logits + (long)r * ldl, cp, vocab, sp, hist, hl, sp.penalized && hl > 0);
  for (int i = threadIdx.x; i < vocab; i += DT) {
    ww.keyA[(long)r * vocab + i] = ~fkey(cp[i]);
    ww.idA[(long)r * vocab + i] = i;
  }
}

// digit counts of one chunk: hist[row][digit][chunk]
__global__ __launch_bounds__(WT) void k_rs_hist(const uint32_t *__restrict__ keys, int vocab, int shift, uint32_t *hist) {
  __shared__ uint32_t h[256];
  const int ch = blockIdx.x, r = blockIdx.y, nch = gridDim.x, tid = threadIdx.x;
  h[tid] = 0;
  __syncthreads();
  const uint32_t *k = keys + (long)r * vocab;
  #pragma unroll
  for (int j = 0; j < WPT; j++) {
    const int i = ch * WIDE_CHUNK + j * WT + tid;
    if (i < vocab) atomicAdd(&h[(k[i] >> shift) & 255u], 1u);
  }
  __syncthreads();
  hist[((long)r * 256 + tid) * nch + ch] = h[tid];
}

// exclusive scan of a row's counts in (digit, chunk) order: the first output position of each (digit, chunk)
__global__ __launch_bounds__(DT) void k_rs_scan(uint32_t *hist, int nch) {
  __shared__ uint32_t ws[DT / 64];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t *h = hist + (long)r * 256 * nch;
  const int E = 256 * nch, per = (E + DT - 1) / DT, i0 = min(E, tid * per), i1 = min(E, i0 + per);
  uint32_t sum = 0;
  for (int i = i0; i < i1; i++) sum += h[i];
  uint32_t inc = sum;  // inclusive scan over the wave
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  if (lane == 63) ws[wave] = inc;
  __syncthreads();
  uint32_t before = inc - sum;
  for (int w = 0; w < wave; w++) before += ws[w];
  for (int i = i0; i < i1; i++) { const uint32_t c = h[i]; h[i] = before; before += c; }
}

// stable scatter of one chunk by the pass's digit: the chunk's keys in 256-key steps; within a step a key's place is
// the digit's running position, plus the same-digit keys of lower waves, plus those of lower lanes of its own wave
__global__ __launch_bounds__(WT) void k_rs_scatter(const uint32_t *__restrict__ kin, const int *__restrict__ iin,
                                                   uint32_t *kout, int *iout, int vocab, int shift,
                                                   const uint32_t *__restrict__ hist) {
  __shared__ uint32_t base[256];
  __shared__ uint32_t wcnt[WT / 64][256];
  const int ch = blockIdx.x, r = blockIdx.y, nch = gridDim.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long ro = (long)r * vocab;
  base[tid] = hist[((long)r * 256 + tid) * nch + ch];
  for (int j = 0; j < WPT; j++) {
    const int i = ch * WIDE_CHUNK + j * WT + tid;
    const bool valid = i < vocab;
    const uint32_t key = valid ? kin[ro + i] : 0u;
    const int id = valid ? iin[ro + i] : 0;
    const uint32_t d = (key >> shift) & 255u;
    #pragma unroll
    for (int w = 0; w < WT / 64; w++) wcnt[w][tid] = 0;
    __syncthreads();
    unsigned long long m = __ballot(valid);
    #pragma unroll
    for (int b = 0; b < 8; b++) {
      const unsigned long long bal = __ballot((d >> b) & 1u);
      m &= ((d >> b) & 1u) ? bal : ~bal;
    }
    const int rank = __popcll(m & ((1ull << lane) - 1ull));
    if (valid && rank == 0) wcnt[wave][d] = (uint32_t)__popcll(m);
    __syncthreads();
    if (valid) {
      uint32_t pos = base[d] + (uint32_t)rank;
      for (int w = 0; w < wave; w++) pos += wcnt[w][d];
      kout[ro + pos] = key;
      iout[ro + pos] = id;
    }
    __syncthreads();
    uint32_t add = 0;
    #pragma unroll
    for (int w = 0; w < WT / 64; w++) add += wcnt[w][tid];
    base[tid] += add;
    __syncthreads();
  }
}

// distribution of each row from its sorted ids (src/sampling/sampler.js:111-142)
__global__ __launch_bounds__(DT) void k_wide_dist(int vocab, SamplerParams sp, const float *__restrict__ scratch,
                                                  WideWork ww, DevDist *out) {
  __shared__ double s_sum;
  __shared__ int s_keep;
  const int r = blockIdx.x, tid = threadIdx.x;
  DevDist *D = out + r;
  int *wids = D->wids, *wpos = D->wpos;
  double *wprobs = D->wprobs;
  const float *cp = scratch + (long)r * vocab;
  const uint32_t *key = ww.keyA + (long)r * vocab;
  const int *sid = ww.idA + (long)r * vocab;
  const int K = sp.topK;
  const bool full = K <= 0 || K >= vocab;
  const int m = full ? vocab : K;
  if (!full && key[K - 1] == key[K]) {
    // a tie at the K-th value: which tied ids the reference's heap keeps depends on its history, so it is replayed
    // (wpos / wres as its ids / values), then its ids are listed in the sorted order
    if (tid == 0) heap_topk(cp, vocab, K, wpos, D->wres);
    __syncthreads();
    for (int i = tid; i < vocab; i += DT) wids[i] = 0;
    __syncthreads();
    for (int j = tid; j < K; j += DT) wids[wpos[j]] = 1;
    __syncthreads();
    if (tid == 0) {
      int c = 0;
      for (int i = 0; i < vocab && c < K; i++) if (wids[sid[i]]) wpos[c++] = sid[i];
    }
    __syncthreads();
    for (int i = tid; i < K; i += DT) wids[i] = wpos[i];
  } else {
    for (int i = tid; i < m; i += DT) wids[i] = sid[i];
  }
  __syncthreads();
  // softmax with temperature: exponentials in parallel, their sum in rank order
  const double mx = (double)cp[wids[0]];
  for (int i = tid; i < m; i += DT) wprobs[i] = exp(((double)cp[wids[i]] - mx) / sp.temperature);
  __syncthreads();
  if (tid == 0) {
    double sum = 0;
    for (int i = 0; i < m; i++) sum += wprobs[i];
    s_sum = sum;
    s_keep = m;
  }
  __syncthreads();
  const double sum = s_sum;
  for (int i = tid; i < m; i += DT) wprobs[i] = wprobs[i] / sum;
  __syncthreads();
  // min-p: the first rank from 1 on whose probability is below minP * probs[0]
  if (sp.minP > 0) {
    const double thr = sp.minP * wprobs[0];
    for (int i = 1 + tid; i < m; i += DT)
      if (wprobs[i] < thr) atomicMin(&s_keep, i);
    __syncthreads();
  }
  if (tid == 0) {
    int keep = s_keep;
    double total = 0;
    if (sp.topP < 1) {  // the running sum at the cut is the reference's total over the kept prefix
      int i = 0;
      while (i < keep) { total += wprobs[i]; i++; if (total >= sp.topP) break; }
      keep = i > 1 ? i : 1;
    } else {
      for (int i = 0; i < keep; i++) total += wprobs[i];
    }
    D->n = keep; D->greedy = 0; D->total = total;
    s_keep = keep;
  }
  for (int i = tid; i < vocab; i += DT) wpos[i] = 0;
  __syncthreads();
  const int keep = s_keep;
  for (int i = tid; i < keep; i += DT) wpos[wids[i]] = i + 1;
}

__global__ void k_set_wide(DevDist *d, int n, int vocab, int *ids, double *probs, int *pos, double *res) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  d[i].wids = ids ? ids + (long)i * vocab : nullptr;
  d[i].wprobs = probs ? probs + (long)i * vocab : nullptr;
  d[i].wpos = pos ? pos + (long)i * vocab : nullptr;
  d[i].wres = res ? res + (long)i * vocab : nullptr;
}

void launch_set_wide(DevDist *d, int n, int vocab, int *ids, double *probs, int *pos, double *res, hipStream_t st) {
  hipLaunchKernelGGL(k_set_wide, dim3((n + 63) / 64), dim3(64), 0, st, d, n, vocab, ids, probs, pos, res);
  ZL_HIP(hipGetLastError());
}

void launch_dist_rows(const float *logits, int ldl, int nrows, int vocab, const SamplerParams &sp, const int *hist,
                      int histLen0, int histInc, float *scratch, const ArgmaxWork &aw, const WideWork *ww,
                      const CandWork *cw, DevDist *out, hipStream_t st) {
  const bool greedy = sp.temperature <= 0.0 || sp.greedyArgmax;
  const int nb = (vocab + AM_CHUNK - 1) / AM_CHUNK;
  if (greedy && !(sp.penalized && hist && histLen0 + (nrows - 1) * histInc > 0) && nb <= ARGMAX_MAX_BLOCKS &&
      nrows <= ARGMAX_MAX_ROWS) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(nb, nrows), dim3(AM_THREADS), 0, st, logits, ldl, vocab, aw.keys, aw.count, out);
    ZL_HIP(hipGetLastError());
    return;
  }
  if (!greedy && ww) {
    ZL_REQUIRE(scratch && ww->vocab >= vocab && ww->rows >= nrows, ZL_ERR_STATE, "sampler work space too small");
    const int nch = (vocab + WIDE_CHUNK - 1) / WIDE_CHUNK;
    hipLaunchKernelGGL(k_wide_prep, dim3(nrows), dim3(DT), 0, st, logits, ldl, vocab, sp, hist, histLen0, histInc, scratch, *ww);
    for (int pass = 0; pass < 4; pass++) {
      const uint32_t *kin = pass & 1 ? ww->keyB : ww->keyA;
      const int *iin = pass & 1 ? ww->idB : ww->idA;
      uint32_t *kout = pass & 1 ? ww->keyA : ww->keyB;
      int *iout = pass & 1 ? ww->idA : ww->idB;
      hipLaunchKernelGGL(k_rs_hist, dim3(nch, nrows), dim3(WT), 0, st, kin, vocab, 8 * pass, ww->hist);
      hipLaunchKernelGGL(k_rs_scan, dim3(nrows), dim3(DT), 0, st, ww->hist, nch);
      hipLaunchKernelGGL(k_rs_scatter, dim3(nch, nrows), dim3(WT), 0, st, kin, iin, kout, iout, vocab, 8 * pass, ww->hist);
    }
    hipLaunchKernelGGL(k_wide_dist, dim3(nrows), dim3(DT), 0, st, vocab, sp, scratch, *ww, out);
    ZL_HIP(hipGetLastError());
    return;
  }
  // two stages (candidate lists of CAND_CHUNK-logit blocks, then the selection over them) where the work space fits;
  // one block per row over the whole row otherwise
  const int ncb = (vocab + CAND_CHUNK - 1) / CAND_CHUNK, cmax = std::min(sp.topK + CAND_SLACK, CAND_CMAX);
  const bool two = !greedy && cw && !sp.penalized && sp.topK >= 1 && sp.topK <= KCAP && ncb <= CAND_MAXB &&
                   cw->vocab >= vocab && cw->rows >= nrows;
  if (two) {
    hipLaunchKernelGGL(k_topk_cand, dim3(ncb, nrows), dim3(CT_T), 0, st, logits, ldl, vocab, sp.topK, cmax, *cw);
    ZL_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(k_dist_rows, dim3(nrows), dim3(DT), 0, st, logits, ldl, vocab, sp, hist, histLen0, histInc, scratch,
                     two ? *cw : CandWork{}, ncb, cmax, out);
  ZL_HIP(hipGetLastError());
}

void launch_draft_draw(const DevDist *dist, SpecState *ss, int j, const int *stopIds, int nStop, Step *draftStep,
                       int advance, Step *targetStep, int *hist, int histLen0, hipStream_t st) {
  hipLaunchKernelGGL(k_draft_draw, dim3(1), dim3(64), 0, st, dist, ss, j, stopIds, nStop, draftStep, advance, targetStep,
                     hist, histLen0);
  ZL_HIP(hipGetLastError());
}

void launch_accept(const DevDist *pdist, const DevDist *qdist, SpecState *ss, int greedy, hipStream_t st) {
  hipLaunchKernelGGL(k_accept, dim3(1), dim3(64), 0, st, pdist, qdist, ss, greedy);
  ZL_HIP(hipGetLastError());
}

void launch_draw_one(const DevDist *dist, uint32_t *rng, int *out, hipStream_t st) {
  hipLaunchKernelGGL(k_draw_one, dim3(1), dim3(64), 0, st, dist, rng, out);
  ZL_HIP(hipGetLastError());
}

}  // namespace zl
