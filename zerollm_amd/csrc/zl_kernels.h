// Kernel argument structures and launchers (zl_kernels.hip, zl_sample.hip).
#pragma once
#include "zl_common.h"
#include "synth.h"

namespace zl {

// Per-pass token/position block in device memory. Kernels read it at run time, so one captured graph serves every
// position, and device-side sampling can feed the next draft token without a host round trip.
struct Step {
  int pos0;        // position of tokens[0]
  int B;           // tokens in this pass
  int pad[2];
  int tokens[64];
};

// Plain view of a repacked matrix (kernel argument).
struct MatView {
  int type, rows, cols, nslab;
  const uint8_t *qs, *qx, *sc;
  const uint16_t *dd;
  const uint8_t *fq;
};
inline MatView view(const DevMat &m) { return MatView{m.type, m.rows, m.cols, m.nslab, m.qs, m.qx, m.sc, m.dd, m.fq}; }

// Quantised activations of several rows (tokens): int8 values, f32 block scales and int block sums (per 32 values),
// optionally the f32 values, and per 32-value block one 16-byte record per weight-format family, which the GEMV reads
// with scalar loads (the block scale as f64 plus the integer corrections the format's block term needs).
// ld = padded row length (multiple of 64); block b of row t is entry t * (ld / 32) + b.
struct RecA { double d, s; };                  // Q8_0, Q4_K, Q5_K: scale, block sum
struct RecB { double d; int32_t s16a, s16b; };  // Q6_K: scale, 32 x the sums of the block's two 16-value halves
struct RecC { double d; int32_t s8, s16; };     // Q4_0, Q5_0: scale, 8 x and 16 x the block sum
struct Act {
  int8_t *q;
  float *d;
  int32_t *s;
  RecA *ra;
  RecB *rb;
  RecC *rc;
  float *f;
  int ld;
};
// The same activation from row t0 on.
inline Act act_rows(const Act &a, int t0) {
  Act r = a;
  const long nb = (long)t0 * (a.ld >> 5);
  r.q = a.q ? a.q + (long)t0 * a.ld : nullptr;
  r.d = a.d ? a.d + nb : nullptr;
  r.s = a.s ? a.s + nb : nullptr;
  r.ra = a.ra ? a.ra + nb : nullptr;
  r.rb = a.rb ? a.rb + nb : nullptr;
  r.rc = a.rc ? a.rc + nb : nullptr;
  r.f = a.f ? a.f + (long)t0 * a.ld : nullptr;
  return r;
}

enum : int { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

struct GemvSeg {
  MatView m;        // tiled planes of the segment's matrix
  uint32_t nqs, nqx, nsc, ndd;  // plane sizes in bytes (buffer-resource bounds)
  int rows;
  int tile0;        // first tile of the segment in the launch's tile numbering
  float *out;
  int ldo;
  const float *bias;
};

// One GEMV launch over up to three matrices of one type laid end to end (q, k, v), or a gate/up pair (SWIGLU, seg[1]
// = up, same tiles). A workgroup handles one 64-row tile and one of `ks` equal ranges of its slabs; with ks > 1 the
// parts' f64 partial sums go to `part` and the last part to arrive (per-tile counters in `cnt`, left at zero) adds them
// in part order and runs the epilogue.
struct GemvArgs {
  // (the fields a kernel needs before its first loads lead, so that they share the first cache lines of the
  // argument block)
  int nseg;
  int ntiles;
  int nslab;
  int ks;
  int kr;           // slabs per K part: ceil(nslab / ks)
  int nwave;        // waves per workgroup
  int M;            // tokens (rows of the activation)
  // Fused activation prologue: when xf is set, the workgroup quantises rows xf[xrow0 + t] (length n, stride ldxf)
  // itself, after RMSNorm with weights nw when nw is set, exactly as k_norm_quant would, instead of reading `act`.
  int ldxf, xrow0, n;
  const float *xf;
  const float *nw;
  double eps;
  GemvSeg seg[3];
  Act act;          // quantised activations read by the kernel
  float *resid;     // EPI_RESID: resid[t * ldr + row] += y
  int ldr;
  float *hb;        // EPI_SWIGLU: hb[t * ldh + row] = silu(gate) * up
  int ldh;
  Act qout;         // EPI_SWIGLU: also quantise hb into qout (when qout.q is set)
  double *part;
  uint32_t *cnt;
};

// Split-K work space of GEMV launches (partial sums and per-tile arrival counters, counters zero between launches).
constexpr int GEMV_MAX_MT = 9;              // tokens per launch
constexpr int GEMV_CNT_TILES = 4096;        // counters available (tiles of launches with ks > 1)
constexpr long GEMV_PART_DOUBLES = 8192L * 2 * GEMV_MAX_MT * 64;  // tiles x K parts <= 8192
struct GemvWork {
  double *part;
  uint32_t *cnt;
};

struct AttnArgs {
  const float *q;
  int ldq;
  const float *k, *v;        // the pass's key / value projections [B][ldkv] (normed, rotated and cached here)
  int ldkv;
  const float *qNorm, *kNorm;
  double eps;
  const float *cosT, *sinT;
  int nRot, neox;
  const void *kcache, *vcache;
  int nHead, nHeadKv, hd, ctx, layer, kvF16;
  int vstride;     // positions per V cache row (V is dimension-major)
  int hpb;         // query heads per score block (set by launch_attention)
  float *scores;   // [token][head][sld] f32 scores
  int sld;
  double scale;
  const Step *step;
  float *out;
  int ldo;
  Act act;
  int qhs;              // floats from one query head to the next in q (hd; 2 hd where q rows are [query | gate])
  const float *gate;    // output gate (q + hd for [query | gate] rows, same strides), or null
  // position-split weighted sum (long contexts): per (token, head, chunk of ATTN_SPLIT_C positions) the chunk's
  // max score, f64 sum of exponentials and f64 weighted sum of V, [B][nHead][nch][hd + 2] doubles; null: the exact
  // position-order f32 chain
  double *part;
  int nch;              // chunks per (token, head) row of part
  double *pinv;         // [token][head] 1 / sum of a row's exponentials (grouped weighted sum of long multi-token passes)
  // contexts above headCtx take the per-head / grouped weighted sum for passes of several tokens, contexts above
  // head1Ctx also for single-token passes (decided once per model when it is loaded: attention_form)
  int headCtx, head1Ctx;
  // passes of at least mmMinB tokens take the matrix-core score dots (k_attn_prep + k_attn_scores_mm), which need qr,
  // the pass's normed and rotated query rows [B][nHead][hd] f32
  int mmMinB, mmAvMinB;  // ... and at least mmAvMinB tokens the matrix-core weighted sums (k_attn_av_mm)
  float *qr;
  int avmf;  // the slice form's chains on the matrix cores (k_attn_av_mfma) instead of the lanes (k_attn_av)
};
constexpr int ATTN_SPLIT_C = 256;  // positions per chunk of the position-split weighted sum

// One Gated DeltaNet layer over the B tokens of a pass (src/model/forward-qwen35.js:45-61). Conv window and delta-rule
// matrices of the layer are read, advanced token by token and written back. The conv window is kept per value head:
// [nV][3][D][K-1] with slots q and k of the head's key head and v of the head itself, so that no workgroup reads what
// another one writes (value heads sharing a key head hold identical copies of its q/k window).
struct DeltaArgs {
  const float *qkv;    // conv input: attn_qkv rows [B][ldqkv] as [q: nK x D | k: nK x D | v: nV x D]
  int ldqkv;
  const float *z;      // attn_gate rows [B][ldz]
  int ldz;
  const float *alpha, *beta;  // ssm_alpha / ssm_beta rows [B][ldab]
  int ldab;
  const float *convW;  // ssm_conv1d [convDim][K]
  float *conv;         // this layer's conv windows [nV][3][D][K-1]
  float *ssm;          // this layer's delta-rule matrices [nV][D (value dim)][D (key dim)]
  const float *dtBias, *ssmA, *normW;
  int nK, nV, K, B;
  double eps;
  Act act;             // the quantised core rows (input of ssm_out), columns hv * D + j
  float *out;          // and the f32 core rows (act.f), or null
  int ldo;
  // per-position capture (verify passes): the layer's conv windows and delta-rule matrices after token b go to
  // capConv / capSsm + b * capStride (floats; the same layout as conv / ssm), when set
  float *capConv, *capSsm;
  long capStride;
  // the heads' output rows ([nV][DELTA_MAX_B][D] floats): written by k_deltanet, normed by k_delta_norm
  float *xcore;
};
constexpr int DELTA_MAX_B = 16;  // tokens per k_deltanet launch (longer passes run as several launches in order)
void launch_deltanet(const DeltaArgs &a, int D, hipStream_t st);

// Launch shape of a GEMV over ntiles tiles of nslab slabs: K parts per tile and waves per workgroup.
void gemv_shape(int ntiles, int nslab, bool swiglu, int *ks, int *nw);
// Launch a GEMV of a.M tokens (chunks of at most GEMV_MAX_MT); float weights read the f32 activation xf (stride ldx).
void launch_gemv(const GemvArgs &a, int epi, const float *xf, int ldx, hipStream_t st);
bool gemv_mfma_ok(const GemvArgs &a);
void launch_gemv_mfma(const GemvArgs &a, int epi, hipStream_t st);
// Two store launches of the same tokens in one kernel (a1 Q4_K on the matrix cores, a2 Q6_K or Q8_0 on the VALU tiles);
// their split-K work spaces must be disjoint.
bool gemv_mix_ok(const GemvArgs &a1, const GemvArgs &a2);
void launch_gemv_mix(const GemvArgs &a1, const GemvArgs &a2, hipStream_t st);
// Single-token Q8_0 GEMV in 16-row groups (zl_gemv_rg.hip): takes f32 input rows (a.xf, RMSNorm'd with a.nw when set)
// and quantises them itself; K <= 3072.
bool gemv_rg_ok(const GemvArgs &a);
void launch_gemv_rg(const GemvArgs &a, int epi, hipStream_t st);
template <int FMT>
void launch_gemv_fmt(const GemvArgs &a, int epi, hipStream_t st);
constexpr int GEMM_MIN_M = 10;  // launches of at least this many tokens take the GEMM (zl_gemm.h)
// GEMM of 10..64 tokens (zl_gemm.h): Q8_0, Q4_K, Q5_K and Q6_K, every weight read once for all the launch's tokens,
// the same bits per token as the GEMV kernels.
template <int FMT>
void launch_gemm_fmt(const GemvArgs &a, int epi, hipStream_t st);
// Whether launch_gemv runs a launch of a.M tokens on the GEMM, and the split-K partial sums (doubles) a launch needs.
bool gemm_takes(const GemvArgs &a);
long gemv_part_need(const GemvArgs &a);
// Token groups of a GEMM launch of a.M <= 64 tokens: G workgroups along the tokens per (K part, tile), 16 U tokens
// each, each group re-reading the matrix. Up to 4 groups while the launch stays within 512 workgroups: at 64 tokens
// the 8B-shaped target's attn_v takes 4 (64 workgroups otherwise), q/k, gate/up, attn_output and ffn_down 2, the
// 0.6B-shaped draft's projections 4 (16-64 workgroups otherwise); measured on 16K-token prefills, target + draft:
// 3.91 + 1.88 s in one group, 3.63 + 1.63 s within 320 workgroups, 3.23 + 1.55 s within 512, 3.31 + 1.59 s within
// 1024. No group is empty: G <= ceil(M / 16).
inline void gemm_groups(const GemvArgs &a, int &U, int &G) {
  const int n16 = (a.M + 15) / 16, blocks = a.ks * a.ntiles;
  G = 1;
  while (G < 4 && 2 * G <= n16 && 2 * G * blocks <= 512) G *= 2;
  U = (n16 + G - 1) / G;
}

// quantizeAct of one 32-value block (src/compute/ref-kernels.js:44-62) held by 32 consecutive lanes: d = amax/127 (f64,
// stored f32), q = round-half-away(v * (1/d)). Every lane gets its q; the block's first lane (i & 31 == 0) also gets
// the f32 scale, the block sum and the sums of the two 16-value halves.
struct QBlock {
  int q;
  float d;
  int s32, s16a, s16b;
};
__device__ inline QBlock quant32(float v) {
  QBlock r;
  const float am = group_fmax(fabsf(v), 32);
  const double scale = (double)am / 127.0;
  const double inv = scale != 0.0 ? 1.0 / scale : 0.0;
  r.q = (int)round((double)v * inv);
  r.d = (float)scale;
  r.s16a = wave_sum_xor(r.q, 16);          // each 16-lane half holds its sum
  r.s16b = __shfl_down(r.s16a, 16, 32);    // the second half's sum, at the block's first lane
  r.s32 = r.s16a + swizzle_xor16(r.s16a);
  return r;
}

// The records of one block (at its first lane).
template <int FMT>
__device__ inline uint4 block_record(const QBlock &b) {
  const double d = (double)b.d;
  const unsigned long long dl = __builtin_bit_cast(unsigned long long, d);
  if (FMT == T_Q6_K) return make_uint4((uint32_t)dl, (uint32_t)(dl >> 32), (uint32_t)(32 * b.s16a), (uint32_t)(32 * b.s16b));
  if (FMT == T_Q4_0 || FMT == T_Q5_0) return make_uint4((uint32_t)dl, (uint32_t)(dl >> 32), (uint32_t)(8 * b.s32), (uint32_t)(16 * b.s32));
  const unsigned long long sl = __builtin_bit_cast(unsigned long long, (double)b.s32);
  return make_uint4((uint32_t)dl, (uint32_t)(dl >> 32), (uint32_t)sl, (uint32_t)(sl >> 32));
}

// Quantise value v (element i of activation row `row`, 32 consecutive lanes per block) into Act a.
__device__ inline void quant_block32(float v, int i, const Act &a, int row) {
  const QBlock b = quant32(v);
  a.q[(long)row * a.ld + i] = (int8_t)b.q;
  if ((i & 31) == 0) {
    const long k = (long)row * (a.ld >> 5) + (i >> 5);
    const double d = (double)b.d;
    a.d[k] = b.d;
    a.s[k] = b.s32;
    a.ra[k] = RecA{d, (double)b.s32};
    a.rb[k] = RecB{d, 32 * b.s16a, 32 * b.s16b};
    a.rc[k] = RecC{d, 8 * b.s32, 16 * b.s32};
  }
}

// RMSNorm scale of one row (src/compute/ref-kernels.js:305-310): 1/sqrt(mean(x^2) + eps), the sum of squares taken by
// 256 threads (tid < 256: strided sequential f64 sums, a 64-lane butterfly, then (w0 + w1) + (w2 + w3) through red[4]).
// Every caller uses this order, so every kernel derives the same scale. All 256 threads return it; the caller
// synchronises the block between the two uses of red.
// Sum of squares of this thread's values xr[base + tid + 256 k], k < K, added to ss in k order; the K loads are issued
// together (unconditionally: a position past n reads xr[0] and adds +0.0, which leaves the f64 sum unchanged).
template <int K>
__device__ inline double sumsq_batch(const float *xr, int base, int n, int tid, double ss) {
  float v[K];
  #pragma unroll
  for (int k = 0; k < K; k++) { const int i = base + tid + 256 * k; v[k] = xr[i < n ? i : 0]; }
  #pragma unroll
  for (int k = 0; k < K; k++) { const double x = base + tid + 256 * k < n ? (double)v[k] : 0.0; ss += x * x; }
  return ss;
}

// The RMSNorm scale from each thread's partial sum of squares: the 64-lane butterfly, then the four waves of the
// 256-thread group (red: 4 doubles of the group; synchronises the block).
__device__ inline double rms_finish(double ss, int n, double eps, int tid, double *red) {
  ss = wave_sum_xor(ss, 64);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  return 1.0 / sqrt(ss / (double)n + eps);
}

__device__ inline double rms_scale256(const float *xr, int n, double eps, int tid, double *red) {
  // thread tid adds x[tid]^2, x[tid + 256]^2, ... in that order (f64), then the 64-lane butterfly and the four waves
  double ss = 0;
  if (n <= 1024) ss = sumsq_batch<4>(xr, 0, n, tid, ss);
  else
    for (int base = 0; base < n; base += 4096) ss = sumsq_batch<16>(xr, base, n, tid, ss);
  return rms_finish(ss, n, eps, tid, red);
}

void launch_attention(const AttnArgs &a, int B, hipStream_t st);
size_t attention_lds(int ctx);
size_t attention_split_lds(int hd, int kvF16);
// The attention form of a model, decided once at load from its context and head size (the environment overrides
// ZEROLLM_ATTN_HEAD_CTX and ZEROLLM_ATTN_HEAD1_CTX move the thresholds, for tests): headCtx / head1Ctx as in AttnArgs
// (INT_MAX: never), split = whether the model needs the position-split weighted sum (its exact chain would not fit).
struct AttnForm { int headCtx, head1Ctx, mmMinB, mmAvMinB; bool split, avmf; };
AttnForm attention_form(int ctx, int hd);
void launch_norm_quant(const float *x, int ldx, int row0, int nrows, const float *w, double eps, int n, int npad,
                       const Act &act, hipStream_t st);
void launch_embed(const MatView &m, const Step *step, int B, float *x, int ldx, hipStream_t st);
void launch_dequant_rows(const MatView &m, const int *rowIds, int nrows, float *out, int ldo, hipStream_t st);
void launch_repack(int type, const uint8_t *raw, long rawRowBytes, int rows, int cols, int nslab, DevMat &m, hipStream_t st);
void launch_frag(const DevMat &m, hipStream_t st);
void launch_synth(int type, uint64_t seed, double std, uint64_t srcCols, uint64_t col0, int rows, int cols, uint8_t *out,
                  hipStream_t st);
void launch_fill(float *p, long n, float v, hipStream_t st);

// ------------------------------------------------------------------------------------------------ sampling
constexpr int KCAP = 256;  // largest top-k (candidate list) the device sampler supports

// Sparse distribution (zerollm's TokenDist, src/sampling/sampler.js:52-62): ids[i] has probability probs[i] / total.
// A sampler with top_k 0 or above KCAP (the reference's full candidate list) keeps up to a vocabulary of entries in
// storage of its own: wids / wprobs in rank order, wpos[id] = rank + 1 of a kept id (0 otherwise), and wres for the
// residual draw; these pointers are null for the fixed lists.
struct DevDist {
  int n;
  int greedy;
  double total;
  int ids[KCAP];
  double probs[KCAP];
  int *wids;
  double *wprobs;
  int *wpos;
  double *wres;
};

// Work space of full-list distributions: the rows' sort keys and ids (two buffers each, [rows][vocab]) and per-chunk
// digit counts ([rows][256][chunks]).
constexpr int WIDE_CHUNK = 4096;  // keys per sort workgroup
struct WideWork {
  uint32_t *keyA, *keyB;
  int *idA, *idB;
  uint32_t *hist;
  int vocab, rows;
};

// Work space of two-stage top-k selection (top_k <= KCAP, no penalties): blocks of CAND_CHUNK logits each keep every
// logit at or above their own k-th largest ([rows][blocks][cmax] ids and values, [rows][blocks] counts); the row's
// selection then runs over those candidates only.
constexpr int CAND_CHUNK = 2048;              // logits per candidate block
constexpr int CAND_MAXB = 128;                // candidate blocks per row at most (vocabularies up to 262144)
constexpr int CAND_SLACK = 32;                // list room above top_k for ties at a block's k-th value
constexpr int CAND_CMAX = KCAP + CAND_SLACK;  // list length the work space is sized for
struct CandWork {
  int *ids;
  float *vals;
  int *cnt;
  int vocab, rows;
};

struct SamplerParams {
  double temperature, topP, minP, repeatPenalty, presence, frequency;
  int topK, repeatLastN, penalized, greedyArgmax;
};

// Per-cycle speculative state on the device.
struct SpecState {
  uint32_t rng;       // mulberry32 state (shared by draft draws and acceptance, one stream as in the reference)
  int kk;             // tokens drafted so far / finally
  int stopped;        // a stop token was drafted
  int a;              // accepted count
  int tok;            // correction / bonus token
  int pad[3];
  int drafted[64];
};

// Work space of the multi-block greedy argmax: per-row block keys and arrival counters (zero between launches).
constexpr int ARGMAX_MAX_BLOCKS = 128, ARGMAX_MAX_ROWS = 65;
struct ArgmaxWork {
  unsigned long long *keys;  // [ARGMAX_MAX_ROWS][blocks]
  uint32_t *count;           // [ARGMAX_MAX_ROWS], zero-initialised
};

// Row r uses history hist[0 .. histLen0 + r * histInc).
// ww: the full-list work space when the sampler keeps full lists (top_k 0 or above KCAP), else null; cw: the two-stage
// selection's work space (unpenalized samplers with top_k <= KCAP), else null.
void launch_dist_rows(const float *logits, int ldl, int nrows, int vocab, const SamplerParams &sp, const int *hist,
                      int histLen0, int histInc, float *scratch, const ArgmaxWork &aw, const WideWork *ww,
                      const CandWork *cw, DevDist *out, hipStream_t st);
// Point rows [0, n) of d at full-list storage of `vocab` entries per row (ids, probs, pos, res), or at null.
void launch_set_wide(DevDist *d, int n, int vocab, int *ids, double *probs, int *pos, double *res, hipStream_t st);
void launch_draft_draw(const DevDist *dist, SpecState *ss, int j, const int *stopIds, int nStop, Step *draftStep,
                       int advance, Step *targetStep, int *hist, int histLen0, hipStream_t st);
void launch_accept(const DevDist *pdist, const DevDist *qdist, SpecState *ss, int greedy, hipStream_t st);
void launch_draw_one(const DevDist *dist, uint32_t *rng, int *out, hipStream_t st);

}  // namespace zl
