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
};
inline MatView view(const DevMat &m) { return MatView{m.type, m.rows, m.cols, m.nslab, m.qs, m.qx, m.sc, m.dd}; }

// Quantised activations of several rows (tokens): int8 values, f32 block scales, int block sums (per 32 and per 16),
// optionally the f32 values. ld = padded row length (multiple of 64).
struct Act {
  int8_t *q;
  float *d;
  int32_t *s;
  int32_t *s16;
  float *f;
  int ld;
};

enum : int { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

struct GemvSeg {
  MatView m;
  int rows;
  float *out;
  int ldo;
  const float *bias;
};

struct GemvArgs {
  GemvSeg seg[3];
  int nseg;
  int rows_total;  // SWIGLU: rows of gate (== rows of up)
  int nslab;
  Act act;
  int M;
  int lpr;
  int wk;
  float *resid;
  int ldr;
  float *hb;
  int ldh;
  // Fused activation prologue: when xf is set, each block quantises rows xf[xrow0 + t] (length n, stride ldxf) itself,
  // after RMSNorm with weights nw when nw is set, exactly as k_norm_quant would, instead of reading `act`.
  const float *xf;
  int ldxf, xrow0, n;
  const float *nw;
  double eps;
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
};

int gemv_lpr(int rows, int nslab);
size_t gemv_lds_bytes(int fmt, int mt, int K);
void launch_gemv(const GemvArgs &a, int epi, const float *xf, int ldx, hipStream_t st);
void launch_attention(const AttnArgs &a, int B, hipStream_t st);
size_t attention_lds(int ctx);
void launch_norm_quant(const float *x, int ldx, int row0, int nrows, const float *w, double eps, int n, int npad,
                       const Act &act, hipStream_t st);
void launch_embed(const MatView &m, const Step *step, int B, float *x, int ldx, hipStream_t st);
void launch_dequant_rows(const MatView &m, const int *rowIds, int nrows, float *out, int ldo, hipStream_t st);
void launch_repack(int type, const uint8_t *raw, long rawRowBytes, int rows, int cols, int nslab, DevMat &m, hipStream_t st);
void launch_synth(int type, uint64_t seed, double std, uint64_t srcCols, uint64_t col0, int rows, int cols, uint8_t *out,
                  hipStream_t st);
void launch_fill(float *p, long n, float v, hipStream_t st);

// ------------------------------------------------------------------------------------------------ sampling
constexpr int KCAP = 256;  // largest top-k (candidate list) the device sampler supports

// Sparse distribution (zerollm's TokenDist, src/sampling/sampler.js:52-62): ids[i] has probability probs[i] / total.
struct DevDist {
  int n;
  int greedy;
  double total;
  int ids[KCAP];
  double probs[KCAP];
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
void launch_dist_rows(const float *logits, int ldl, int nrows, int vocab, const SamplerParams &sp, const int *hist,
                      int histLen0, int histInc, float *scratch, const ArgmaxWork &aw, DevDist *out, hipStream_t st);
void launch_draft_draw(const DevDist *dist, SpecState *ss, int j, const int *stopIds, int nStop, Step *draftStep,
                       int advance, Step *targetStep, int *hist, int histLen0, hipStream_t st);
void launch_accept(const DevDist *pdist, const DevDist *qdist, SpecState *ss, int greedy, hipStream_t st);
void launch_draw_one(const DevDist *dist, uint32_t *rng, int *out, hipStream_t st);

}  // namespace zl
