// Runtime of the zerollm MI355X library: model construction (GGUF or synthetic) with weight repacking, the forward
// pass as one captured HIP graph per (batch, logits mode), the on-device speculative cycle, and the C ABI
// (include/zerollm_hip.h).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <functional>
#include <atomic>
#include <map>
#include <set>
#include <tuple>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "zerollm_hip.h"
#include "gguf.h"
#include "zl_kernels.h"

namespace zl {

static thread_local std::string g_err;
static int g_device = -1;

static void ensure_init() {
  if (g_device < 0) {
    int n = 0;
    ZL_HIP(hipGetDeviceCount(&n));
    ZL_REQUIRE(n > 0, ZL_ERR_HIP, "no GPU visible");
    ZL_HIP(hipSetDevice(0));
    g_device = 0;
  }
}

static int pad64(int n) { return (n + 63) / 64 * 64; }

// ---------------------------------------------------------------------------------------------- allocations
// Zero device memory before any stream uses it: hipMemset runs on the null stream, which does not order with the
// library's non-blocking streams, so it is waited for here.
static void zero_now(void *p, size_t n) {
  ZL_HIP(hipMemset(p, 0, n));
  ZL_HIP(hipDeviceSynchronize());
}

struct Arena {
  std::vector<void *> ptrs;
  int64_t bytes = 0;
  void *alloc(size_t n) {
    void *p = nullptr;
    if (n == 0) n = 16;
    ZL_HIP(hipMalloc(&p, n));
    ptrs.push_back(p);
    bytes += (int64_t)n;
    return p;
  }
  void release() {
    for (void *p : ptrs) hipFree(p);
    ptrs.clear();
    bytes = 0;
  }
};

// Planes of a rows x cols matrix of `type` (not yet filled): rows are padded to whole 64-row tiles, which stay zero.
static DevMat alloc_planes(Arena &ar, int type, int rows, int cols) {
  DevMat m;
  m.type = type; m.rows = rows; m.cols = cols;
  m.nslab = (cols + 63) / 64;
  int64_t rb = ggml_row_bytes(type, cols);
  ZL_REQUIRE(rb > 0, ZL_ERR_UNSUPPORTED, "unsupported tensor type " + std::to_string(type) + " for " + std::to_string(cols) + " columns");
  if (!is_quant(type)) {
    ZL_REQUIRE(type == T_F32 || type == T_F16 || type == T_BF16, ZL_ERR_UNSUPPORTED,
               "reference kernels: unsupported tensor type " + std::to_string(type) + " (supported: F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)");
    m.qs = (uint8_t *)ar.alloc((size_t)rb * rows);
    return m;
  }
  const long T = tiles_of(rows), ns = T * 64 * m.nslab;
  ZL_REQUIRE(ns * qs_bytes(type) < (1L << 32), ZL_ERR_UNSUPPORTED, "matrix too large");
  auto zalloc = [&](size_t n) { void *p = ar.alloc(n); zero_now(p, n); return p; };
  m.qs = (uint8_t *)zalloc(ns * qs_bytes(type));
  if (qx_bytes(type)) m.qx = (uint8_t *)zalloc(ns * qx_bytes(type));
  if (sc_bytes(type)) m.sc = (uint8_t *)zalloc(ns * sc_bytes(type));
  m.dd = (uint16_t *)zalloc(T * dd_per_tile(type, m.nslab) * 2);
  if (type == T_Q4_K) m.fq = (uint8_t *)zalloc(ns * qs_bytes(type));
  return m;
}

// Rows [row0, row0 + n) of m as a matrix of its own (row0 a multiple of 64): an offset into each plane.
static DevMat row_view(const DevMat &m, int row0, int n) {
  DevMat v = m;
  v.rows = n;
  if (!is_quant(m.type)) {
    v.qs = m.qs + (size_t)ggml_row_bytes(m.type, m.cols) * row0;
    return v;
  }
  ZL_REQUIRE(row0 % 64 == 0, ZL_ERR_ARG, "row view must start at a 64-row tile");
  const long ns = (long)row0 * m.nslab;
  v.qs = m.qs + ns * qs_bytes(m.type);
  if (m.qx) v.qx = m.qx + ns * qx_bytes(m.type);
  if (m.sc) v.sc = m.sc + ns * sc_bytes(m.type);
  v.dd = m.dd + (long)(row0 / 64) * dd_per_tile(m.type, m.nslab);
  if (m.fq) v.fq = m.fq + ns * qs_bytes(m.type);
  return v;
}

// Fill the planes of m (or of a row view of a larger matrix) from raw ggml rows (device pointer).
static void fill_planes(const DevMat &m, const uint8_t *draw, hipStream_t st) {
  const int64_t rb = ggml_row_bytes(m.type, m.cols);
  if (!is_quant(m.type)) {
    ZL_HIP(hipMemcpyAsync(m.qs, draw, (size_t)rb * m.rows, hipMemcpyDeviceToDevice, st));
    return;
  }
  DevMat mm = m;
  launch_repack(m.type, draw, rb, m.rows, m.cols, m.nslab, mm, st);
  if (m.fq) launch_frag(m, st);
}

// Allocate the planes of a rows x cols matrix of `type` and repack raw ggml rows (device pointer) into them.
static DevMat make_mat(Arena &ar, int type, int rows, int cols, const uint8_t *draw, hipStream_t st) {
  DevMat m = alloc_planes(ar, type, rows, cols);
  fill_planes(m, draw, st);
  return m;
}

// Matrices that one GEMV launch reads together (q, k, v): consecutive ones of the same type share one allocation
// (each padded to whole tiles). stage(i) puts tensor i's raw rows at `draw` and returns its type.
static std::vector<DevMat> make_group(Arena &ar, const std::vector<int> &types, const std::vector<int> &rows, int cols,
                                      const std::function<void(size_t)> &stage, const uint8_t *draw, hipStream_t st) {
  std::vector<DevMat> out(rows.size());
  size_t i = 0;
  while (i < rows.size()) {
    size_t j = i + 1;
    int total = tiles_of(rows[i]) * 64;
    while (j < rows.size() && types[j] == types[i] && is_quant(types[i])) total += tiles_of(rows[j++]) * 64;
    DevMat all = alloc_planes(ar, types[i], total, cols);
    int r0 = 0;
    for (size_t k = i; k < j; k++) {
      stage(k);
      out[k] = row_view(all, r0, rows[k]);
      fill_planes(out[k], draw, st);
      ZL_HIP(hipStreamSynchronize(st));
      r0 += tiles_of(rows[k]) * 64;
    }
    i = j;
  }
  return out;
}

// ---------------------------------------------------------------------------------------------- model
struct Layer {
  DevMat wq, wk, wv, wo, wgate, wup, wdown;
  float *attnNorm = nullptr, *ffnNorm = nullptr, *qNorm = nullptr, *kNorm = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
  // qwen35: a Gated DeltaNet layer (rec) or a gated attention layer; ai / ri index the KV cache / the recurrent state
  bool rec = false;
  int ai = -1, ri = -1;
  DevMat wqkv, wz, walpha, wbeta, wssmout;
  float *conv = nullptr, *dtBias = nullptr, *ssmA = nullptr, *ssmNorm = nullptr;
};

// Recurrent-state snapshots of a hybrid model in HBM (StateCheckpoints, src/model/state-checkpoints.js:18-85): at most
// `max` positional checkpoints (smallest position evicted) plus one rollback slot; buffers are reused.
struct Snap {
  int pos = -1;
  float *buf = nullptr;
};
struct Checkpoints {
  int max = 6, every = 0;
  std::set<int> boundary;
  std::vector<Snap> list;  // ascending pos
  Snap rollback;           // pos -1: empty
  std::vector<float *> spare;
  // wantsBefore (src/model/state-checkpoints.js:37-39)
  bool wants_before(int pos, int token, bool wantLogits, bool prevNoLogits) const {
    return pos > 0 && ((wantLogits && prevNoLogits) || boundary.count(token) || (every > 0 && pos % every == 0));
  }
  bool has(int pos) const {
    for (auto &c : list) if (c.pos == pos) return true;
    return false;
  }
  // plan (:61-67): the snapshot restored (0 = zeros) and the tokens replayed when n < pos
  void plan(int n, int pos, int *from, int *replay) const {
    if (n >= pos) { *from = pos; *replay = 0; return; }
    int f = 0;
    for (auto &c : list) if (c.pos <= n && c.pos > f) f = c.pos;
    if (rollback.pos >= 0 && rollback.pos <= n && rollback.pos > f) f = rollback.pos;
    *from = f;
    *replay = n - f;
  }
  // dropAfter (:70-73)
  void drop_after(int n) {
    std::vector<Snap> keep;
    for (auto &c : list) {
      if (c.pos <= n) keep.push_back(c);
      else spare.push_back(c.buf);
    }
    list = keep;
    if (rollback.pos > n) rollback.pos = -1;
  }
  void clear() {
    for (auto &c : list) spare.push_back(c.buf);
    list.clear();
    rollback.pos = -1;
  }
  const Snap *find(int pos) const {
    for (auto &c : list) if (c.pos == pos) return &c;
    return rollback.pos == pos ? &rollback : nullptr;
  }
};

}  // namespace zl

struct zl_model {
  uint64_t uid = 0;  // never reused: keys the speculative-cycle graphs that capture this model's passes
  zl_config cfg{};
  int ctx = 0, kvF16 = 0, maxBatch = 16, logitsBatch = 16;
  int vstride = 0;  // positions per V cache row
  bool closed = false;
  zl::Arena ar;
  int64_t weightBytes = 0;
  zl::DevMat tokEmbd, output;
  float *outputNorm = nullptr;
  std::vector<zl::Layer> layers;
  float *cosT = nullptr, *sinT = nullptr;
  void *kcache = nullptr, *vcache = nullptr;
  float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *hb = nullptr, *logits = nullptr;
  float *scores = nullptr;  // attention scores [maxBatch][n_head][ctx]
  double *attnPart = nullptr;  // position-split weighted-sum partials (contexts beyond ZEROLLM_ATTN_EXACT_CTX), or null
  double *attnInv = nullptr;   // [maxBatch][n_head] 1 / sum of exponentials (grouped weighted sum)
  int attnNch = 0;
  int attnHeadCtx = 0, attnHead1Ctx = 0, attnMmMinB = 0, attnMmAvMinB = 0;  // attention form thresholds, at load
  bool attnAvmf = false;
  float *qr = nullptr;  // the pass's normed and rotated query rows [maxBatch][n_head][head_dim] (matrix-core scores)
  zl::Act act{};    // quantised input of the q/k/v, attention-output and gate/up GEMVs
  zl::Act act2{};   // quantised FFN hidden state (written by the gate/up GEMV, read by the down GEMV)
  zl::GemvWork gw{};
  // hybrid (qwen35) models: the live recurrent state, one block [conv windows of every recurrent layer | delta-rule
  // matrices of every recurrent layer] (convFloats / ssmFloats per layer), its snapshots, the DeltaNet inputs
  bool hybrid = false;
  int nAttn = 0, nRec = 0;
  long convFloats = 0, ssmFloats = 0;
  float *state = nullptr;
  // per-position capture of the recurrent state in passes that return every row's logits (verify passes): slot b
  // holds the state after the pass's token b (capPos0 + b + 1 tokens processed); capN valid slots (0: none)
  float *capture = nullptr;
  int capSlots = 0, capPos0 = 0, capN = 0;
  zl::Checkpoints ck;
  bool prevNoLogits = false;
  float *dqkv = nullptr, *dz = nullptr, *dalpha = nullptr, *dbeta = nullptr;
  float *dxcore = nullptr;      // DeltaNet: the heads' output rows, between the recurrence and the gated norm
  zl::Step *dstep = nullptr;
  hipStream_t st = nullptr;
  hipStream_t cst = nullptr;  // graphs are captured on their own stream
  std::vector<int> tokens;
  std::map<int, hipGraphExec_t> graphs;
  std::map<int, hipGraph_t> graphDefs;
  ~zl_model();
};

struct zl_sampler {
  zl::SamplerParams sp{};
  zl::Arena ar;
  zl::SpecState *ss = nullptr;      // device
  zl::SpecState *hss = nullptr;     // pinned host mirror
  zl::DevDist *pdist = nullptr, *qdist = nullptr, *tmpdist = nullptr;
  zl::DevDist *hdist = nullptr;     // pinned
  int *dhist = nullptr;             // device history (tail + drafted)
  int *dstop = nullptr;
  int *dtok = nullptr, *htok = nullptr;
  float *scratch = nullptr;
  int scratchVocab = 0;
  zl::ArgmaxWork am{};
  bool wide = false;      // full candidate lists (top_k 0 or above KCAP)
  zl::WideWork ww{};      // their sort work space ([65 rows][vocab])
  zl::CandWork cw{};      // two-stage top-k selection work space (unpenalized samplers with top_k <= KCAP)
  hipStream_t st = nullptr;
  // whole speculative cycles captured as two graphs (draft phase, verify phase) per (target uid, draft uid, fed
  // tokens, drafts, stop ids, phase); they capture this sampler's buffers, so they live and die with it
  hipStream_t cst = nullptr;
  std::map<std::tuple<uint64_t, uint64_t, int, int, int, int>, std::pair<hipGraphExec_t, hipGraph_t>> cycles;
  ~zl_sampler();
};

struct zl_mat {
  zl::Arena ar;
  std::vector<zl::DevMat> copies;
  hipStream_t st = nullptr;
  ~zl_mat() {
    if (st) hipStreamSynchronize(st);
    ar.release();
    if (st) hipStreamDestroy(st);
  }
};

// Live samplers, so that freeing a model can drop the cycle graphs that captured its buffers.
static std::mutex g_samplers_mu;
static std::set<zl_sampler *> g_samplers;
constexpr size_t CYCLE_GRAPHS_MAX = 64;  // cached cycle graphs per sampler; beyond it the cache starts over

static void drop_cycles(zl_sampler *s, uint64_t uid) {  // uid 0: every entry
  if (s->st) hipStreamSynchronize(s->st);
  if (s->cst) hipStreamSynchronize(s->cst);
  for (auto it = s->cycles.begin(); it != s->cycles.end();) {
    if (uid == 0 || std::get<0>(it->first) == uid || std::get<1>(it->first) == uid) {
      hipGraphExecDestroy(it->second.first);
      hipGraphDestroy(it->second.second);
      it = s->cycles.erase(it);
    } else {
      ++it;
    }
  }
}

zl_model::~zl_model() {
  {
    std::lock_guard<std::mutex> lk(g_samplers_mu);
    for (zl_sampler *s : g_samplers) drop_cycles(s, uid);
  }
  if (st) hipStreamSynchronize(st);
  for (auto &g : graphs) hipGraphExecDestroy(g.second);
  for (auto &g : graphDefs) hipGraphDestroy(g.second);
  ar.release();
  if (st) hipStreamDestroy(st);
  if (cst) hipStreamDestroy(cst);
}

zl_sampler::~zl_sampler() {
  {
    std::lock_guard<std::mutex> lk(g_samplers_mu);
    g_samplers.erase(this);
  }
  if (st) hipStreamSynchronize(st);
  for (auto &c : cycles) { hipGraphExecDestroy(c.second.first); hipGraphDestroy(c.second.second); }
  if (cst) hipStreamDestroy(cst);
  ar.release();
  if (hss) hipHostFree(hss);
  if (hdist) hipHostFree(hdist);
  if (htok) hipHostFree(htok);
  if (st) hipStreamDestroy(st);
}

namespace zl {

// Small kernels that set per-pass state from kernel arguments (no host buffer has to outlive an async copy).
__global__ void k_set_step(Step *d, Step h) { if (threadIdx.x == 0) *d = h; }
struct HistArgs { int n; int ids[128]; };
__global__ void k_set_hist(int *d, HistArgs h) {
  for (int i = threadIdx.x; i < h.n; i += blockDim.x) d[i] = h.ids[i];
}
struct StopArgs { int n; int ids[64]; };
__global__ void k_set_stop(int *d, StopArgs h) {
  for (int i = threadIdx.x; i < h.n; i += blockDim.x) d[i] = h.ids[i];
}
__global__ void k_spec_reset(SpecState *ss) {
  if (threadIdx.x == 0) { ss->kk = 0; ss->stopped = 0; ss->a = 0; ss->tok = -1; }
}
__global__ void k_set_rng(SpecState *ss, uint32_t v) { if (threadIdx.x == 0) ss->rng = v; }

static void set_step(zl_model *m, int pos0, const int *toks, int B) {
  Step h;
  memset(&h, 0, sizeof(h));
  h.pos0 = pos0; h.B = B;
  for (int i = 0; i < B; i++) h.tokens[i] = toks[i];
  hipLaunchKernelGGL(k_set_step, dim3(1), dim3(64), 0, m->st, m->dstep, h);
  ZL_HIP(hipGetLastError());
}

static int qdim(const zl_model *m) { return m->cfg.n_head * m->cfg.head_dim; }
static int kvdim(const zl_model *m) { return m->cfg.n_head_kv * m->cfg.head_dim; }

static int64_t mat_bytes(const DevMat &mm) { int64_t rb = ggml_row_bytes(mm.type, mm.cols); return rb < 0 ? 0 : rb * mm.rows; }

// Quantised activation rows (B rows of ld values, ld a multiple of 64), zeroed; with the f32 copy when f32 is set.
static Act alloc_act(Arena &ar, int B, int ld, bool f32) {
  Act a{};
  a.ld = ld;
  const size_t nb = (size_t)B * (ld / 32);
  auto zalloc = [&](size_t n) { void *p = ar.alloc(n); zero_now(p, n); return p; };
  a.q = (int8_t *)zalloc((size_t)B * ld);
  a.d = (float *)zalloc(nb * 4);
  a.s = (int32_t *)zalloc(nb * 4);
  a.ra = (RecA *)zalloc(nb * sizeof(RecA));
  a.rb = (RecB *)zalloc(nb * sizeof(RecB));
  a.rc = (RecC *)zalloc(nb * sizeof(RecC));
  a.f = f32 ? (float *)zalloc((size_t)B * ld * 4) : nullptr;
  return a;
}

static GemvWork alloc_gemv_work(Arena &ar) {
  GemvWork w;
  w.part = (double *)ar.alloc(GEMV_PART_DOUBLES * 8);
  w.cnt = (uint32_t *)ar.alloc(GEMV_CNT_TILES * 4);
  zero_now(w.cnt, GEMV_CNT_TILES * 4);
  return w;
}

// Allocate KV cache, activations, RoPE tables; compute pass bytes.
static void finish_model(zl_model *m, const float *ropeFreqs) {
  const zl_config &c = m->cfg;
  ZL_REQUIRE(c.head_dim == 128 || c.head_dim == 64 || c.head_dim == 256, ZL_ERR_UNSUPPORTED,
             "head_dim " + std::to_string(c.head_dim) + " is not supported (64, 128 or 256)");
  ZL_REQUIRE(c.n_head % c.n_head_kv == 0, ZL_ERR_UNSUPPORTED, "n_head must be a multiple of n_head_kv");
  // The weighted sum of attention is the reference's position-order f32 chain, bit for bit: for heads of at most 128
  // dimensions at any context (the per-head form beyond AVH_CTX positions keeps its softmax row in the scores buffer),
  // for larger heads wherever the softmax row fits the kernel's LDS (about 29900 positions). Longer contexts of larger
  // heads, or contexts beyond ZEROLLM_ATTN_EXACT_CTX when that is set, take the position-split weighted sum (f64 chunk
  // sums, online-softmax merge): more accurate than the chain, but not its bits, and on random-weight models the
  // difference is amplified through the int8 activation quantisation (see the split-path tests).
  const char *ex = getenv("ZEROLLM_ATTN_EXACT_CTX");
  const AttnForm form = attention_form(m->ctx, c.head_dim);
  const bool split = form.split || (ex && m->ctx > atoi(ex));
  m->attnHeadCtx = form.headCtx;
  m->attnHead1Ctx = form.head1Ctx;
  m->attnMmMinB = form.mmMinB;
  m->attnMmAvMinB = form.mmAvMinB;
  m->attnAvmf = form.avmf;
  const int half = c.n_rot / 2;
  // RoPE tables exactly as ropeTables (src/compute/ref-kernels.js:329-342), in f64 on the host, stored f32
  std::vector<float> cs((size_t)m->ctx * half), sn((size_t)m->ctx * half);
  for (int i = 0; i < half; i++) {
    double freq = pow((double)c.rope_base, (-2.0 * i) / c.n_rot);
    if (ropeFreqs) freq /= (double)ropeFreqs[i];
    for (int p = 0; p < m->ctx; p++) {
      cs[(size_t)p * half + i] = (float)cos(p * freq);
      sn[(size_t)p * half + i] = (float)sin(p * freq);
    }
  }
  m->cosT = (float *)m->ar.alloc(cs.size() * 4);
  m->sinT = (float *)m->ar.alloc(sn.size() * 4);
  ZL_HIP(hipMemcpy(m->cosT, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  ZL_HIP(hipMemcpy(m->sinT, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  // KV cache slots: every layer, or only the attention layers of a hybrid model
  m->nAttn = m->nRec = 0;
  for (auto &L : m->layers) {
    L.ai = L.rec ? -1 : m->nAttn++;
    L.ri = L.rec ? m->nRec++ : -1;
  }
  // K: [slot][kv head][pos][dim]; V: [slot][kv head][dim][vstride] (vstride = ctx rounded up to 16 positions)
  m->vstride = (m->ctx + 15) / 16 * 16;
  const size_t kElems = (size_t)std::max(m->nAttn, 1) * c.n_head_kv * m->ctx * c.head_dim;
  const size_t vElems = (size_t)std::max(m->nAttn, 1) * c.n_head_kv * c.head_dim * m->vstride;
  m->kcache = m->ar.alloc(kElems * (m->kvF16 ? 2 : 4));
  m->vcache = m->ar.alloc(vElems * (m->kvF16 ? 2 : 4));
  zero_now(m->kcache, kElems * (m->kvF16 ? 2 : 4));
  zero_now(m->vcache, vElems * (m->kvF16 ? 2 : 4));
  const int B = m->maxBatch;
  const int inner = m->hybrid ? c.ssm_d_inner : 0;
  if (m->hybrid) {
    const int D = c.ssm_d_state, convDim = 2 * c.ssm_n_group * D + inner;
    m->convFloats = (long)c.ssm_dt_rank * 3 * D * (c.ssm_conv_kernel - 1);
    m->ssmFloats = (long)c.ssm_dt_rank * D * D;
    const size_t sb = (size_t)m->nRec * (m->convFloats + m->ssmFloats) * 4;
    m->state = (float *)m->ar.alloc(std::max<size_t>(sb, 16));
    zero_now(m->state, std::max<size_t>(sb, 16));
    const char *ce = getenv("ZEROLLM_STATE_CAPTURE");
    if (!(ce && ce[0] == '0') && sb > 0) {
      m->capSlots = std::min(m->logitsBatch, DELTA_MAX_B);
      m->capture = (float *)m->ar.alloc(sb * m->capSlots);
    }
    m->dqkv = (float *)m->ar.alloc((size_t)B * convDim * 4);
    m->dz = (float *)m->ar.alloc((size_t)B * inner * 4);
    m->dalpha = (float *)m->ar.alloc((size_t)B * c.ssm_dt_rank * 4);
    m->dbeta = (float *)m->ar.alloc((size_t)B * c.ssm_dt_rank * 4);
    m->dxcore = (float *)m->ar.alloc((size_t)c.ssm_dt_rank * DELTA_MAX_B * c.ssm_d_state * 4);
  }
  m->x = (float *)m->ar.alloc((size_t)B * c.n_embd * 4);
  m->q = (float *)m->ar.alloc((size_t)B * qdim(m) * (m->hybrid ? 2 : 1) * 4);
  m->k = (float *)m->ar.alloc((size_t)B * kvdim(m) * 4);
  m->v = (float *)m->ar.alloc((size_t)B * kvdim(m) * 4);
  m->hb = (float *)m->ar.alloc((size_t)B * c.n_ff * 4);
  m->logits = (float *)m->ar.alloc((size_t)m->logitsBatch * c.vocab * 4);
  m->scores = (float *)m->ar.alloc((size_t)B * c.n_head * m->ctx * 4);
  m->qr = (float *)m->ar.alloc((size_t)B * c.n_head * c.head_dim * 4);
  m->attnInv = (double *)m->ar.alloc((size_t)B * c.n_head * 8);
  if (split) {
    m->attnNch = (m->ctx + ATTN_SPLIT_C - 1) / ATTN_SPLIT_C;
    m->attnPart = (double *)m->ar.alloc((size_t)B * c.n_head * m->attnNch * (c.head_dim + 2) * 8);
  }
  const int ld = pad64(std::max(std::max(c.n_embd, inner), std::max(qdim(m), c.n_ff)));
  m->act = alloc_act(m->ar, B, ld, true);
  m->act2 = alloc_act(m->ar, B, pad64(c.n_ff), false);
  m->gw = alloc_gemv_work(m->ar);
  m->dstep = (Step *)m->ar.alloc(sizeof(Step));
  zero_now(m->dstep, sizeof(Step));
  int64_t wb = 0;
  for (auto &L : m->layers)
    wb += mat_bytes(L.wq) + mat_bytes(L.wk) + mat_bytes(L.wv) + mat_bytes(L.wo) + mat_bytes(L.wgate) + mat_bytes(L.wup) +
          mat_bytes(L.wdown) + mat_bytes(L.wqkv) + mat_bytes(L.wz) + mat_bytes(L.walpha) + mat_bytes(L.wbeta) + mat_bytes(L.wssmout);
  wb += mat_bytes(m->output);
  m->weightBytes = wb;
  ZL_HIP(hipStreamSynchronize(m->st));
}

// ---------------------------------------------------------------------------------------------- forward pass
struct SegSpec { const DevMat *m; float *out; int ldo; const float *bias; };

// Arguments of one GEMV launch over `segs` (laid end to end in tile order; SWIGLU: gate, up on the same tiles).
static GemvArgs gemv_args(const SegSpec *segs, int nseg, int B, int epi, const Act &act, const GemvWork &gw) {
  GemvArgs a;
  memset(&a, 0, sizeof(a));
  ZL_REQUIRE(nseg >= 1 && nseg <= 3, ZL_ERR_ARG, "gemv: 1 to 3 matrices per launch");
  // the kernels take segment 0 alone in the residual and SwiGLU epilogues (no segment selection among the tiles)
  ZL_REQUIRE(epi == EPI_STORE || nseg == (epi == EPI_SWIGLU ? 2 : 1), ZL_ERR_ARG, "gemv: one matrix per residual launch, two per gate/up launch");
  a.nseg = nseg;
  int t0 = 0;
  for (int i = 0; i < a.nseg; i++) {
    const DevMat &mm = *segs[i].m;
    GemvSeg &g = a.seg[i];
    g.m = view(mm);
    g.rows = mm.rows;
    g.out = segs[i].out;
    g.ldo = segs[i].ldo;
    g.bias = segs[i].bias;
    if (is_quant(mm.type)) {
      const long ts = (long)tiles_of(mm.rows) * mm.nslab;
      g.nqs = (uint32_t)(ts * 64 * qs_bytes(mm.type));
      g.nqx = (uint32_t)(ts * 64 * qx_bytes(mm.type));
      g.nsc = (uint32_t)(ts * 64 * sc_bytes(mm.type));
      g.ndd = (uint32_t)(tiles_of(mm.rows) * dd_per_tile(mm.type, mm.nslab) * 2);
    }
    g.tile0 = epi == EPI_SWIGLU ? 0 : t0;
    if (epi != EPI_SWIGLU || i == 0) t0 += tiles_of(mm.rows);
  }
  ZL_REQUIRE(epi != EPI_SWIGLU || (a.nseg == 2 && segs[1].m->rows == segs[0].m->rows), ZL_ERR_ARG, "gemv: gate and up differ");
  a.ntiles = t0;
  a.nslab = segs[0].m->nslab;
  gemv_shape(a.ntiles, a.nslab, epi == EPI_SWIGLU, &a.ks, &a.nwave);
  a.kr = (a.nslab + a.ks - 1) / a.ks;
  a.M = B;
  a.act = act;
  a.part = gw.part;
  a.cnt = gw.cnt;
  return a;
}
static GemvArgs gemv_args(const std::vector<SegSpec> &segs, int B, int epi, const Act &act, const GemvWork &gw) {
  return gemv_args(segs.data(), (int)segs.size(), B, epi, act, gw);
}

// Single-token launches of Q8_0 matrices take the 16-row-group kernel (zl_gemv_rg.hip), which quantises its f32 input
// itself; ZEROLLM_GEMV_RG=0 keeps them on the tile kernels (timing comparisons).
static bool use_rg() {
  static const bool on = [] {
    const char *e = getenv("ZEROLLM_GEMV_RG");
    return !(e && e[0] == '0');
  }();
  return on;
}
// ZEROLLM_GEMV_MIX=0 keeps every store launch a kernel of its own.
static bool use_mix() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("ZEROLLM_GEMV_MIX");
    v = (e && e[0] == '0') ? 0 : 1;
  }
  return v == 1;
}

static bool rg_path(const std::vector<const DevMat *> &ms, int B) {
  if (!use_rg() || B != 1) return false;
  for (const DevMat *d : ms)
    if (d->type != T_Q8_0 || d->nslab > 48) return false;
  return true;
}

// One GEMV launch of the model's pass reading quantised activation `act` (float weights: the f32 rows xf, stride ldx).
// RESID adds into x; SWIGLU writes hb and, with qout set, its quantisation. A single-token Q8_0 launch reads the f32
// rows xf instead and quantises them itself.
static void gemv_group(zl_model *m, const std::vector<SegSpec> &segs, int B, int epi, const Act &act, const float *xf,
                       int ldx, const Act *qout = nullptr) {
  GemvArgs a = gemv_args(segs, B, epi, act, m->gw);
  a.resid = m->x;
  a.ldr = m->cfg.n_embd;
  a.hb = m->hb;
  a.ldh = m->cfg.n_ff;
  if (qout) a.qout = *qout;
  std::vector<const DevMat *> ms;
  for (const SegSpec &sg : segs) ms.push_back(sg.m);
  if (rg_path(ms, B) && xf) {
    a.xf = xf; a.ldxf = ldx; a.xrow0 = 0; a.n = segs[0].m->cols; a.nw = nullptr; a.eps = 0.0;
    a.qout = Act{};
    launch_gemv_rg(a, epi, m->st);
    return;
  }
  launch_gemv(a, epi, xf, ldx, m->st);
}

// RMSNorm (weights nw; none when null) + quantisation of rows x[row0 .. row0+B) (length n, stride ldx) into act.
static void norm_quant(zl_model *m, const float *x, int ldx, int row0, int B, const float *nw, int n, const Act &act) {
  launch_norm_quant(x, ldx, row0, B, nw, (double)m->cfg.rms_eps, n, pad64(n), act, m->st);
}

// A GEMV input that is f32 rows, RMSNorm'd with nw first when nw is set: x[row0 .. row0+B) (length n, stride ldx).
struct Prologue { const float *x; int ldx, row0; const float *nw; int n; };

// Rows of at most this many values in total are quantised inside each GEMV workgroup (the repeated work then costs
// less than a launch); longer ones by one k_norm_quant launch.
constexpr long FUSE_MAX_VALUES = 4096;

// Launches of the same input rows. A launch of quantised matrices with fewer than 256 tiles (few, large workgroups)
// quantises short rows itself; otherwise one k_norm_quant launch writes m->act first, and the f32 normed rows for
// float weights.
// With norm unset the k_norm_quant launch is left out (m->act already holds these rows: GEMV timing probes).
static void gemv_rows(zl_model *m, const std::vector<std::vector<SegSpec>> &groups, const std::vector<int> &epis, int B,
                      const Prologue &p, const Act *qout = nullptr, bool norm = true) {
  std::vector<bool> fused(groups.size()), rg(groups.size());
  bool need = false;
  for (size_t i = 0; i < groups.size(); i++) {
    bool q = true;
    int tiles = 0;
    std::vector<const DevMat *> ms;
    for (size_t k = 0; k < groups[i].size(); k++) {
      q = q && is_quant(groups[i][k].m->type);
      if (epis[i] != EPI_SWIGLU || k == 0) tiles += tiles_of(groups[i][k].m->rows);
      ms.push_back(groups[i][k].m);
    }
    rg[i] = norm && rg_path(ms, B);
    fused[i] = !rg[i] && q && tiles < 256 && (long)B * pad64(p.n) <= FUSE_MAX_VALUES;
    need = need || !(fused[i] || rg[i]);
  }
  if (need && norm) norm_quant(m, p.x, p.ldx, p.row0, B, p.nw, p.n, m->act);
  auto args_of = [&](size_t i) {
    GemvArgs a = gemv_args(groups[i], B, epis[i], m->act, m->gw);
    a.resid = m->x;
    a.ldr = m->cfg.n_embd;
    a.hb = m->hb;
    a.ldh = m->cfg.n_ff;
    if (qout && epis[i] == EPI_SWIGLU && !rg[i]) a.qout = *qout;
    if (fused[i] || rg[i]) {
      a.xf = p.x; a.ldxf = p.ldx; a.xrow0 = p.row0; a.n = p.n; a.nw = p.nw; a.eps = (double)m->cfg.rms_eps;
    }
    return a;
  };
  for (size_t i = 0; i < groups.size(); i++) {
    GemvArgs a = args_of(i);
    if (i + 1 < groups.size() && use_mix() && !rg[i] && !rg[i + 1] && epis[i] == EPI_STORE && epis[i + 1] == EPI_STORE) {
      // a Q4_K store launch on the matrix cores and the next store launch of another format share one kernel
      GemvArgs b = args_of(i + 1);
      b.part += (long)a.ntiles * a.ks * GEMV_MAX_MT * 64 * 2;  // disjoint split-K work spaces
      b.cnt += a.ntiles;
      if ((long)(a.ntiles + b.ntiles) <= GEMV_CNT_TILES &&
          (long)(a.ntiles * a.ks + b.ntiles * b.ks) * 2 * GEMV_MAX_MT * 64 <= GEMV_PART_DOUBLES && gemv_mix_ok(a, b)) {
        launch_gemv_mix(a, b, m->st);
        i++;
        continue;
      }
    }
    if (rg[i]) launch_gemv_rg(a, epis[i], m->st);
    else launch_gemv(a, epis[i], m->act.f, m->act.ld, m->st);
  }
}

// Enqueue one forward pass of B tokens (tokens and positions from m->dstep). want: 0 none, 1 last, 2 all.
static void enqueue_forward(zl_model *m, int B, int want) {
  const zl_config &c = m->cfg;
  const int d = c.n_embd, qd = qdim(m), kvd = kvdim(m), ff = c.n_ff;
  const double eps = (double)c.rms_eps;
  launch_embed(view(m->tokEmbd), m->dstep, B, m->x, d, m->st);
  // consecutive quantised matrices of one type that read the same input share a launch (at most 3 per launch)
  auto group_by_type = [](const std::vector<SegSpec> &v) {
    std::vector<std::vector<SegSpec>> groups;
    size_t i0 = 0;
    while (i0 < v.size()) {
      size_t i1 = i0 + 1;
      while (i1 < v.size() && i1 - i0 < 3 && v[i1].m->type == v[i0].m->type && is_quant(v[i0].m->type)) i1++;
      groups.emplace_back(v.begin() + i0, v.begin() + i1);
      i0 = i1;
    }
    return groups;
  };
  for (int l = 0; l < c.n_layer; l++) {
    Layer &L = m->layers[l];
    if (L.rec) {
      // Gated DeltaNet layer (src/model/forward-qwen35.js:45-61): attn_qkv, attn_gate, ssm_alpha, ssm_beta of the
      // normed rows; the recurrence; ssm_out added to the residual
      const int D = c.ssm_d_state, nV = c.ssm_dt_rank, inner = c.ssm_d_inner, convDim = 2 * c.ssm_n_group * D + inner;
      auto groups = group_by_type({{&L.wqkv, m->dqkv, convDim, nullptr}, {&L.wz, m->dz, inner, nullptr},
                                   {&L.walpha, m->dalpha, nV, nullptr}, {&L.wbeta, m->dbeta, nV, nullptr}});
      gemv_rows(m, groups, std::vector<int>(groups.size(), EPI_STORE), B, Prologue{m->x, d, 0, L.attnNorm, d});
      DeltaArgs da;
      memset(&da, 0, sizeof(da));
      da.qkv = m->dqkv; da.ldqkv = convDim; da.z = m->dz; da.ldz = inner; da.alpha = m->dalpha; da.beta = m->dbeta;
      da.ldab = nV; da.convW = L.conv;
      da.conv = m->state + (long)L.ri * m->convFloats;
      da.ssm = m->state + (long)m->nRec * m->convFloats + (long)L.ri * m->ssmFloats;
      da.dtBias = L.dtBias; da.ssmA = L.ssmA; da.normW = L.ssmNorm;
      da.nK = c.ssm_n_group; da.nV = nV; da.K = c.ssm_conv_kernel; da.B = B; da.eps = eps;
      da.act = m->act; da.out = m->act.f; da.ldo = m->act.ld;
      da.xcore = m->dxcore;
      if (want == 2 && m->capture && B <= m->capSlots) {
        const long stride = (long)m->nRec * (m->convFloats + m->ssmFloats);
        da.capConv = m->capture + (long)L.ri * m->convFloats;
        da.capSsm = m->capture + (long)m->nRec * m->convFloats + (long)L.ri * m->ssmFloats;
        da.capStride = stride;
      }
      launch_deltanet(da, D, m->st);
      gemv_group(m, {{&L.wssmout, nullptr, 0, nullptr}}, B, EPI_RESID, m->act, m->act.f, m->act.ld);
    } else {
      // q, k, v (q rows per head [query | gate] in a hybrid model's gated attention)
      const int qld = m->hybrid ? 2 * qd : qd;
      auto groups = group_by_type({{&L.wq, m->q, qld, L.bq}, {&L.wk, m->k, kvd, L.bk}, {&L.wv, m->v, kvd, L.bv}});
      gemv_rows(m, groups, std::vector<int>(groups.size(), EPI_STORE), B, Prologue{m->x, d, 0, L.attnNorm, d});
      AttnArgs aa;
      memset(&aa, 0, sizeof(aa));
      aa.q = m->q; aa.ldq = qld; aa.kcache = m->kcache; aa.vcache = m->vcache;
      aa.k = m->k; aa.v = m->v; aa.ldkv = kvd; aa.qNorm = L.qNorm; aa.kNorm = L.kNorm; aa.eps = eps;
      aa.cosT = m->cosT; aa.sinT = m->sinT; aa.nRot = c.n_rot; aa.neox = c.neox;
      aa.nHead = c.n_head; aa.nHeadKv = c.n_head_kv; aa.hd = c.head_dim; aa.ctx = m->ctx; aa.layer = L.ai; aa.kvF16 = m->kvF16;
      aa.vstride = m->vstride; aa.hpb = 1; aa.scores = m->scores; aa.sld = m->ctx;
      aa.scale = 1.0 / sqrt((double)c.head_dim);
      aa.step = m->dstep; aa.out = m->act.f; aa.ldo = m->act.ld; aa.act = m->act;
      aa.qhs = m->hybrid ? 2 * c.head_dim : c.head_dim;
      aa.gate = m->hybrid ? m->q + c.head_dim : nullptr;
      aa.part = m->attnPart; aa.nch = m->attnNch; aa.pinv = m->attnInv;
      aa.headCtx = m->attnHeadCtx; aa.head1Ctx = m->attnHead1Ctx;
      aa.mmMinB = m->attnMmMinB; aa.mmAvMinB = m->attnMmAvMinB; aa.qr = m->qr;
      aa.avmf = m->attnAvmf ? 1 : 0;
      // a single-token Q8_0 attn_output GEMV quantises the f32 head outputs itself: the attention writes them alone
      if (rg_path({&L.wo}, B)) aa.act.q = nullptr;
      launch_attention(aa, B, m->st);
      gemv_group(m, {{&L.wo, nullptr, 0, nullptr}}, B, EPI_RESID, m->act, m->act.f, m->act.ld);
    }
    ZL_REQUIRE(L.wgate.type == L.wup.type, ZL_ERR_UNSUPPORTED, "ffn_gate and ffn_up must share a type");
    // the gate/up launch quantises hb for a quantised down matrix itself; otherwise it is quantised here (a
    // single-token Q8_0 down launch quantises hb itself, and a single-token Q8_0 gate/up launch does not quantise it)
    const bool qdown = is_quant(L.wdown.type), fusedq = qdown && is_quant(L.wgate.type);
    const bool guRg = rg_path({&L.wgate, &L.wup}, B), dnRg = rg_path({&L.wdown}, B);
    gemv_rows(m, {{{&L.wgate, nullptr, 0, nullptr}, {&L.wup, nullptr, 0, nullptr}}}, {EPI_SWIGLU}, B,
              Prologue{m->x, d, 0, L.ffnNorm, d}, fusedq && !guRg ? &m->act2 : nullptr);
    if (qdown && !dnRg && (!fusedq || guRg)) norm_quant(m, m->hb, ff, 0, B, nullptr, ff, m->act2);
    gemv_group(m, {{&L.wdown, nullptr, 0, nullptr}}, B, EPI_RESID, m->act2, m->hb, ff);
  }
  if (want == 2) gemv_rows(m, {{{&m->output, m->logits, c.vocab, nullptr}}}, {EPI_STORE}, B, Prologue{m->x, d, 0, m->outputNorm, d});
  else if (want == 1) gemv_rows(m, {{{&m->output, m->logits, c.vocab, nullptr}}}, {EPI_STORE}, 1, Prologue{m->x, d, B - 1, m->outputNorm, d});
}

static hipGraphExec_t graph_for(zl_model *m, int B, int want) {
  const int key = B * 4 + want;
  auto it = m->graphs.find(key);
  if (it != m->graphs.end()) return it->second;
  hipGraph_t g = nullptr;
  hipStream_t run = m->st;
  m->st = m->cst;
  struct Back { zl_model *m; hipStream_t s; ~Back() { m->st = s; } } back{m, run};
  ZL_HIP(hipStreamBeginCapture(m->cst, hipStreamCaptureModeThreadLocal));
  try {
    enqueue_forward(m, B, want);
  } catch (...) {
    hipStreamEndCapture(m->cst, &g);
    if (g) hipGraphDestroy(g);
    throw;
  }
  ZL_HIP(hipStreamEndCapture(m->cst, &g));
  hipGraphExec_t ex;
  ZL_HIP(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
  m->graphs[key] = ex;
  m->graphDefs[key] = g;
  return ex;
}

// Graph capture can be switched off (ZEROLLM_HIP_GRAPHS=0): the same kernels are then launched one by one, which
// some tracing tools need.
static bool use_graphs() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("ZEROLLM_HIP_GRAPHS");
    v = (e && e[0] == '0') ? 0 : 1;
  }
  return v == 1;
}

// Passes of more than ZEROLLM_GRAPH_MAXB tokens are launched kernel by kernel (default: every pass from its graph).
static int graph_max_b() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("ZEROLLM_GRAPH_MAXB");
    v = e ? std::max(0, atoi(e)) : INT_MAX;
  }
  return v;
}

// One pass; the caller has set m->dstep.
static void launch_pass(zl_model *m, int B, int want) {
  m->capN = 0;  // the pass moves the recurrent state: earlier captures no longer describe it
  if (use_graphs() && B <= graph_max_b()) ZL_HIP(hipGraphLaunch(graph_for(m, B, want), m->st));
  else enqueue_forward(m, B, want);
  if (want == 2 && m->capture && B <= m->capSlots) {
    m->capPos0 = (int)m->tokens.size();
    m->capN = B;
  }
}

// Milliseconds per call of `enqueue` (which enqueues work on st), over `iters` calls captured into one HIP graph and
// replayed once after a warm-up replay: launch gaps are then those of the forward pass's graphs.
static float time_graph(hipStream_t st, int iters, const std::function<void(int)> &enqueue) {
  if (!use_graphs()) {
    // graphs switched off (tracing and counter tools): the same launches one by one, timed with events
    for (int i = 0; i < iters; i++) enqueue(i);  // warm-up
    hipEvent_t a, e;
    ZL_HIP(hipEventCreate(&a));
    ZL_HIP(hipEventCreate(&e));
    struct E { hipEvent_t a, b; ~E() { hipEventDestroy(a); hipEventDestroy(b); } } ev{a, e};
    ZL_HIP(hipEventRecord(a, st));
    for (int i = 0; i < iters; i++) enqueue(i);
    ZL_HIP(hipEventRecord(e, st));
    ZL_HIP(hipEventSynchronize(e));
    float t = 0;
    ZL_HIP(hipEventElapsedTime(&t, a, e));
    return t / iters;
  }
  hipGraph_t g = nullptr;
  hipGraphExec_t ex = nullptr;
  ZL_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  try {
    for (int i = 0; i < iters; i++) enqueue(i);
  } catch (...) {
    hipStreamEndCapture(st, &g);
    if (g) hipGraphDestroy(g);
    throw;
  }
  ZL_HIP(hipStreamEndCapture(st, &g));
  struct G { hipGraph_t g; hipGraphExec_t e; ~G() { if (e) hipGraphExecDestroy(e); if (g) hipGraphDestroy(g); } } gg{g, nullptr};
  ZL_HIP(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
  gg.e = ex;
  ZL_HIP(hipGraphLaunch(ex, st));  // warm-up
  hipEvent_t a, e;
  ZL_HIP(hipEventCreate(&a));
  ZL_HIP(hipEventCreate(&e));
  struct E { hipEvent_t a, b; ~E() { hipEventDestroy(a); hipEventDestroy(b); } } ev{a, e};
  ZL_HIP(hipEventRecord(a, st));
  ZL_HIP(hipGraphLaunch(ex, st));
  ZL_HIP(hipEventRecord(e, st));
  ZL_HIP(hipEventSynchronize(e));
  float t = 0;
  ZL_HIP(hipEventElapsedTime(&t, a, e));
  return t / iters;
}

// Time `iters` back-to-back launches of one GEMV of the pass (which: 0 first q/k/v group, 1 wo, 2 gate+up, 3 down,
// 4 output head) with M tokens, cycling through the layers' weights (cache-cold), between two events on the model's
// stream. Uses the model's activation buffers as the last pass left them.
static void probe_gemv(zl_model *m, int which, int M, int iters, float *ms, int64_t *bytes) {
  ZL_REQUIRE(!m->closed, ZL_ERR_STATE, "model is closed");
  ZL_REQUIRE(which >= 0 && which <= 4 && M >= 1 && M <= m->maxBatch && iters >= 1, ZL_ERR_ARG, "bad probe arguments");
  const zl_config &c = m->cfg;
  auto segs_of = [&](int l) -> std::vector<SegSpec> {
    Layer &L = m->layers[l];
    switch (which) {
      case 0: {
        std::vector<SegSpec> v{{&L.wq, m->q, qdim(m), nullptr}};
        if (L.wk.type == L.wq.type) v.push_back({&L.wk, m->k, kvdim(m), nullptr});
        if (L.wk.type == L.wq.type && L.wv.type == L.wq.type) v.push_back({&L.wv, m->v, kvdim(m), nullptr});
        return v;
      }
      case 1: return {{&L.wo, nullptr, 0, nullptr}};
      case 2: return {{&L.wgate, nullptr, 0, nullptr}, {&L.wup, nullptr, 0, nullptr}};
      case 3: return {{&L.wdown, nullptr, 0, nullptr}};
      default: return {{&m->output, m->logits, c.vocab, nullptr}};
    }
  };
  const int epi = which == 1 || which == 3 ? EPI_RESID : which == 2 ? EPI_SWIGLU : EPI_STORE;
  int64_t b = 0;
  for (auto &sg : segs_of(0)) b += mat_bytes(*sg.m);
  *bytes = b;
  // the residual epilogues accumulate into x: keep a copy and restore it afterwards
  float *xsave = (float *)nullptr;
  const size_t xb = (size_t)m->maxBatch * c.n_embd * 4;
  ZL_HIP(hipMalloc(&xsave, xb));
  struct F { float *p; ~F() { hipFree(p); } } fr{xsave};
  ZL_HIP(hipMemcpyAsync(xsave, m->x, xb, hipMemcpyDeviceToDevice, m->st));
  // the GEMV launch exactly as the pass issues it: q/k/v, gate/up and the output head read the residual rows (a fused
  // prologue inside the GEMV, or quantised rows that a k_norm_quant launch wrote first: the warm-up launches write
  // them, the timed launches are the GEMV alone); wo reads the attention output, down the gate/up launch's quantised hb
  auto launch = [&](int l, bool norm) {
    const Layer &L = m->layers[l];
    const int d = c.n_embd;
    if (which == 0) gemv_rows(m, {segs_of(l)}, {EPI_STORE}, M, Prologue{m->x, d, 0, L.attnNorm, d}, nullptr, norm);
    else if (which == 1) gemv_group(m, segs_of(l), M, epi, m->act, m->act.f, m->act.ld);
    else if (which == 2)
      gemv_rows(m, {segs_of(l)}, {EPI_SWIGLU}, M, Prologue{m->x, d, 0, L.ffnNorm, d},
                is_quant(L.wdown.type) && is_quant(L.wgate.type) ? &m->act2 : nullptr, norm);
    else if (which == 3) gemv_group(m, segs_of(l), M, epi, m->act2, m->hb, c.n_ff);
    else gemv_rows(m, {segs_of(l)}, {EPI_STORE}, M, Prologue{m->x, d, 0, m->outputNorm, d}, nullptr, norm);
  };
  for (int l = 0; l < std::min(c.n_layer, iters); l++) launch(which == 4 ? 0 : l, true);  // warm-up (outside capture)
  *ms = time_graph(m->st, iters, [&](int i) { launch(which == 4 ? 0 : i % c.n_layer, false); });
  ZL_HIP(hipMemcpyAsync(m->x, xsave, xb, hipMemcpyDeviceToDevice, m->st));
  ZL_HIP(hipStreamSynchronize(m->st));
}

// PoolModel.forwardBatch checks (src/compute/pool.js:146-155), same messages.
static void check_batch(zl_model *m, const int32_t *tokens, int B, int want) {
  ZL_REQUIRE(!m->closed, ZL_ERR_STATE, "model is closed");
  ZL_REQUIRE(B >= 1 && B <= m->maxBatch, ZL_ERR_BATCH, "batch of " + std::to_string(B) + " tokens (max " + std::to_string(m->maxBatch) + ")");
  const int pos = (int)m->tokens.size();
  ZL_REQUIRE(pos + B <= m->ctx, ZL_ERR_CONTEXT, "context full (" + std::to_string(m->ctx) + " tokens)");
  for (int i = 0; i < B; i++)
    ZL_REQUIRE(tokens[i] >= 0 && tokens[i] < m->cfg.vocab, ZL_ERR_TOKEN, "token id " + std::to_string(tokens[i]) + " out of range");
  ZL_REQUIRE(!(want == 2 && B > m->logitsBatch), ZL_ERR_BATCH,
             "logits for all positions of a batch of " + std::to_string(B) + " tokens (this pool supports " + std::to_string(m->logitsBatch) +
                 "; raise the logitsBatch option)");
}

// One pass of B tokens at the current position (the caller has checked the batch).
static void pass(zl_model *m, const int32_t *tokens, int B, int want) {
  set_step(m, (int)m->tokens.size(), tokens, B);
  launch_pass(m, B, want);
  for (int i = 0; i < B; i++) m->tokens.push_back(tokens[i]);
}

// ---- recurrent-state snapshots of hybrid models (src/model/state-checkpoints.js:42-81), device-to-device copies on the
// model's stream, ordered with the passes
static size_t state_bytes(const zl_model *m) { return (size_t)m->nRec * (m->convFloats + m->ssmFloats) * 4; }

static float *snap_buffer(zl_model *m) {
  if (!m->ck.spare.empty()) {
    float *b = m->ck.spare.back();
    m->ck.spare.pop_back();
    return b;
  }
  return (float *)m->ar.alloc(state_bytes(m));
}

// save (:42-50): a checkpoint of the live state at the current position
static void checkpoint(zl_model *m) {
  Checkpoints &ck = m->ck;
  const int pos = (int)m->tokens.size();
  if (pos == 0 || ck.max <= 0 || ck.has(pos)) return;
  float *buf;
  if ((int)ck.list.size() >= ck.max) {  // drop the smallest position, reuse its buffer
    buf = ck.list.front().buf;
    ck.list.erase(ck.list.begin());
  } else {
    buf = snap_buffer(m);
  }
  ZL_HIP(hipMemcpyAsync(buf, m->state, state_bytes(m), hipMemcpyDeviceToDevice, m->st));
  Snap sn;
  sn.pos = pos;
  sn.buf = buf;
  ck.list.push_back(sn);
  std::sort(ck.list.begin(), ck.list.end(), [](const Snap &a, const Snap &b) { return a.pos < b.pos; });
}

// mark (:53-58): the rollback slot, skipped where a checkpoint holds the position
static void mark_rollback(zl_model *m) {
  Checkpoints &ck = m->ck;
  const int pos = (int)m->tokens.size();
  if (pos == 0 || ck.has(pos)) { ck.rollback.pos = -1; return; }
  if (!ck.rollback.buf) ck.rollback.buf = snap_buffer(m);
  ZL_HIP(hipMemcpyAsync(ck.rollback.buf, m->state, state_bytes(m), hipMemcpyDeviceToDevice, m->st));
  ck.rollback.pos = pos;
}

// restore (:76-81): the live state of snapshot position `from` (0: zeros)
static void restore_state(zl_model *m, int from) {
  if (from == 0) {
    ZL_HIP(hipMemsetAsync(m->state, 0, state_bytes(m), m->st));
    return;
  }
  const Snap *c = m->ck.find(from);
  ZL_REQUIRE(c != nullptr, ZL_ERR_STATE, "no recurrent-state snapshot at position " + std::to_string(from));
  ZL_HIP(hipMemcpyAsync(m->state, c->buf, state_bytes(m), hipMemcpyDeviceToDevice, m->st));
}

// PoolModel.#hybridBatch (src/compute/pool.js:182-196): a snapshot before the tokens the policy names; the batch is split
// there (never when every position returns logits), segments run as separate passes.
// Returns the size of the last pass.
static int hybrid_batch(zl_model *m, const int32_t *tokens, int B, int want) {
  Checkpoints &ck = m->ck;
  const int pos = (int)m->tokens.size();
  if (ck.wants_before(pos, tokens[0], want == 2 || (want == 1 && B == 1), m->prevNoLogits)) checkpoint(m);
  std::vector<int> cuts{0};
  if (want != 2)
    for (int i = 1; i < B; i++)
      if (ck.wants_before(pos + i, tokens[i], want == 1 && i == B - 1, true)) cuts.push_back(i);
  cuts.push_back(B);
  for (size_t c = 0; c + 1 < cuts.size(); c++) {
    if (c > 0) checkpoint(m);
    const bool last = c + 2 == cuts.size();
    pass(m, tokens + cuts[c], cuts[c + 1] - cuts[c], last ? want : 0);
  }
  m->prevNoLogits = want == 0;
  return cuts[cuts.size() - 1] - cuts[cuts.size() - 2];
}

static void forward(zl_model *m, const int32_t *tokens, int B, int want) {
  check_batch(m, tokens, B, want);
  if (m->hybrid) hybrid_batch(m, tokens, B, want);
  else pass(m, tokens, B, want);
}

// PoolModel.truncate (src/compute/pool.js:278-294): positional KV is bookkeeping; a hybrid model restores the nearest
// snapshot at or before n and replays the tokens in between (passes of at most maxBatch tokens). Returns the replay count.
static int truncate_model(zl_model *m, int n) {
  const int pos = (int)m->tokens.size();
  if (n >= pos) return 0;
  if (n < 0) n = 0;
  if (!m->hybrid) {
    m->tokens.resize(n);
    return 0;
  }
  ZL_REQUIRE(!m->closed, ZL_ERR_STATE, "model is closed");
  int from, replay;
  m->ck.plan(n, pos, &from, &replay);
  // the state after n tokens was captured by the last verify pass: copy it instead of restore + replay (the same bits:
  // the replay would run the same tokens from the same state). Only without boundary / periodic checkpoints, whose
  // snapshots a replay would also take; the replay count, the checkpoint after it and the rollback slot are as the
  // reference leaves them.
  if (replay > 0 && m->capN > 0 && n > m->capPos0 && n <= m->capPos0 + m->capN && m->ck.boundary.empty() &&
      m->ck.every == 0) {
    m->ck.drop_after(n);
    ZL_HIP(hipMemcpyAsync(m->state, m->capture + (size_t)(n - m->capPos0 - 1) * (state_bytes(m) / 4), state_bytes(m),
                          hipMemcpyDeviceToDevice, m->st));
    m->tokens.resize(n);
    m->capN = n - m->capPos0;  // positions up to n keep their captured states
    checkpoint(m);
    m->prevNoLogits = false;
    return replay;
  }
  std::vector<int32_t> tail(m->tokens.begin() + from, m->tokens.begin() + n);
  m->ck.drop_after(n);
  restore_state(m, from);
  m->tokens.resize(from);
  m->prevNoLogits = false;
  for (size_t i = 0; i < tail.size(); i += m->maxBatch)
    hybrid_batch(m, tail.data() + i, (int)std::min<size_t>(m->maxBatch, tail.size() - i), 0);
  if (replay > 0) checkpoint(m);
  m->prevNoLogits = false;
  return replay;
}

static void reset_model(zl_model *m) {
  m->tokens.clear();
  if (m->hybrid) {
    ZL_HIP(hipMemsetAsync(m->state, 0, state_bytes(m), m->st));
    m->ck.clear();
    m->prevNoLogits = false;
  }
}

// ---------------------------------------------------------------------------------------------- construction
static zl_model *new_model(const zl_model_opts *o) {
  static std::atomic<uint64_t> next_uid{1};
  std::unique_ptr<zl_model> m(new zl_model());
  m->uid = next_uid++;
  int mb = o && o->max_batch > 0 ? o->max_batch : 16;
  m->maxBatch = std::max(1, std::min(mb, 64));
  int lb = o && o->logits_batch > 0 ? o->logits_batch : 16;
  m->logitsBatch = std::max(1, std::min(lb, m->maxBatch));
  m->kvF16 = o ? (o->kv_f16 ? 1 : 0) : 0;
  if (o && o->max_checkpoints != 0) m->ck.max = std::max(0, o->max_checkpoints);
  if (o && o->checkpoint_every > 0) m->ck.every = o->checkpoint_every;
  if (o && o->boundary_ids) for (int i = 0; i < o->n_boundary; i++) m->ck.boundary.insert(o->boundary_ids[i]);
  ZL_HIP(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
  ZL_HIP(hipStreamCreateWithFlags(&m->cst, hipStreamNonBlocking));
  return m.release();
}

static void check_config(const zl_config &c) {
  ZL_REQUIRE(c.n_embd > 0 && c.n_layer > 0 && c.n_ff > 0 && c.n_head > 0 && c.n_head_kv > 0 && c.head_dim > 0 && c.vocab > 0,
             ZL_ERR_ARG, "bad model config");
  ZL_REQUIRE(c.n_rot > 0 && c.n_rot <= c.head_dim && c.n_rot % 2 == 0, ZL_ERR_ARG, "bad rope dimension count");
  if (c.hybrid) {
    // qwen35 layout checks (src/model/config.js:146-151) and what the DeltaNet kernel takes
    ZL_REQUIRE(c.full_attn_interval >= 1 && c.ssm_n_group > 0 && c.ssm_dt_rank > 0 && c.ssm_d_state > 0, ZL_ERR_FORMAT, "bad qwen35 layout");
    ZL_REQUIRE(c.ssm_d_inner % c.ssm_dt_rank == 0, ZL_ERR_FORMAT, "ssm.inner_size is not a multiple of ssm.time_step_rank");
    ZL_REQUIRE(c.ssm_dt_rank % c.ssm_n_group == 0, ZL_ERR_FORMAT, "ssm.time_step_rank is not a multiple of ssm.group_count");
    ZL_REQUIRE(c.ssm_d_inner / c.ssm_dt_rank == c.ssm_d_state, ZL_ERR_UNSUPPORTED, "DeltaNet value and key head sizes differ");
    ZL_REQUIRE(c.ssm_conv_kernel == 4, ZL_ERR_UNSUPPORTED, "DeltaNet conv kernel must be 4");
  }
}

static float *upload_vec(zl_model *m, const std::vector<float> &v) {
  float *p = (float *)m->ar.alloc(v.size() * 4);
  ZL_HIP(hipMemcpy(p, v.data(), v.size() * 4, hipMemcpyHostToDevice));
  return p;
}

// ---- from GGUF (modelConfig, src/model/config.js:275-325; tensors as RefModel, src/model/forward.js:114-132)
static zl_model *load_gguf(const char *path, const zl_model_opts *o) {
  GGUF g = read_gguf(path);
  const GGUFValue *av = g.get("general.architecture");
  ZL_REQUIRE(av && av->type == 8, ZL_ERR_FORMAT, "GGUF has no general.architecture");
  const std::string arch = av->str;
  int archId = arch == "llama" ? 0 : arch == "qwen2" ? 1 : arch == "qwen3" ? 2 : arch == "qwen35" ? 3 : -1;
  ZL_REQUIRE(archId >= 0, ZL_ERR_UNSUPPORTED, "architecture \"" + arch + "\" is not supported by the HIP path (supported: llama, qwen2, qwen3, qwen35)");
  auto need = [&](const std::string &k) {
    const GGUFValue *v = g.get(arch + "." + k);
    ZL_REQUIRE(v != nullptr, ZL_ERR_FORMAT, "GGUF is missing metadata key " + arch + "." + k);
    return v->num;
  };
  zl_config c{};
  c.arch = archId;
  c.n_embd = (int)need("embedding_length");
  c.n_head = (int)need("attention.head_count");
  c.n_head_kv = (int)g.num(arch + ".attention.head_count_kv", c.n_head);
  double hd = g.num(arch + ".attention.key_length", (double)c.n_embd / c.n_head);
  ZL_REQUIRE(hd == (double)(int)hd, ZL_ERR_FORMAT, "cannot determine integer head_dim");
  c.head_dim = (int)hd;
  const GGUFTensor *te = g.tensor("token_embd.weight");
  const GGUFValue *toks = g.get("tokenizer.ggml.tokens");
  double vs = g.num(arch + ".vocab_size", -1);
  if (vs < 0) vs = toks && toks->type == 9 ? (double)toks->arrLen : te ? (double)te->dims[1] : -1;
  ZL_REQUIRE(vs > 0, ZL_ERR_FORMAT, "cannot determine vocab size");
  c.vocab = (int)vs;
  c.n_layer = (int)need("block_count");
  if (archId == 3) {
    // qwen35 (src/model/config.js:93-97, 126-156): block_count includes trailing multi-token-prediction blocks
    c.n_layer -= (int)g.num(arch + ".nextn_predict_layers", 0);
    c.hybrid = 1;
    c.full_attn_interval = (int)g.num(arch + ".full_attention_interval", 4);
    c.ssm_conv_kernel = (int)need("ssm.conv_kernel");
    c.ssm_d_state = (int)need("ssm.state_size");
    c.ssm_n_group = (int)need("ssm.group_count");
    c.ssm_dt_rank = (int)need("ssm.time_step_rank");
    c.ssm_d_inner = (int)need("ssm.inner_size");
  }
  c.n_ctx_train = (int)need("context_length");
  c.n_ff = (int)need("feed_forward_length");
  c.n_rot = (int)g.num(arch + ".rope.dimension_count", c.head_dim);
  c.rms_eps = (float)g.num(arch + ".attention.layer_norm_rms_epsilon", 1e-5);
  c.rope_base = (float)g.num(arch + ".rope.freq_base", 10000);
  c.neox = archId != 0;
  c.qk_norm = c.hybrid || g.tensor("blk.0.attn_q_norm.weight") != nullptr;
  c.qkv_bias = g.tensor("blk.0.attn_q.bias") != nullptr;
  c.tied = g.tensor("output.weight") == nullptr;
  c.has_rope_freqs = g.tensor("rope_freqs.weight") != nullptr;
  check_config(c);

  std::unique_ptr<zl_model> m(new_model(o));
  m->cfg = c;
  int want_ctx = o && o->ctx > 0 ? o->ctx : 2048;
  m->ctx = std::min(want_ctx, c.n_ctx_train);
  FILE *f = fopen(path, "rb");
  ZL_REQUIRE(f != nullptr, ZL_ERR_IO, std::string("cannot open ") + path);
  struct Closer { FILE *f; ~Closer() { fclose(f); } } closer{f};
  // staging: pinned host chunk + device buffer sized for the largest tensor
  uint64_t maxBytes = 0;
  for (auto &t : g.tensors) maxBytes = std::max(maxBytes, t.nBytes);
  uint8_t *dstage = (uint8_t *)nullptr;
  ZL_HIP(hipMalloc(&dstage, std::max<uint64_t>(maxBytes, 16)));
  const size_t CH = 64u << 20;
  uint8_t *hst = nullptr;
  ZL_HIP(hipHostMalloc(&hst, CH));
  struct Freer { uint8_t *d, *h; ~Freer() { hipFree(d); hipHostFree(h); } } freer{dstage, hst};
  auto read_dev = [&](const GGUFTensor &t) {
    for (uint64_t off = 0; off < t.nBytes; off += CH) {
      size_t n = (size_t)std::min<uint64_t>(CH, t.nBytes - off);
      ZL_HIP(hipStreamSynchronize(m->st));
      if (fseeko(f, (off_t)(t.absOffset + off), SEEK_SET) != 0 || fread(hst, 1, n, f) != n)
        throw Error(ZL_ERR_IO, "tensor " + t.name + ": unexpected end of file");
      ZL_HIP(hipMemcpyAsync(dstage + off, hst, n, hipMemcpyHostToDevice, m->st));
    }
    ZL_HIP(hipStreamSynchronize(m->st));
  };
  auto req = [&](const std::string &n) -> const GGUFTensor & {
    const GGUFTensor *t = g.tensor(n);
    ZL_REQUIRE(t != nullptr, ZL_ERR_FORMAT, "tensor not found in GGUF: " + n);
    return *t;
  };
  auto W = [&](const std::string &n, int rows, int cols) {
    const GGUFTensor &t = req(n);
    ZL_REQUIRE(t.dims.size() >= 2 && (int)t.dims[0] == cols && (int)t.dims[1] == rows, ZL_ERR_FORMAT, "tensor " + n + " has unexpected shape");
    read_dev(t);
    DevMat mm = make_mat(m->ar, t.type, rows, cols, dstage, m->st);
    ZL_HIP(hipStreamSynchronize(m->st));
    return mm;
  };
  auto V = [&](const std::string &n, int len) -> float * {
    const GGUFTensor &t = req(n);
    ZL_REQUIRE((int)t.dims[0] == len, ZL_ERR_FORMAT, "tensor " + n + " has unexpected length");
    std::vector<uint8_t> raw(t.nBytes);
    if (fseeko(f, (off_t)t.absOffset, SEEK_SET) != 0 || fread(raw.data(), 1, t.nBytes, f) != t.nBytes) throw Error(ZL_ERR_IO, "tensor " + n + ": read failed");
    std::vector<float> v(len);
    if (t.type == T_F32) memcpy(v.data(), raw.data(), (size_t)len * 4);
    else throw Error(ZL_ERR_UNSUPPORTED, "vector tensor " + n + " must be F32");
    return upload_vec(m.get(), v);
  };
  auto Vopt = [&](const std::string &n, int len) -> float * { return g.tensor(n) ? V(n, len) : nullptr; };
  // an F32 tensor of any shape with `count` values (ssm_conv1d [kernel, channels])
  auto VN = [&](const std::string &n, long count) -> float * {
    const GGUFTensor &t = req(n);
    long e = 1;
    for (auto d : t.dims) e *= (long)d;
    ZL_REQUIRE(t.type == T_F32 && e == count, ZL_ERR_FORMAT, "tensor " + n + " has unexpected type or size");
    std::vector<float> v(count);
    if (fseeko(f, (off_t)t.absOffset, SEEK_SET) != 0 || fread(v.data(), 4, count, f) != (size_t)count) throw Error(ZL_ERR_IO, "tensor " + n + ": read failed");
    return upload_vec(m.get(), v);
  };
  auto group = [&](const std::vector<std::string> &nm, const std::vector<int> &rows, int cols) {
    std::vector<int> types;
    for (size_t i = 0; i < nm.size(); i++) {
      const GGUFTensor &t = req(nm[i]);
      ZL_REQUIRE(t.dims.size() >= 2 && (int)t.dims[0] == cols && (int)t.dims[1] == rows[i], ZL_ERR_FORMAT, "tensor " + nm[i] + " has unexpected shape");
      types.push_back(t.type);
    }
    return make_group(m->ar, types, rows, cols, [&](size_t i) { read_dev(req(nm[i])); }, dstage, m->st);
  };
  const int qd = c.n_head * c.head_dim, kvd = c.n_head_kv * c.head_dim;
  m->hybrid = c.hybrid != 0;
  m->tokEmbd = W("token_embd.weight", c.vocab, c.n_embd);
  m->outputNorm = V("output_norm.weight", c.n_embd);
  m->output = c.tied ? m->tokEmbd : W("output.weight", c.vocab, c.n_embd);
  std::vector<float> ropeFreqs;
  if (c.has_rope_freqs) {
    const GGUFTensor &t = req("rope_freqs.weight");
    ropeFreqs.resize(t.dims[0]);
    if (fseeko(f, (off_t)t.absOffset, SEEK_SET) != 0 || fread(ropeFreqs.data(), 4, t.dims[0], f) != t.dims[0]) throw Error(ZL_ERR_IO, "rope_freqs read failed");
  }
  for (int l = 0; l < c.n_layer; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    Layer L;
    L.attnNorm = V(p + "attn_norm.weight", c.n_embd);
    L.rec = m->hybrid && (l + 1) % c.full_attn_interval != 0;
    if (L.rec) {
      // Gated DeltaNet layer tensors (src/model/forward-qwen35.js:111-132, 186-194)
      const int D = c.ssm_d_state, nV = c.ssm_dt_rank, inner = c.ssm_d_inner, convDim = 2 * c.ssm_n_group * D + inner;
      auto g4 = group({p + "attn_qkv.weight", p + "attn_gate.weight", p + "ssm_alpha.weight", p + "ssm_beta.weight"},
                      {convDim, inner, nV, nV}, c.n_embd);
      L.wqkv = g4[0]; L.wz = g4[1]; L.walpha = g4[2]; L.wbeta = g4[3];
      L.conv = VN(p + "ssm_conv1d.weight", (long)convDim * c.ssm_conv_kernel);
      L.dtBias = V(p + "ssm_dt.bias", nV);
      L.ssmA = V(p + "ssm_a", nV);
      L.ssmNorm = V(p + "ssm_norm.weight", D);
      L.wssmout = W(p + "ssm_out.weight", c.n_embd, inner);
    } else {
      auto g3 = group({p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"}, {m->hybrid ? 2 * qd : qd, kvd, kvd}, c.n_embd);
      L.wq = g3[0]; L.wk = g3[1]; L.wv = g3[2];
      L.wo = W(p + "attn_output.weight", c.n_embd, qd);
      L.bq = Vopt(p + "attn_q.bias", qd); L.bk = Vopt(p + "attn_k.bias", kvd); L.bv = Vopt(p + "attn_v.bias", kvd);
      L.qNorm = Vopt(p + "attn_q_norm.weight", c.head_dim); L.kNorm = Vopt(p + "attn_k_norm.weight", c.head_dim);
    }
    L.ffnNorm = V(p + (m->hybrid ? "post_attention_norm.weight" : "ffn_norm.weight"), c.n_embd);
    L.wgate = W(p + "ffn_gate.weight", c.n_ff, c.n_embd);
    L.wup = W(p + "ffn_up.weight", c.n_ff, c.n_embd);
    L.wdown = W(p + "ffn_down.weight", c.n_embd, c.n_ff);
    m->layers.push_back(L);
  }
  finish_model(m.get(), c.has_rope_freqs ? ropeFreqs.data() : nullptr);
  return m.release();
}

// ---- synthetic
static void synth_to_device(const zl_synth_tensor &t, uint8_t *out, hipStream_t st) {
  ZL_REQUIRE(zl_synth::block_values(t.type) > 0, ZL_ERR_UNSUPPORTED, "synthetic tensors support F32, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K");
  ZL_REQUIRE(t.cols % zl_synth::block_values(t.type) == 0, ZL_ERR_ARG, std::string("synthetic tensor ") + (t.name ? t.name : "") + ": cols not a whole number of blocks");
  launch_synth(t.type, t.seed, t.std, (uint64_t)(t.src_cols > 0 ? t.src_cols : t.cols), (uint64_t)t.col0, (int)t.rows, (int)t.cols, out, st);
}

static zl_model *build_synth(const zl_config *cfg, const zl_synth_tensor *ts, int n, const zl_model_opts *o) {
  zl_config c = *cfg;
  check_config(c);
  std::map<std::string, const zl_synth_tensor *> byName;
  for (int i = 0; i < n; i++) byName[ts[i].name] = &ts[i];
  std::unique_ptr<zl_model> m(new_model(o));
  m->cfg = c;
  int want_ctx = o && o->ctx > 0 ? o->ctx : 2048;
  m->ctx = std::min(want_ctx, c.n_ctx_train);
  size_t maxBytes = 16;
  for (int i = 0; i < n; i++) if (!ts[i].fill) maxBytes = std::max(maxBytes, (size_t)ggml_row_bytes(ts[i].type, ts[i].cols) * (size_t)ts[i].rows);
  uint8_t *dstage = nullptr;
  ZL_HIP(hipMalloc(&dstage, maxBytes));
  struct Freer { uint8_t *d; ~Freer() { hipFree(d); } } freer{dstage};
  auto req = [&](const std::string &nm) -> const zl_synth_tensor & {
    auto it = byName.find(nm);
    ZL_REQUIRE(it != byName.end(), ZL_ERR_ARG, "synthetic model has no tensor " + nm);
    return *it->second;
  };
  auto W = [&](const std::string &nm, int rows, int cols) {
    const zl_synth_tensor &t = req(nm);
    ZL_REQUIRE(t.rows == rows && t.cols == cols && !t.fill, ZL_ERR_ARG, "synthetic tensor " + nm + " has unexpected shape");
    synth_to_device(t, dstage, m->st);
    DevMat mm = make_mat(m->ar, t.type, rows, cols, dstage, m->st);
    ZL_HIP(hipStreamSynchronize(m->st));
    return mm;
  };
  auto V = [&](const std::string &nm, int len) -> float * {
    const zl_synth_tensor &t = req(nm);
    ZL_REQUIRE(t.rows * t.cols == len, ZL_ERR_ARG, "synthetic vector " + nm + " has unexpected length");
    if (t.fill == 1) return upload_vec(m.get(), std::vector<float>(len, t.fill_value));
    if (t.fill == 2 || t.fill == 3) {
      std::vector<float> v(len);
      const int rc = zl_synth_tensor_bytes(&t, 0, v.data());
      ZL_REQUIRE(rc == ZL_OK, rc, "synthetic vector " + nm + ": " + g_err);
      return upload_vec(m.get(), v);
    }
    ZL_REQUIRE(t.type == T_F32, ZL_ERR_ARG, "synthetic vector " + nm + " must be F32");
    float *p = (float *)m->ar.alloc((size_t)len * 4);
    synth_to_device(t, (uint8_t *)p, m->st);
    return p;
  };
  auto Vopt = [&](const std::string &nm, int len) -> float * { return byName.count(nm) ? V(nm, len) : nullptr; };
  const int qd = c.n_head * c.head_dim, kvd = c.n_head_kv * c.head_dim;
  m->hybrid = c.hybrid != 0;
  m->tokEmbd = W("token_embd.weight", c.vocab, c.n_embd);
  m->outputNorm = V("output_norm.weight", c.n_embd);
  m->output = c.tied ? m->tokEmbd : W("output.weight", c.vocab, c.n_embd);
  // matrices read by one launch: consecutive ones of a type share an allocation
  auto group = [&](const std::vector<std::string> &nm, const std::vector<int> &rows, int cols) {
    std::vector<int> types;
    for (size_t i = 0; i < nm.size(); i++) {
      const zl_synth_tensor &t = req(nm[i]);
      ZL_REQUIRE(t.rows == rows[i] && t.cols == cols && !t.fill, ZL_ERR_ARG, "synthetic tensor " + nm[i] + " has unexpected shape");
      types.push_back(t.type);
    }
    return make_group(m->ar, types, rows, cols, [&](size_t i) { synth_to_device(req(nm[i]), dstage, m->st); }, dstage, m->st);
  };
  for (int l = 0; l < c.n_layer; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    Layer L;
    L.attnNorm = V(p + "attn_norm.weight", c.n_embd);
    L.rec = m->hybrid && (l + 1) % c.full_attn_interval != 0;
    if (L.rec) {
      const int D = c.ssm_d_state, nV = c.ssm_dt_rank, inner = c.ssm_d_inner, convDim = 2 * c.ssm_n_group * D + inner;
      auto g4 = group({p + "attn_qkv.weight", p + "attn_gate.weight", p + "ssm_alpha.weight", p + "ssm_beta.weight"},
                      {convDim, inner, nV, nV}, c.n_embd);
      L.wqkv = g4[0]; L.wz = g4[1]; L.walpha = g4[2]; L.wbeta = g4[3];
      L.conv = V(p + "ssm_conv1d.weight", convDim * c.ssm_conv_kernel);
      L.dtBias = V(p + "ssm_dt.bias", nV);
      L.ssmA = V(p + "ssm_a", nV);
      L.ssmNorm = V(p + "ssm_norm.weight", D);
      L.wssmout = W(p + "ssm_out.weight", c.n_embd, inner);
      L.ffnNorm = V(p + "post_attention_norm.weight", c.n_embd);
      L.wgate = W(p + "ffn_gate.weight", c.n_ff, c.n_embd);
      L.wup = W(p + "ffn_up.weight", c.n_ff, c.n_embd);
      L.wdown = W(p + "ffn_down.weight", c.n_embd, c.n_ff);
      m->layers.push_back(L);
      continue;
    }
    {
      auto g3 = group({p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"}, {m->hybrid ? 2 * qd : qd, kvd, kvd}, c.n_embd);
      L.wq = g3[0]; L.wk = g3[1]; L.wv = g3[2];
    }
    L.wo = W(p + "attn_output.weight", c.n_embd, qd);
    L.bq = Vopt(p + "attn_q.bias", qd); L.bk = Vopt(p + "attn_k.bias", kvd); L.bv = Vopt(p + "attn_v.bias", kvd);
    L.qNorm = Vopt(p + "attn_q_norm.weight", c.head_dim); L.kNorm = Vopt(p + "attn_k_norm.weight", c.head_dim);
    L.ffnNorm = V(p + (m->hybrid ? "post_attention_norm.weight" : "ffn_norm.weight"), c.n_embd);
    L.wgate = W(p + "ffn_gate.weight", c.n_ff, c.n_embd);
    L.wup = W(p + "ffn_up.weight", c.n_ff, c.n_embd);
    L.wdown = W(p + "ffn_down.weight", c.n_embd, c.n_ff);
    m->layers.push_back(L);
  }
  ZL_REQUIRE(!c.has_rope_freqs, ZL_ERR_UNSUPPORTED, "synthetic models do not take rope_freqs");
  finish_model(m.get(), nullptr);
  return m.release();
}

// ---------------------------------------------------------------------------------------------- sampler
static zl_sampler *new_sampler(const zl_sampler_opts *o) {
  std::unique_ptr<zl_sampler> s(new zl_sampler());
  SamplerParams &p = s->sp;
  p.temperature = o->temperature; p.topP = o->top_p; p.minP = o->min_p; p.repeatPenalty = o->repeat_penalty;
  p.presence = o->presence_penalty; p.frequency = o->frequency_penalty; p.topK = o->top_k; p.repeatLastN = o->repeat_last_n;
  p.penalized = (p.repeatPenalty != 1.0 || p.presence != 0.0 || p.frequency != 0.0) ? 1 : 0;
  p.greedyArgmax = o->greedy_argmax ? 1 : 0;
  s->wide = !(p.temperature <= 0.0 || p.greedyArgmax) && (p.topK <= 0 || p.topK > KCAP);
  ZL_HIP(hipStreamCreateWithFlags(&s->st, hipStreamNonBlocking));
  s->ss = (SpecState *)s->ar.alloc(sizeof(SpecState));
  zero_now(s->ss, sizeof(SpecState));
  ZL_HIP(hipHostMalloc((void **)&s->hss, sizeof(SpecState)));
  s->pdist = (DevDist *)s->ar.alloc(sizeof(DevDist) * 65);
  s->qdist = (DevDist *)s->ar.alloc(sizeof(DevDist) * 64);
  s->tmpdist = (DevDist *)s->ar.alloc(sizeof(DevDist));
  zero_now(s->pdist, sizeof(DevDist) * 65);  // fixed lists: null full-list pointers
  zero_now(s->qdist, sizeof(DevDist) * 64);
  zero_now(s->tmpdist, sizeof(DevDist));
  ZL_HIP(hipHostMalloc((void **)&s->hdist, sizeof(DevDist)));
  s->dhist = (int *)s->ar.alloc(sizeof(int) * 256);
  s->dstop = (int *)s->ar.alloc(sizeof(int) * 64);
  s->dtok = (int *)s->ar.alloc(sizeof(int) * 4);
  ZL_HIP(hipHostMalloc((void **)&s->htok, sizeof(int) * 4));
  s->am.keys = (unsigned long long *)s->ar.alloc(sizeof(unsigned long long) * ARGMAX_MAX_ROWS * ARGMAX_MAX_BLOCKS);
  s->am.count = (uint32_t *)s->ar.alloc(sizeof(uint32_t) * ARGMAX_MAX_ROWS);
  zero_now(s->am.count, sizeof(uint32_t) * ARGMAX_MAX_ROWS);
  hipLaunchKernelGGL(k_set_rng, dim3(1), dim3(64), 0, s->st, s->ss, o->seed);
  ZL_HIP(hipGetLastError());
  ZL_HIP(hipStreamSynchronize(s->st));
  return s.release();
}

// The sampler's work space for rows of `vocab` logits: the penalised copies of up to 65 rows, and for full candidate
// lists their sort buffers and each distribution's storage (65 target rows, 64 draft rows, one for single draws).
// Allocated before any graph capture that uses them; storage for a smaller vocabulary stays allocated (graphs
// captured with it keep their pointers).
static void ensure_scratch(zl_sampler *s, int vocab) {
  if ((s->sp.penalized || s->wide) && s->scratchVocab < vocab) {
    s->scratch = (float *)s->ar.alloc((size_t)65 * vocab * 4);
    s->scratchVocab = vocab;
  }
  const bool sampled = !(s->sp.temperature <= 0.0 || s->sp.greedyArgmax);
  if (sampled && !s->wide && !s->sp.penalized && s->cw.vocab < vocab) {
    const size_t nb = (size_t)(vocab + CAND_CHUNK - 1) / CAND_CHUNK, n = 65 * nb * CAND_CMAX;
    s->cw.ids = (int *)s->ar.alloc(n * 4);
    s->cw.vals = (float *)s->ar.alloc(n * 4);
    s->cw.cnt = (int *)s->ar.alloc(65 * nb * 4);
    s->cw.vocab = vocab;
    s->cw.rows = 65;
  }
  if (!s->wide || s->ww.vocab >= vocab) return;
  const size_t n = (size_t)65 * vocab, nch = (vocab + WIDE_CHUNK - 1) / WIDE_CHUNK;
  s->ww.keyA = (uint32_t *)s->ar.alloc(n * 4);
  s->ww.keyB = (uint32_t *)s->ar.alloc(n * 4);
  s->ww.idA = (int *)s->ar.alloc(n * 4);
  s->ww.idB = (int *)s->ar.alloc(n * 4);
  s->ww.hist = (uint32_t *)s->ar.alloc((size_t)65 * 256 * nch * 4);
  s->ww.vocab = vocab;
  s->ww.rows = 65;
  auto give = [&](DevDist *d, int cnt) {
    const size_t m = (size_t)cnt * vocab;
    launch_set_wide(d, cnt, vocab, (int *)s->ar.alloc(m * 4), (double *)s->ar.alloc(m * 8), (int *)s->ar.alloc(m * 4),
                    (double *)s->ar.alloc(m * 8), s->st);
  };
  give(s->pdist, 65);
  give(s->qdist, 64);
  give(s->tmpdist, 1);
  ZL_HIP(hipStreamSynchronize(s->st));
}

// Upload the last repeatLastN ids of a history (only those can matter) and return how many were kept.
static int upload_hist(zl_sampler *s, hipStream_t st, const int32_t *hist, int nh) {
  if (!s->sp.penalized || !hist || nh <= 0) return 0;
  int keep = std::min(nh, s->sp.repeatLastN);
  HistArgs h;
  h.n = keep;
  for (int i = 0; i < keep; i++) h.ids[i] = hist[nh - keep + i];
  hipLaunchKernelGGL(k_set_hist, dim3(1), dim3(128), 0, st, s->dhist, h);
  ZL_HIP(hipGetLastError());
  return keep;
}

// Make stream `a` wait for the work already queued on stream `b`.
static void stream_wait(hipStream_t a, hipStream_t b) {
  if (a == b) return;
  hipEvent_t e;
  ZL_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  ZL_HIP(hipEventRecord(e, b));
  ZL_HIP(hipStreamWaitEvent(a, e, 0));
  ZL_HIP(hipEventDestroy(e));
}

static void dist_of_row(zl_sampler *s, zl_model *m, int row, const int32_t *hist, int nh, DevDist *out) {
  ZL_REQUIRE(!m->closed, ZL_ERR_STATE, "model is closed");
  ZL_REQUIRE(row >= 0 && row < m->logitsBatch, ZL_ERR_ARG, "logits row out of range");
  ensure_scratch(s, m->cfg.vocab);
  const int keep = upload_hist(s, m->st, hist, nh);
  launch_dist_rows(m->logits + (size_t)row * m->cfg.vocab, m->cfg.vocab, 1, m->cfg.vocab, s->sp, keep ? s->dhist : nullptr, keep, 0,
                   s->scratch, s->am, s->wide ? &s->ww : nullptr, &s->cw, out, m->st);
}

// ---------------------------------------------------------------------------------------------- speculative cycle
// The work `body` enqueues on stream cs, captured and instantiated as one graph.
template <class F>
static hipGraphExec_t capture_graph(hipStream_t cs, F &&body, hipGraph_t *def) {
  hipGraph_t g = nullptr;
  ZL_HIP(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal));
  try {
    body();
  } catch (...) {
    hipStreamEndCapture(cs, &g);
    if (g) hipGraphDestroy(g);
    throw;
  }
  ZL_HIP(hipStreamEndCapture(cs, &g));
  hipGraphExec_t ex;
  ZL_HIP(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
  *def = g;
  return ex;
}

// One phase of a speculative cycle of dense models as a single graph (whole-cycle capture):
//   phase 0, the draft: reset of the cycle state, the feed pass of nFeed tokens (whose step record the host has set),
//            then for j < kk the draft distribution, the on-device draw (which writes the next draft step and the
//            target's verify row) and, but for the last draft, the next single-token draft pass;
//   phase 1, the verify: the (kk + 1)-row target pass, its distributions and the acceptance.
// The kernels are those the per-pass graphs hold, in the same order, so a captured cycle computes what the
// launch-by-launch cycle computes. Penalised samplers (whose history length is a kernel argument per draw) and hybrid
// models (whose rollback bookkeeping is host logic) take the launch-by-launch cycle.
static hipGraphExec_t cycle_graph(zl_model *T, zl_model *D, zl_sampler *s, int nFeed, int kk, int nStop, int phase) {
  const auto key = std::make_tuple(T->uid, D->uid, nFeed, kk, nStop, phase);
  {
    std::lock_guard<std::mutex> lk(g_samplers_mu);  // a model freed on another thread drops entries under this lock
    auto it = s->cycles.find(key);
    if (it != s->cycles.end()) return it->second.first;
    if (s->cycles.size() >= CYCLE_GRAPHS_MAX) drop_cycles(s, 0);
  }
  if (!s->cst) ZL_HIP(hipStreamCreateWithFlags(&s->cst, hipStreamNonBlocking));
  hipStream_t cs = s->cst;
  hipStream_t ts = T->st, dsv = D->st;
  T->st = cs;
  D->st = cs;
  struct Back { zl_model *T, *D; hipStream_t a, b; ~Back() { T->st = a; D->st = b; } } back{T, D, ts, dsv};
  const bool greedy = s->sp.temperature <= 0.0 || s->sp.greedyArgmax;
  hipGraph_t def = nullptr;
  hipGraphExec_t ex = capture_graph(cs, [&] {
    if (phase == 0) {
      hipLaunchKernelGGL(k_spec_reset, dim3(1), dim3(64), 0, cs, s->ss);
      enqueue_forward(D, nFeed, 1);
      for (int j = 0; j < kk; j++) {
        launch_dist_rows(D->logits, D->cfg.vocab, 1, D->cfg.vocab, s->sp, nullptr, j, 0, s->scratch, s->am, s->wide ? &s->ww : nullptr, &s->cw, s->qdist + j, cs);
        launch_draft_draw(s->qdist + j, s->ss, j, s->dstop, nStop, D->dstep, j == 0 ? nFeed : 1, T->dstep, s->dhist, 0, cs);
        if (j < kk - 1) enqueue_forward(D, 1, 1);
      }
    } else {
      enqueue_forward(T, kk + 1, 2);
      launch_dist_rows(T->logits, T->cfg.vocab, kk + 1, T->cfg.vocab, s->sp, nullptr, 0, 1, s->scratch, s->am, s->wide ? &s->ww : nullptr, &s->cw, s->pdist, cs);
      launch_accept(s->pdist, s->qdist, s->ss, greedy ? 1 : 0, cs);
    }
    ZL_HIP(hipGetLastError());
  }, &def);
  std::lock_guard<std::mutex> lk(g_samplers_mu);
  s->cycles[key] = {ex, def};
  return ex;
}

// ZEROLLM_CYCLE_GRAPH=0 keeps the launch-by-launch cycle (read per cycle, so a test can compare the two).
static bool use_cycle_graphs() {
  const char *e = getenv("ZEROLLM_CYCLE_GRAPH");
  return !(e && e[0] == '0');
}

static void spec_cycle(zl_model *T, zl_model *D, zl_sampler *s, const int32_t *feed, int nFeed, int pending, int kk,
                       const int32_t *stopIds, int nStop, const int32_t *hist, int nh, zl_spec_result *out) {
  ZL_REQUIRE(!T->closed && !D->closed, ZL_ERR_STATE, "model is closed");
  ZL_REQUIRE(T->cfg.vocab == D->cfg.vocab, ZL_ERR_ARG, "draft vocabulary differs from the target's");
  ZL_REQUIRE(kk >= 0 && kk <= 63 && kk + 1 <= T->logitsBatch && kk + 1 <= T->maxBatch, ZL_ERR_BATCH, "kk + 1 exceeds the target's verify limit");
  ZL_REQUIRE(nStop >= 0 && nStop <= 64, ZL_ERR_ARG, "at most 64 stop ids");
  ZL_REQUIRE(pending >= 0 && pending < T->cfg.vocab, ZL_ERR_TOKEN, "token id " + std::to_string(pending) + " out of range");
  ZL_REQUIRE((int)T->tokens.size() + kk + 1 <= T->ctx, ZL_ERR_CONTEXT, "context full (" + std::to_string(T->ctx) + " tokens)");
  if (kk > 0) {
    ZL_REQUIRE(nFeed >= 1, ZL_ERR_ARG, "the draft must be fed at least the pending token");
    ZL_REQUIRE((int)D->tokens.size() + nFeed + kk - 1 <= D->ctx, ZL_ERR_CONTEXT, "context full (" + std::to_string(D->ctx) + " tokens)");
    for (int i = 0; i < nFeed; i++) ZL_REQUIRE(feed[i] >= 0 && feed[i] < D->cfg.vocab, ZL_ERR_TOKEN, "token id " + std::to_string(feed[i]) + " out of range");
  }
  ensure_scratch(s, T->cfg.vocab);
  // everything runs on the target's stream, in order
  hipStream_t st = T->st;
  stream_wait(st, D->st);
  stream_wait(st, s->st);
  hipStream_t dst = D->st;
  D->st = st;  // draft graphs launch on this stream for the cycle (graphs do not bind a stream)
  struct Restore { zl_model *D; hipStream_t s; ~Restore() { D->st = s; } } restore{D, dst};
  hipEvent_t e0, e1, em;
  ZL_HIP(hipEventCreate(&e0));
  ZL_HIP(hipEventCreate(&e1));
  ZL_HIP(hipEventCreate(&em));
  struct EvFree { hipEvent_t a, b, c; ~EvFree() { hipEventDestroy(a); hipEventDestroy(b); hipEventDestroy(c); } } evf{e0, e1, em};
  ZL_HIP(hipEventRecord(e0, st));
  // target verify step: [pending, x_1..x_kk] at the target's position; drafts are written by the draws
  {
    Step h;
    memset(&h, 0, sizeof(h));
    h.pos0 = (int)T->tokens.size(); h.B = kk + 1; h.tokens[0] = pending;
    hipLaunchKernelGGL(k_set_step, dim3(1), dim3(64), 0, st, T->dstep, h);
  }
  const bool whole = use_graphs() && use_cycle_graphs() && kk > 0 && !T->hybrid && !D->hybrid && !s->sp.penalized &&
                     nFeed <= D->maxBatch;
  if (!whole) hipLaunchKernelGGL(k_spec_reset, dim3(1), dim3(64), 0, st, s->ss);  // (the captured cycle resets it)
  const int keep = upload_hist(s, st, hist, nh);
  {
    StopArgs sa;
    sa.n = nStop;
    for (int i = 0; i < nStop; i++) sa.ids[i] = stopIds[i];
    if (nStop) hipLaunchKernelGGL(k_set_stop, dim3(1), dim3(64), 0, st, s->dstop, sa);
  }
  ZL_HIP(hipGetLastError());
  const int *dh = s->sp.penalized ? s->dhist : nullptr;
  int posF = 0;  // the draft's position after feeding
  if (whole) {
    // whole-cycle capture: the host sets the draft's feed step, then two graph launches run the cycle
    check_batch(D, feed, nFeed, 1);
    set_step(D, (int)D->tokens.size(), feed, nFeed);
    for (int i = 0; i < nFeed; i++) D->tokens.push_back(feed[i]);
    ZL_HIP(hipGraphLaunch(cycle_graph(T, D, s, nFeed, kk, nStop, 0), st));
    ZL_HIP(hipEventRecord(em, st));
    ZL_HIP(hipGraphLaunch(cycle_graph(T, D, s, nFeed, kk, nStop, 1), st));
  } else if (kk > 0) {
    ZL_REQUIRE(!D->hybrid || (D->ck.boundary.empty() && D->ck.every == 0), ZL_ERR_UNSUPPORTED,
               "a hybrid draft with boundary-token or periodic checkpoints is driven with zl_forward, not zl_spec_cycle");
    // feedLogits (src/model/speculative.js:51-61): chunks of maxBatch, logits of the last one
    int lastChunk = 1;
    for (int i = 0; i < nFeed;) {
      int c = std::min(D->maxBatch, nFeed - i);
      bool last = i + c == nFeed;
      check_batch(D, feed + i, c, last ? 1 : 0);
      if (D->hybrid) {
        lastChunk = hybrid_batch(D, feed + i, c, last ? 1 : 0);
      } else {
        pass(D, feed + i, c, last ? 1 : 0);
        lastChunk = c;
      }
      i += c;
    }
    posF = (int)D->tokens.size();
    if (D->hybrid) mark_rollback(D);  // draft.markRollback after feedLogits (src/model/speculative.js:168)
    for (int j = 0; j < kk; j++) {
      launch_dist_rows(D->logits, D->cfg.vocab, 1, D->cfg.vocab, s->sp, dh, keep + j, 0, s->scratch, s->am, s->wide ? &s->ww : nullptr, &s->cw, s->qdist + j, st);
      launch_draft_draw(s->qdist + j, s->ss, j, s->dstop, nStop, D->dstep, j == 0 ? lastChunk : 1, T->dstep, s->dhist, keep, st);
      if (j < kk - 1) launch_pass(D, 1, 1);
    }
  }
  if (!whole) {
    ZL_HIP(hipEventRecord(em, st));
    if (T->hybrid) {  // the checkpoint policy before the verify pass (#hybridBatch: never split when all rows return logits)
      if (T->ck.wants_before((int)T->tokens.size(), pending, true, T->prevNoLogits)) checkpoint(T);
      T->prevNoLogits = false;
    }
    launch_pass(T, kk + 1, 2);
    launch_dist_rows(T->logits, T->cfg.vocab, kk + 1, T->cfg.vocab, s->sp, dh, keep, 1, s->scratch, s->am, s->wide ? &s->ww : nullptr, &s->cw, s->pdist, st);
    launch_accept(s->pdist, s->qdist, s->ss, (s->sp.temperature <= 0.0 || s->sp.greedyArgmax) ? 1 : 0, st);
  }
  ZL_HIP(hipEventRecord(e1, st));
  ZL_HIP(hipMemcpyAsync(s->hss, s->ss, sizeof(SpecState), hipMemcpyDeviceToHost, st));
  ZL_HIP(hipStreamSynchronize(st));
  const SpecState &r = *s->hss;
  const int kkA = kk > 0 ? r.kk : 0;
  out->kk = kkA;
  out->accepted = r.a;
  out->token = r.tok;
  for (int j = 0; j < kkA; j++) out->drafted[j] = r.drafted[j];
  float ms = 0, md = 0;
  ZL_HIP(hipEventElapsedTime(&ms, e0, e1));
  ZL_HIP(hipEventElapsedTime(&md, e0, em));
  out->ms_total = ms;
  out->ms_draft = md;
  // bookkeeping as the reference's calls leave it: the draft processed x_1..x_{kk-1} (the last draft is not fed,
  // nor anything after a stop token); the target processed [pending, x_1..x_kk]
  for (int j = 0; j + 1 < kkA; j++) D->tokens.push_back(r.drafted[j]);
  T->tokens.push_back(pending);
  for (int j = 0; j < kkA; j++) T->tokens.push_back(r.drafted[j]);
  if (D->hybrid && kk > 0 && kkA < kk) {
    // a stop token ended the drafts early, but the captured draft passes ran kk - 1 times: the recurrent state went past
    // what the reference feeds, so it is rebuilt from the rollback snapshot taken after feeding (a replay of
    // x_1 .. x_{kkA-1}), as the reference's state stands
    std::vector<int32_t> tail(D->tokens.begin() + posF, D->tokens.end());
    restore_state(D, posF);
    D->tokens.resize(posF);
    for (size_t i = 0; i < tail.size(); i += D->maxBatch)
      hybrid_batch(D, tail.data() + i, (int)std::min<size_t>(D->maxBatch, tail.size() - i), 0);
    D->prevNoLogits = false;
  }
}

// ---------------------------------------------------------------------------------------------- static work space
// The work space of zl_mat_gemv_noalloc, for callers that cannot allocate device memory: the quantised activation
// rows (int8 values, scales, sums, the per-block records and the f32 copy that float weights read) and the split-K
// partial sums and arrival counters of one GEMV. One array per GPU, held until the process ends; every call on a GPU
// shares it and leaves its contents behind, so calls that overlap on one GPU race.
constexpr int NOALLOC_MAX_M = 16;        // tokens per call
constexpr int NOALLOC_MAX_K = 16384;     // values per row
constexpr size_t NOALLOC_PART_DOUBLES = 786432;  // 6 MiB of split-K partial sums
constexpr size_t al256(size_t n) { return (n + 255) / 256 * 256; }
constexpr size_t NOALLOC_BLOCKS = (size_t)NOALLOC_MAX_M * (NOALLOC_MAX_K / 32);
constexpr size_t NOALLOC_OFF_Q = 0;
constexpr size_t NOALLOC_OFF_F = NOALLOC_OFF_Q + al256((size_t)NOALLOC_MAX_M * NOALLOC_MAX_K);
constexpr size_t NOALLOC_OFF_D = NOALLOC_OFF_F + al256((size_t)NOALLOC_MAX_M * NOALLOC_MAX_K * 4);
constexpr size_t NOALLOC_OFF_S = NOALLOC_OFF_D + al256(NOALLOC_BLOCKS * 4);
constexpr size_t NOALLOC_OFF_RA = NOALLOC_OFF_S + al256(NOALLOC_BLOCKS * 4);
constexpr size_t NOALLOC_OFF_RB = NOALLOC_OFF_RA + al256(NOALLOC_BLOCKS * sizeof(RecA));
constexpr size_t NOALLOC_OFF_RC = NOALLOC_OFF_RB + al256(NOALLOC_BLOCKS * sizeof(RecB));
constexpr size_t NOALLOC_OFF_PART = NOALLOC_OFF_RC + al256(NOALLOC_BLOCKS * sizeof(RecC));
constexpr size_t NOALLOC_OFF_CNT = NOALLOC_OFF_PART + al256(NOALLOC_PART_DOUBLES * 8);
constexpr size_t NOALLOC_BYTES = NOALLOC_OFF_CNT + al256((size_t)GEMV_CNT_TILES * 4);
static_assert(NOALLOC_BYTES <= (8u << 20), "the static work space stays within 8 MiB");

static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

// Device address of `scratch` on each GPU (the host-side name is not a device address: host code uses these).
constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static unsigned char *g_scratch[NOALLOC_MAX_DEVICES];

// Set-up, once per GPU with that GPU current: look up the array's address and clear the arrival counters (each
// split-K launch's last workgroup resets its own counters, so they stay zero between calls).
static unsigned char *noalloc_scratch() {
  int dev = -1;
  ZL_HIP(hipGetDevice(&dev));
  ZL_REQUIRE(dev >= 0 && dev < NOALLOC_MAX_DEVICES, ZL_ERR_UNSUPPORTED, "static work space: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    ZL_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    ZL_REQUIRE(p != nullptr, ZL_ERR_HIP, "static work space: no device address");
    unsigned char *b = (unsigned char *)p;
    launch_fill((float *)(b + NOALLOC_OFF_CNT), GEMV_CNT_TILES, 0.0f, nullptr);  // 0.0f is all-zero bits
    ZL_HIP(hipStreamSynchronize(nullptr));
    g_scratch[dev] = b;
  }
  return g_scratch[dev];
}

// zl_mat_gemv on device rows with the static work space: the same kernels (activation quantisation, then the GEMV
// dispatch of launch_gemv) as zl_mat_gemv, so the results are the same bits.
static void mat_gemv_noalloc(zl_mat *m, const float *x, int M, float *y, hipStream_t st) {
  const DevMat &mm = m->copies[0];
  ZL_REQUIRE(M >= 1 && M <= NOALLOC_MAX_M && mm.cols <= NOALLOC_MAX_K, ZL_ERR_ARG,
             "zl_mat_gemv_noalloc: at most " + std::to_string(NOALLOC_MAX_M) + " tokens of at most " +
                 std::to_string(NOALLOC_MAX_K) + " values (asked for " + std::to_string(M) + " of " +
                 std::to_string(mm.cols) + ")");
  unsigned char *b = noalloc_scratch();
  const int ld = pad64(mm.cols);
  Act act{};
  act.ld = ld;
  act.q = (int8_t *)(b + NOALLOC_OFF_Q);
  act.f = (float *)(b + NOALLOC_OFF_F);
  act.d = (float *)(b + NOALLOC_OFF_D);
  act.s = (int32_t *)(b + NOALLOC_OFF_S);
  act.ra = (RecA *)(b + NOALLOC_OFF_RA);
  act.rb = (RecB *)(b + NOALLOC_OFF_RB);
  act.rc = (RecC *)(b + NOALLOC_OFF_RC);
  GemvWork gw;
  gw.part = (double *)(b + NOALLOC_OFF_PART);
  gw.cnt = (uint32_t *)(b + NOALLOC_OFF_CNT);
  const SegSpec seg{&mm, y, mm.rows, nullptr};
  GemvArgs a = gemv_args(&seg, 1, M, EPI_STORE, act, gw);
  ZL_REQUIRE(a.ks == 1 || (a.ntiles <= GEMV_CNT_TILES && (size_t)gemv_part_need(a) <= NOALLOC_PART_DOUBLES),
             ZL_ERR_ARG, "zl_mat_gemv_noalloc: this matrix's split-K partial sums exceed the static work space");
  if (use_rg() && M == 1 && mm.type == T_Q8_0 && mm.nslab <= 48) {  // the probe's single-token path (no quantisation pass)
    a.xf = x; a.ldxf = mm.cols; a.xrow0 = 0; a.n = mm.cols; a.nw = nullptr; a.eps = 0.0;
    launch_gemv_rg(a, EPI_STORE, st);
    return;
  }
  launch_norm_quant(x, mm.cols, 0, M, nullptr, 0.0, mm.cols, ld, act, st);
  launch_gemv(a, EPI_STORE, act.f, act.ld, st);
}

}  // namespace zl

// ================================================================================================ C ABI
using namespace zl;

#define ZL_API_BEGIN try {
#define ZL_API_END                              \
  g_err.clear();                                \
  return ZL_OK;                                 \
  }                                             \
  catch (const zl::Error &e) {                  \
    g_err = e.what();                           \
    return e.code;                              \
  }                                             \
  catch (const std::exception &e) {             \
    g_err = e.what();                           \
    return ZL_ERR_HIP;                          \
  }

extern "C" {

const char *zl_last_error(void) { return g_err.c_str(); }

int zl_init(int device) {
  ZL_API_BEGIN
  int n = 0;
  ZL_HIP(hipGetDeviceCount(&n));
  ZL_REQUIRE(device >= 0 && device < n, ZL_ERR_ARG, "no such GPU: " + std::to_string(device));
  ZL_HIP(hipSetDevice(device));
  g_device = device;
  noalloc_scratch();
  ZL_API_END
}

int zl_device_query(zl_device_info *out) {
  ZL_API_BEGIN
  ensure_init();
  hipDeviceProp_t p;
  ZL_HIP(hipGetDeviceProperties(&p, g_device));
  memset(out, 0, sizeof(*out));
  snprintf(out->name, sizeof(out->name), "%s", p.gcnArchName);
  out->compute_units = p.multiProcessorCount;
  out->hbm_bytes = (int64_t)p.totalGlobalMem;
  out->lds_per_block = (int)p.sharedMemPerBlock;
  out->clock_khz = p.clockRate;
  out->mem_clock_khz = p.memoryClockRate;
  out->mem_bus_width = p.memoryBusWidth;
  ZL_API_END
}

int zl_model_load(const char *path, const zl_model_opts *opts, zl_model **out) {
  ZL_API_BEGIN
  ZL_REQUIRE(path && out, ZL_ERR_ARG, "null argument");
  ensure_init();
  *out = load_gguf(path, opts);
  ZL_API_END
}

int zl_model_synth(const zl_config *cfg, const zl_synth_tensor *tensors, int n, const zl_model_opts *opts, zl_model **out) {
  ZL_API_BEGIN
  ZL_REQUIRE(cfg && tensors && out && n > 0, ZL_ERR_ARG, "null argument");
  ensure_init();
  *out = build_synth(cfg, tensors, n, opts);
  ZL_API_END
}

int zl_model_config(const zl_model *m, zl_config *out) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && out, ZL_ERR_ARG, "null argument");
  *out = m->cfg;
  ZL_API_END
}

int zl_model_info_get(const zl_model *m, zl_model_info *out) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && out, ZL_ERR_ARG, "null argument");
  out->ctx = m->ctx; out->max_batch = m->maxBatch; out->logits_batch = m->logitsBatch; out->kv_f16 = m->kvF16;
  out->weight_bytes = m->weightBytes; out->device_bytes = m->ar.bytes;
  out->state_bytes = m->hybrid ? (int64_t)state_bytes(m) : 0;
  out->state_capture_slots = m->capture ? m->capSlots : 0;
  ZL_API_END
}

int zl_model_free(zl_model *m) {
  ZL_API_BEGIN
  delete m;
  ZL_API_END
}

int zl_forward(zl_model *m, const int32_t *tokens, int n, int logits_mode, float *host_logits) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && tokens, ZL_ERR_ARG, "null argument");
  ZL_REQUIRE(logits_mode >= 0 && logits_mode <= 2, ZL_ERR_ARG, "logits_mode must be 0, 1 or 2");
  forward(m, tokens, n, logits_mode);
  if (host_logits && logits_mode) {
    size_t rows = logits_mode == 2 ? (size_t)n : 1;
    ZL_HIP(hipMemcpyAsync(host_logits, m->logits, rows * m->cfg.vocab * 4, hipMemcpyDeviceToHost, m->st));
  }
  if (host_logits) ZL_HIP(hipStreamSynchronize(m->st));
  ZL_API_END
}

int zl_model_logits(const zl_model *m, int row0, int nrows, float *host_out) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && host_out, ZL_ERR_ARG, "null argument");
  ZL_REQUIRE(row0 >= 0 && nrows >= 0 && row0 + nrows <= m->logitsBatch, ZL_ERR_ARG, "logits rows out of range");
  ZL_HIP(hipMemcpyAsync(host_out, m->logits + (size_t)row0 * m->cfg.vocab, (size_t)nrows * m->cfg.vocab * 4, hipMemcpyDeviceToHost, m->st));
  ZL_HIP(hipStreamSynchronize(m->st));
  ZL_API_END
}

int zl_truncate(zl_model *m, int n, int *replayed) {
  ZL_API_BEGIN
  ZL_REQUIRE(m, ZL_ERR_ARG, "null argument");
  const int r = truncate_model(m, n);
  if (replayed) *replayed = r;
  ZL_API_END
}

int zl_truncate_plan(const zl_model *m, int n, int *from, int *replay) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && from && replay, ZL_ERR_ARG, "null argument");
  const int pos = (int)m->tokens.size();
  if (m->hybrid) m->ck.plan(std::max(n, 0), pos, from, replay);
  else { *from = std::min(std::max(n, 0), pos); *replay = 0; }
  ZL_API_END
}

int zl_mark_rollback(zl_model *m) {
  ZL_API_BEGIN
  ZL_REQUIRE(m, ZL_ERR_ARG, "null argument");
  if (m->hybrid && !m->closed) mark_rollback(m);
  ZL_API_END
}

int zl_reset(zl_model *m) {
  ZL_API_BEGIN
  ZL_REQUIRE(m, ZL_ERR_ARG, "null argument");
  reset_model(m);
  ZL_API_END
}

int zl_model_checkpoints(const zl_model *m, int32_t *pos, int cap) {
  if (!m) return -1;
  const int n = (int)m->ck.list.size();
  for (int i = 0; i < n && i < cap; i++) pos[i] = m->ck.list[i].pos;
  return n;
}

// The live recurrent state in the reference's layout (RecurrentState, src/model/recurrent-state.js:8-37): conv
// [layer][channel][kernel-1] (q/k channels of key head h from value head h's copy), ssm [layer][vHead][dv][dk].
int zl_model_recurrent_state(zl_model *m, float *conv, float *ssm) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && m->hybrid, ZL_ERR_ARG, "not a hybrid model");
  const zl_config &c = m->cfg;
  const int D = c.ssm_d_state, nK = c.ssm_n_group, nV = c.ssm_dt_rank, M = c.ssm_conv_kernel - 1;
  const long convDim = 2L * nK * D + (long)nV * D;
  std::vector<float> h((size_t)m->nRec * (m->convFloats + m->ssmFloats));
  ZL_HIP(hipMemcpyAsync(h.data(), m->state, h.size() * 4, hipMemcpyDeviceToHost, m->st));
  ZL_HIP(hipStreamSynchronize(m->st));
  for (int r = 0; r < m->nRec; r++) {
    const float *w = h.data() + (size_t)r * m->convFloats;
    float *o = conv ? conv + (size_t)r * convDim * M : nullptr;
    if (o)
      for (long ch = 0; ch < convDim; ch++) {
        int hv, grp, i;
        if (ch < 2L * nK * D) { grp = (int)(ch / ((long)nK * D)); const int r2 = (int)(ch % ((long)nK * D)); hv = r2 / D; i = r2 % D; }
        else { grp = 2; hv = (int)((ch - 2L * nK * D) / D); i = (int)((ch - 2L * nK * D) % D); }
        for (int t = 0; t < M; t++) o[ch * M + t] = w[(((long)hv * 3 + grp) * D + i) * M + t];
      }
  }
  if (ssm) memcpy(ssm, h.data() + (size_t)m->nRec * m->convFloats, (size_t)m->nRec * m->ssmFloats * 4);
  ZL_API_END
}

int zl_model_pos(const zl_model *m) { return m ? (int)m->tokens.size() : -1; }

int zl_model_tokens(const zl_model *m, int32_t *out, int cap) {
  if (!m) return -1;
  int n = (int)m->tokens.size();
  for (int i = 0; i < n && i < cap; i++) out[i] = m->tokens[i];
  return n;
}

int zl_synth_tensor_bytes(const zl_synth_tensor *t, int use_device, void *host_out) {
  ZL_API_BEGIN
  ZL_REQUIRE(t && host_out, ZL_ERR_ARG, "null argument");
  if (t->fill == 1) {
    for (int64_t i = 0; i < t->rows * t->cols; i++) ((float *)host_out)[i] = t->fill_value;
    return ZL_OK;
  }
  if (t->fill == 3) {
    for (int64_t i = 0; i < t->rows * t->cols; i++) ((float *)host_out)[i] = i < t->src_cols ? t->fill_value : (float)t->std;
    return ZL_OK;
  }
  ZL_REQUIRE(t->fill == 0 || (t->fill == 2 && t->type == T_F32), ZL_ERR_ARG, "fill 2 (offset normal values) needs type F32");
  const int bv = zl_synth::block_values(t->type), bb = zl_synth::block_bytes(t->type);
  ZL_REQUIRE(bv > 0 && t->cols % bv == 0, ZL_ERR_UNSUPPORTED, "unsupported synthetic tensor type/shape");
  const int64_t nbr = t->cols / bv;
  const size_t bytes = (size_t)(t->rows * nbr) * bb;
  const uint64_t src = (uint64_t)(t->src_cols > 0 ? t->src_cols : t->cols);
  if (use_device) {
    ensure_init();
    uint8_t *d = nullptr;
    ZL_HIP(hipMalloc(&d, bytes));
    struct F { uint8_t *d; ~F() { hipFree(d); } } fr{d};
    launch_synth(t->type, t->seed, t->std, src, (uint64_t)t->col0, (int)t->rows, (int)t->cols, d, nullptr);
    ZL_HIP(hipMemcpy(host_out, d, bytes, hipMemcpyDeviceToHost));
  } else {
    uint8_t *o = (uint8_t *)host_out;
    const int64_t total = t->rows * nbr;
    int nt = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (total < 4096) nt = 1;
    std::vector<std::thread> th;
    for (int w = 0; w < nt; w++) {
      th.emplace_back([=]() {
        for (int64_t i = total * w / nt; i < total * (w + 1) / nt; i++)
          zl_synth::synth_block(t->type, t->seed, t->std, src, (uint64_t)t->col0, (uint64_t)(i / nbr), (uint64_t)(i % nbr), o + i * bb);
      });
    }
    for (auto &x : th) x.join();
  }
  if (t->fill == 2)
    for (int64_t i = 0; i < t->rows * t->cols; i++) ((float *)host_out)[i] = (float)((double)t->fill_value + (double)((float *)host_out)[i]);
  ZL_API_END
}

int zl_sampler_create(const zl_sampler_opts *opts, zl_sampler **out) {
  ZL_API_BEGIN
  ZL_REQUIRE(opts && out, ZL_ERR_ARG, "null argument");
  /* options the device sampler does not take are refused before any device call: a history window above 64 ids */
  ZL_REQUIRE(opts->repeat_last_n >= 0 && opts->repeat_last_n <= 64, ZL_ERR_UNSUPPORTED,
             "repeat_last_n must be 0..64 on the GPU sampler");
  ensure_init();
  *out = new_sampler(opts);
  std::lock_guard<std::mutex> lk(g_samplers_mu);
  g_samplers.insert(*out);
  ZL_API_END
}

int zl_sampler_cycle_graphs(zl_sampler *s, int *n) {
  ZL_API_BEGIN
  ZL_REQUIRE(s && n, ZL_ERR_ARG, "null argument");
  std::lock_guard<std::mutex> lk(g_samplers_mu);
  *n = (int)s->cycles.size();
  ZL_API_END
}

int zl_sampler_free(zl_sampler *s) {
  ZL_API_BEGIN
  delete s;
  ZL_API_END
}

int zl_sampler_get_rng(zl_sampler *s, uint32_t *state) {
  ZL_API_BEGIN
  ZL_REQUIRE(s && state, ZL_ERR_ARG, "null argument");
  ZL_HIP(hipDeviceSynchronize());
  ZL_HIP(hipMemcpy(state, &s->ss->rng, 4, hipMemcpyDeviceToHost));
  ZL_API_END
}

int zl_sampler_set_rng(zl_sampler *s, uint32_t state) {
  ZL_API_BEGIN
  ZL_REQUIRE(s, ZL_ERR_ARG, "null argument");
  ZL_HIP(hipDeviceSynchronize());
  hipLaunchKernelGGL(k_set_rng, dim3(1), dim3(64), 0, s->st, s->ss, state);
  ZL_HIP(hipStreamSynchronize(s->st));
  ZL_API_END
}

int zl_sample(zl_sampler *s, zl_model *m, int row, const int32_t *hist, int n_hist, int32_t *token) {
  ZL_API_BEGIN
  ZL_REQUIRE(s && m && token, ZL_ERR_ARG, "null argument");
  stream_wait(m->st, s->st);
  dist_of_row(s, m, row, hist, n_hist, s->tmpdist);
  launch_draw_one(s->tmpdist, &s->ss->rng, s->dtok, m->st);
  ZL_HIP(hipMemcpyAsync(s->htok, s->dtok, 4, hipMemcpyDeviceToHost, m->st));
  ZL_HIP(hipStreamSynchronize(m->st));
  *token = s->htok[0];
  ZL_API_END
}

int zl_distribution(zl_sampler *s, zl_model *m, int row, const int32_t *hist, int n_hist, int32_t *ids, double *probs,
                    int cap, int *n, double *total, int *greedy) {
  ZL_API_BEGIN
  ZL_REQUIRE(s && m && ids && probs && n && total && greedy, ZL_ERR_ARG, "null argument");
  stream_wait(m->st, s->st);
  dist_of_row(s, m, row, hist, n_hist, s->tmpdist);
  ZL_HIP(hipMemcpyAsync(s->hdist, s->tmpdist, sizeof(DevDist), hipMemcpyDeviceToHost, m->st));
  ZL_HIP(hipStreamSynchronize(m->st));
  const DevDist &d = *s->hdist;
  ZL_REQUIRE(d.n <= cap, ZL_ERR_ARG, "distribution capacity too small");
  if (d.wids) {  // a full list: its kept entries from the list's own storage
    ZL_HIP(hipMemcpy(ids, d.wids, sizeof(int32_t) * d.n, hipMemcpyDeviceToHost));
    ZL_HIP(hipMemcpy(probs, d.wprobs, sizeof(double) * d.n, hipMemcpyDeviceToHost));
  } else {
    for (int i = 0; i < d.n; i++) { ids[i] = d.ids[i]; probs[i] = d.probs[i]; }
  }
  *n = d.n; *total = d.total; *greedy = d.greedy;
  ZL_API_END
}

int zl_spec_cycle(zl_model *target, zl_model *draft, zl_sampler *s, const int32_t *feed, int n_feed, int32_t pending, int kk,
                  const int32_t *stop_ids, int n_stop, const int32_t *hist, int n_hist, zl_spec_result *out) {
  ZL_API_BEGIN
  ZL_REQUIRE(target && draft && s && out, ZL_ERR_ARG, "null argument");
  spec_cycle(target, draft, s, feed, n_feed, pending, kk, stop_ids, n_stop, hist, n_hist, out);
  ZL_API_END
}

// ---- kernel probes
int zl_mat_upload(int type, const void *raw, int64_t rows, int64_t cols, zl_mat **out) {
  ZL_API_BEGIN
  ZL_REQUIRE(raw && out && rows > 0 && cols > 0, ZL_ERR_ARG, "bad argument");
  ensure_init();
  int64_t rb = ggml_row_bytes(type, cols);
  ZL_REQUIRE(rb > 0, ZL_ERR_UNSUPPORTED, "unsupported type/shape");
  std::unique_ptr<zl_mat> m(new zl_mat());
  ZL_HIP(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
  uint8_t *d = nullptr;
  ZL_HIP(hipMalloc(&d, (size_t)rb * rows));
  struct F { uint8_t *d; ~F() { hipFree(d); } } fr{d};
  ZL_HIP(hipMemcpy(d, raw, (size_t)rb * rows, hipMemcpyHostToDevice));
  m->copies.push_back(make_mat(m->ar, type, (int)rows, (int)cols, d, m->st));
  ZL_HIP(hipStreamSynchronize(m->st));
  *out = m.release();
  ZL_API_END
}

int zl_mat_synth(int type, int64_t rows, int64_t cols, uint64_t seed, double stdv, int copies, zl_mat **out) {
  ZL_API_BEGIN
  ZL_REQUIRE(out && rows > 0 && cols > 0 && copies >= 1, ZL_ERR_ARG, "bad argument");
  ensure_init();
  int64_t rb = ggml_row_bytes(type, cols);
  ZL_REQUIRE(rb > 0 && zl_synth::block_values(type) > 0, ZL_ERR_UNSUPPORTED, "unsupported type/shape");
  std::unique_ptr<zl_mat> m(new zl_mat());
  ZL_HIP(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
  uint8_t *d = nullptr;
  ZL_HIP(hipMalloc(&d, (size_t)rb * rows));
  struct F { uint8_t *d; ~F() { hipFree(d); } } fr{d};
  for (int c = 0; c < copies; c++) {
    launch_synth(type, seed + (uint64_t)c * 0x9E3779B97F4A7C15ull, stdv, (uint64_t)cols, 0, (int)rows, (int)cols, d, m->st);
    m->copies.push_back(make_mat(m->ar, type, (int)rows, (int)cols, d, m->st));
    ZL_HIP(hipStreamSynchronize(m->st));
  }
  *out = m.release();
  ZL_API_END
}

int zl_mat_free(zl_mat *m) {
  ZL_API_BEGIN
  delete m;
  ZL_API_END
}

int zl_mat_dequant(zl_mat *m, int64_t row0, int64_t nrows, float *out) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && out && row0 >= 0 && nrows > 0 && row0 + nrows <= m->copies[0].rows, ZL_ERR_ARG, "bad argument");
  const DevMat &mm = m->copies[0];
  std::vector<int> ids(nrows);
  for (int64_t i = 0; i < nrows; i++) ids[i] = (int)(row0 + i);
  int *dids = nullptr;
  float *dout = nullptr;
  ZL_HIP(hipMalloc(&dids, nrows * 4));
  ZL_HIP(hipMalloc(&dout, (size_t)nrows * mm.nslab * 64 * 4));
  struct F { int *a; float *b; ~F() { hipFree(a); hipFree(b); } } fr{dids, dout};
  ZL_HIP(hipMemcpy(dids, ids.data(), nrows * 4, hipMemcpyHostToDevice));
  launch_dequant_rows(view(mm), dids, (int)nrows, dout, mm.cols, m->st);
  ZL_HIP(hipStreamSynchronize(m->st));
  ZL_HIP(hipMemcpy(out, dout, (size_t)nrows * mm.cols * 4, hipMemcpyDeviceToHost));
  ZL_API_END
}

// activations for probes: quantise M rows of x (host) on the device
struct ProbeAct {
  Arena ar;
  Act act{};
  GemvWork gw{};
  float *x = nullptr;
};
static void probe_act(ProbeAct &pa, const float *x, int64_t K, int M, hipStream_t st) {
  const int ld = pad64((int)K);
  pa.act = alloc_act(pa.ar, M, ld, true);
  pa.gw = alloc_gemv_work(pa.ar);
  pa.x = (float *)pa.ar.alloc((size_t)M * K * 4);
  if (x) ZL_HIP(hipMemcpy(pa.x, x, (size_t)M * K * 4, hipMemcpyHostToDevice));
  else launch_fill(pa.x, (long)M * K, 0.5f, st);
  launch_norm_quant(pa.x, (int)K, 0, M, nullptr, 0.0, (int)K, ld, pa.act, st);
}

// A probe GEMV of M rows x (f32, stride = cols; quantised into act) as the model's passes run it: a single-token Q8_0
// launch takes the 16-row-group kernel on the f32 rows, everything else the tile kernels on act.
static void launch_probe_gemv(const DevMat &mm, const float *x, const Act &act, const GemvWork &gw, int M, float *y,
                              hipStream_t st) {
  GemvArgs a = gemv_args({{&mm, y, mm.rows, nullptr}}, M, EPI_STORE, act, gw);
  if (rg_path({&mm}, M)) {
    a.xf = x; a.ldxf = mm.cols; a.xrow0 = 0; a.n = mm.cols; a.nw = nullptr; a.eps = 0.0;
    launch_gemv_rg(a, EPI_STORE, st);
    return;
  }
  launch_gemv(a, EPI_STORE, act.f, act.ld, st);
}
static void probe_gemv(const DevMat &mm, const ProbeAct &pa, int M, float *y, hipStream_t st) {
  launch_probe_gemv(mm, pa.x, pa.act, pa.gw, M, y, st);
}

int zl_mat_gemv(zl_mat *m, const float *x, int M, float *y) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && x && y && M >= 1 && M <= 64, ZL_ERR_ARG, "bad argument");
  const DevMat &mm = m->copies[0];
  ProbeAct pa;
  struct R { ProbeAct *p; ~R() { p->ar.release(); } } rel{&pa};
  probe_act(pa, x, mm.cols, M, m->st);
  float *dy = (float *)pa.ar.alloc((size_t)M * mm.rows * 4);
  probe_gemv(mm, pa, M, dy, m->st);
  ZL_HIP(hipStreamSynchronize(m->st));
  ZL_HIP(hipMemcpy(y, dy, (size_t)M * mm.rows * 4, hipMemcpyDeviceToHost));
  ZL_API_END
}

int zl_mat_gemv_time(zl_mat *m, int M, int iters, float *ms_per_call) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && ms_per_call && M >= 1 && M <= 64 && iters >= 1, ZL_ERR_ARG, "bad argument");
  const DevMat &m0 = m->copies[0];
  ProbeAct pa;
  struct R { ProbeAct *p; ~R() { p->ar.release(); } } rel{&pa};
  probe_act(pa, nullptr, m0.cols, M, m->st);
  float *dy = (float *)pa.ar.alloc((size_t)M * m0.rows * 4);
  const int nc = (int)m->copies.size();
  for (int i = 0; i < nc; i++) probe_gemv(m->copies[i], pa, M, dy, m->st);  // warm-up (outside capture)
  const float ms = time_graph(m->st, iters, [&](int i) { probe_gemv(m->copies[i % nc], pa, M, dy, m->st); });
  *ms_per_call = ms;
  ZL_API_END
}

int zl_mat_gemv_noalloc(zl_mat *m, const float *x, int M, float *y, void *stream) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && x && y, ZL_ERR_ARG, "bad argument");
  hipStream_t st = stream ? (hipStream_t)stream : m->st;
  mat_gemv_noalloc(m, x, M, y, st);
  if (!stream) ZL_HIP(hipStreamSynchronize(st));
  ZL_API_END
}

int zl_quant_act(const float *x, int64_t K, int M, int8_t *q, float *d, int32_t *s) {
  ZL_API_BEGIN
  ZL_REQUIRE(x && q && d && s && K > 0 && K % 32 == 0 && M >= 1, ZL_ERR_ARG, "bad argument");
  ensure_init();
  hipStream_t st;
  ZL_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  struct S { hipStream_t s; ~S() { hipStreamDestroy(s); } } ss{st};
  ProbeAct pa;
  struct R { ProbeAct *p; ~R() { p->ar.release(); } } rel{&pa};
  probe_act(pa, x, K, M, st);
  ZL_HIP(hipStreamSynchronize(st));
  const int ld = pa.act.ld;
  for (int t = 0; t < M; t++) {
    ZL_HIP(hipMemcpy(q + t * K, pa.act.q + (size_t)t * ld, K, hipMemcpyDeviceToHost));
    ZL_HIP(hipMemcpy(d + t * (K / 32), pa.act.d + (size_t)t * (ld / 32), (K / 32) * 4, hipMemcpyDeviceToHost));
    ZL_HIP(hipMemcpy(s + t * (K / 32), pa.act.s + (size_t)t * (ld / 32), (K / 32) * 4, hipMemcpyDeviceToHost));
  }
  ZL_API_END
}

int zl_probe_gemv(zl_model *m, int which, int M, int iters, float *ms_per_launch, int64_t *bytes_per_launch) {
  ZL_API_BEGIN
  ZL_REQUIRE(m && ms_per_launch && bytes_per_launch, ZL_ERR_ARG, "null argument");
  probe_gemv(m, which, M, iters, ms_per_launch, bytes_per_launch);
  ZL_API_END
}

}  // extern "C"
