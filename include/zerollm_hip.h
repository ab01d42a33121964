/*
 * zerollm_hip — C ABI of the MI355X-native speculative-decoding step of zerollm.
 *
 * The reference (fordi-off/zerollm) is a Node.js engine whose fast path is a worker pool running WebAssembly SIMD
 * kernels; it has no FFI of its own. The functions below are the boundary a Node N-API addon (or any FFI: ctypes,
 * cgo, JNI) binds to put this library behind the reference's model interface as `--kernels hip`. Each declaration
 * names the reference interface it replaces. Plain pointers and sizes only; every call returns a status code
 * (ZL_OK = 0) and leaves a message in zl_last_error() on failure. Calls on one model are serialised by the caller,
 * as the reference's are (docs/DECISIONS.md:190-218). One GPU.
 */
#ifndef ZEROLLM_HIP_H
#define ZEROLLM_HIP_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------------- status */
#define ZL_OK 0
#define ZL_ERR_ARG 1          /* bad argument */
#define ZL_ERR_HIP 2          /* HIP runtime failure */
#define ZL_ERR_FORMAT 3       /* malformed GGUF */
#define ZL_ERR_UNSUPPORTED 4  /* architecture / tensor type / shape this library does not run */
#define ZL_ERR_STATE 5        /* model closed, or call out of order */
#define ZL_ERR_CONTEXT 6      /* "context full (N tokens)" */
#define ZL_ERR_TOKEN 7        /* "token id X out of range" */
#define ZL_ERR_BATCH 8        /* "batch of B tokens (max M)" / logitsBatch exceeded */
#define ZL_ERR_IO 9           /* file read failure */

/* Message of the last failed call on this thread (empty after a successful call). */
const char *zl_last_error(void);

/* Select and initialise the GPU. Replaces the worker pool start-up (src/compute/pool.js:33-121). */
int zl_init(int device);

typedef struct {
  char name[128];
  int compute_units;
  int64_t hbm_bytes;
  int lds_per_block;
  int clock_khz;
  int mem_clock_khz;
  int mem_bus_width;
} zl_device_info;
int zl_device_query(zl_device_info *out);

/* ---------------------------------------------------------------------------------------------- model */
typedef struct zl_model zl_model;

/* PoolModel.create options (src/compute/pool.js:27-31): ctx (0 = 2048, capped at the trained context), kv precision,
 * maxBatch (default 16, cap 64, src/compute/layout.js:23), logitsBatch (default min(maxBatch, 16), layout.js:48).
 * Hybrid (qwen35) models only, the checkpoint policy (src/model/state-checkpoints.js:18-35): max_checkpoints (0: the
 * default 6, negative: none), checkpoint_every (0: off) and the boundary token ids that get a snapshot before them
 * (<|im_start|>). */
typedef struct {
  int ctx;
  int kv_f16;
  int max_batch;
  int logits_batch;
  int max_checkpoints;
  int checkpoint_every;
  const int32_t *boundary_ids;
  int n_boundary;
} zl_model_opts;

/* ModelConfig (src/model/config.js:233-267); arch: 0 llama, 1 qwen2, 2 qwen3, 3 qwen35. The qwen35 hybrid
 * (src/model/config.js:126-156): layer l is a Gated DeltaNet layer unless (l + 1) % full_attn_interval == 0; DeltaNet
 * shape ssm.conv_kernel, ssm.state_size (key head size), ssm.group_count (key heads), ssm.time_step_rank (value heads),
 * ssm.inner_size (value heads x value head size); its attention layers project [query | gate] per head. */
typedef struct {
  int arch;
  int n_ctx_train, n_embd, n_layer, n_ff, n_head, n_head_kv, head_dim, n_rot, vocab;
  float rms_eps, rope_base;
  int neox, qk_norm, qkv_bias, tied, has_rope_freqs;
  int hybrid, full_attn_interval, ssm_conv_kernel, ssm_d_state, ssm_n_group, ssm_dt_rank, ssm_d_inner;
} zl_config;

typedef struct {
  int ctx, max_batch, logits_batch, kv_f16;
  int64_t weight_bytes;      /* quantised matrix bytes streamed by one pass (all layers + output head) */
  int64_t device_bytes;      /* HBM held by the model */
  int64_t state_bytes;       /* recurrent state of a hybrid model (each snapshot holds as much); 0 otherwise */
  int state_capture_slots;   /* hybrid: verify passes of up to this many tokens capture the state after each token,
                                and zl_truncate into such a window copies it instead of replaying (0: restore + replay) */
} zl_model_info;

/* Load a GGUF model into HBM (RefModel/PoolModel construction: src/model/forward.js:105-153,
 * src/compute/pool.js:42-121; config from metadata as modelConfig, src/model/config.js:275-325). */
int zl_model_load(const char *gguf_path, const zl_model_opts *opts, zl_model **out);
int zl_model_config(const zl_model *m, zl_config *out);
int zl_model_info_get(const zl_model *m, zl_model_info *out);
/* PoolModel.close (src/compute/pool.js:302-316); safe on NULL. */
int zl_model_free(zl_model *m);

/* PoolModel.forwardBatch (src/compute/pool.js:145-160) / forward (:135): run n tokens at positions pos..pos+n-1.
 * logits_mode 0 = none, 1 = last token, 2 = every token (row b = distribution after tokens[b]). When host_logits is
 * not NULL the logits are copied there (vocab or n*vocab floats); they also stay on the device for zl_sample. */
int zl_forward(zl_model *m, const int32_t *tokens, int n, int logits_mode, float *host_logits);
/* PoolModel.truncate (src/compute/pool.js:278-294): positional KV is bookkeeping only; a hybrid model restores the
 * nearest recurrent-state snapshot at or before n and replays the tokens in between (*replayed, may be NULL). When the
 * last pass returned every row's logits and n falls inside it, the state the pass captured after token n is copied
 * instead (the same bits); *replayed and the checkpoints are what the reference's restore + replay leaves. */
int zl_truncate(zl_model *m, int n, int *replayed);
/* PoolModel.truncatePlan (src/compute/pool.js:256): the snapshot position truncate(n) restores and the replay count. */
int zl_truncate_plan(const zl_model *m, int n, int *from, int *replay);
/* PoolModel.markRollback (src/compute/pool.js:269): the rollback snapshot of a hybrid model; no-op for KV-cache models. */
int zl_mark_rollback(zl_model *m);
/* PoolModel.checkpointPositions (src/compute/pool.js:253): the count; copies up to cap positions (ascending). */
int zl_model_checkpoints(const zl_model *m, int32_t *pos, int cap);
/* PoolModel.getRecurrentState (src/compute/pool.js:259) in the reference's layout (src/model/recurrent-state.js:8-37):
 * conv [recurrent layer][channel][conv_kernel-1], ssm [recurrent layer][value head][value dim][key dim]; either may be
 * NULL. */
int zl_model_recurrent_state(zl_model *m, float *conv, float *ssm);
/* PoolModel.reset (src/compute/pool.js:296-299). */
int zl_reset(zl_model *m);
/* PoolModel.pos / tokens (src/compute/pool.js:40, 57). zl_model_tokens returns the count, copies up to cap ids. */
int zl_model_pos(const zl_model *m);
int zl_model_tokens(const zl_model *m, int32_t *out, int cap);
/* Copy rows [row0, row0+nrows) of the device logits of the last forward to the host. */
int zl_model_logits(const zl_model *m, int row0, int nrows, float *host_out);

/* ---------------------------------------------------------------------------------------------- synthetic models */
/* One tensor of a synthetic model: values std * N(0,1) from stream `seed` (element (r, c) is deviate
 * r * src_cols + col0 + c), quantised with this library's quantisers into ggml type `type`; with fill = 1 a
 * constant F32 tensor of fill_value (norm weights); with fill = 2 an F32 tensor of fill_value + std * N(0,1); with
 * fill = 3 an F32 tensor of fill_value in its first src_cols elements and std in the rest (a two-level norm weight).
 * Mirrors the reference generators' role (tools/make-tiny-gguf.js:28-149, tools/make-synth-qwen35.js:30-60). */
typedef struct {
  const char *name;
  int type;
  int64_t rows, cols;
  uint64_t seed;
  double std;
  int64_t src_cols, col0;
  int fill;
  float fill_value;
} zl_synth_tensor;

/* Raw ggml bytes of one synthetic tensor, generated on the GPU (use_device = 1) or the CPU; identical either way. */
int zl_synth_tensor_bytes(const zl_synth_tensor *t, int use_device, void *host_out);
/* Build a model directly in HBM from synthetic tensors (names as in a GGUF: token_embd.weight, blk.N.attn_q.weight...). */
int zl_model_synth(const zl_config *cfg, const zl_synth_tensor *tensors, int n, const zl_model_opts *opts, zl_model **out);

/* ---------------------------------------------------------------------------------------------- sampler */
typedef struct zl_sampler zl_sampler;

/* createSampler options (src/sampling/sampler.js:4-15, 81-92). Any top_k: 0 (or at least the vocabulary) keeps every
 * id as a candidate, as the reference does; repeat_last_n must be 0..64. greedy_argmax = 1 makes it the plain argmax
 * sampler (src/model/generate.js:4-8). */
typedef struct {
  double temperature, top_p, min_p, repeat_penalty, presence_penalty, frequency_penalty;
  int top_k, repeat_last_n;
  uint32_t seed;
  int greedy_argmax;
} zl_sampler_opts;

int zl_sampler_create(const zl_sampler_opts *opts, zl_sampler **out);
int zl_sampler_free(zl_sampler *s);
/* mulberry32 state of the sampler's single random stream (src/util/rng.js:4-13). */
int zl_sampler_get_rng(zl_sampler *s, uint32_t *state);
int zl_sampler_set_rng(zl_sampler *s, uint32_t state);
/* Diagnostic, no counterpart in the reference: the whole-cycle graphs this sampler holds. Freeing a model drops the
 * graphs that captured it; past 64 graphs the cache starts over. */
int zl_sampler_cycle_graphs(zl_sampler *s, int *n);
/* sample(logits, history) = draw(distribution(...)) on logits row `row` of the model's last forward
 * (src/sampling/sampler.js:94-153). Only the id crosses to the host. */
int zl_sample(zl_sampler *s, zl_model *m, int row, const int32_t *hist, int n_hist, int32_t *token);
/* distribution() of that row, returned to the host (ids/probs capacity `cap`). */
int zl_distribution(zl_sampler *s, zl_model *m, int row, const int32_t *hist, int n_hist, int32_t *ids, double *probs,
                    int cap, int *n, double *total, int *greedy);

/* ---------------------------------------------------------------------------------------------- speculative step */
typedef struct {
  int kk;          /* tokens actually drafted (fewer than asked if a stop token was drafted) */
  int accepted;    /* a */
  int token;       /* correction (first rejection) or bonus token */
  int32_t drafted[64];
  float ms_total;  /* device time of the cycle */
  float ms_draft;  /* device time of the draft phase (feed + proposals); the rest is verification + acceptance */
} zl_spec_result;

/* One cycle of generateSpeculative (src/model/speculative.js:155-209) on the GPU: feed `feed` to the draft
 * (feedLogits, :51-61), draft kk tokens with on-device draws (:169-177), verify [pending, x_1..x_kk] in one target
 * pass with per-position logits (forwardRows, :39-48), then the accept / residual / bonus draws (:192-209). The
 * host keeps the loop bookkeeping (kk, emission, stop/max checks, truncation), as the reference's loop does; both
 * models' token lists are updated as the reference's calls would leave them. hist = sampler history before the
 * cycle (only its last repeat_last_n ids matter); stop_ids = ids that end drafting. */
int zl_spec_cycle(zl_model *target, zl_model *draft, zl_sampler *s, const int32_t *feed, int n_feed, int32_t pending,
                  int kk, const int32_t *stop_ids, int n_stop, const int32_t *hist, int n_hist, zl_spec_result *out);

/* ---------------------------------------------------------------------------------------------- kernel probes */
/* These expose single kernels for parity tests and the GEMV microbenchmark (tools/kbench.mjs is the reference's). */
typedef struct zl_mat zl_mat;
/* Upload raw ggml rows (rows x cols of `type`) and repack them into the device layout. */
int zl_mat_upload(int type, const void *raw, int64_t rows, int64_t cols, zl_mat **out);
/* Build `copies` distinct synthetic copies of a rows x cols matrix in HBM (for cache-cold timing). */
int zl_mat_synth(int type, int64_t rows, int64_t cols, uint64_t seed, double std, int copies, zl_mat **out);
int zl_mat_free(zl_mat *m);
/* dequantRow for rows [row0, row0+nrows) (src/compute/ref-kernels.js:80-120). */
int zl_mat_dequant(zl_mat *m, int64_t row0, int64_t nrows, float *out);
/* y[t][r] = matvec(W, Act(x[t])) for M tokens (src/compute/ref-kernels.js:127-302), copy 0. */
int zl_mat_gemv(zl_mat *m, const float *x, int M, float *y);
/* Time `iters` GEMVs with M device-resident tokens, cycling through the copies; returns mean ms per call. */
int zl_mat_gemv_time(zl_mat *m, int M, int iters, float *ms_per_call);
/* zl_mat_gemv with nothing allocated. No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). x: M x cols f32 rows and y:
 * M x rows f32, both in device memory. The activation quantisation and the split-K partial sums use one static device
 * array per GPU (under 8 MiB, held until the process ends): at most 16 tokens of at most 16384 values, and matrices
 * whose split-K partials fit 6 MiB; larger requests fail with ZL_ERR_ARG. stream: a hipStream_t to enqueue on (the
 * call returns at once; the caller synchronises), or NULL for the matrix's own stream (the call returns when y holds
 * the result). Every call on one GPU shares the array, so calls that overlap on a GPU race. Same kernels, same bits
 * as zl_mat_gemv. */
int zl_mat_gemv_noalloc(zl_mat *m, const float *x, int M, float *y, void *stream);
/* quantizeAct of M rows of length K (src/compute/ref-kernels.js:44-62). */
int zl_quant_act(const float *x, int64_t K, int M, int8_t *q, float *d, int32_t *s);

/* ---------------------------------------------------------------------------------------------- timing probe */
/* Mean duration of `iters` back-to-back launches of one GEMV of the forward pass (which: 0 first q/k/v group, 1 wo,
 * 2 gate+up, 3 down, 4 output head) with M tokens, cycling through the layers' weights, timed with HIP events on the
 * model's stream; also the weight bytes one launch streams. The GEMV kernel alone is timed: where the pass quantises
 * the input rows in a k_norm_quant launch first, that launch runs once before the timed ones. Measurement aid (the reference times its kernels with
 * tools/kbench.mjs). */
int zl_probe_gemv(zl_model *m, int which, int M, int iters, float *ms_per_launch, int64_t *bytes_per_launch);

#ifdef __cplusplus
}
#endif
#endif
