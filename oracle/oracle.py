"""ORACLE — test infrastructure only (used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg).

ctypes wrapper of liboracle.so, the C restatement of zerollm's plain-JS reference path (oracle/zl_oracle.c). The
product (zerollm_amd/) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

F32P = C.POINTER(C.c_float)
F64P = C.POINTER(C.c_double)
I32P = C.POINTER(C.c_int32)
I8P = C.POINTER(C.c_int8)
U8P = C.POINTER(C.c_uint8)


class orc_cfg(C.Structure):
    _fields_ = [("nEmbd", C.c_int), ("nLayer", C.c_int), ("nFF", C.c_int), ("nHead", C.c_int), ("nHeadKv", C.c_int),
                ("headDim", C.c_int), ("nRot", C.c_int), ("vocab", C.c_int), ("neox", C.c_int), ("ctx", C.c_int),
                ("kvF16", C.c_int), ("eps", C.c_double), ("ropeBase", C.c_double), ("hybrid", C.c_int),
                ("interval", C.c_int), ("convK", C.c_int), ("dk", C.c_int), ("dv", C.c_int), ("nK", C.c_int),
                ("nV", C.c_int)]


class orc_rng(C.Structure):
    _fields_ = [("a", C.c_uint32)]


class orc_sampler_opts(C.Structure):
    _fields_ = [("temperature", C.c_double), ("topP", C.c_double), ("minP", C.c_double), ("repeatPenalty", C.c_double),
                ("presence", C.c_double), ("frequency", C.c_double), ("topK", C.c_int), ("repeatLastN", C.c_int)]


_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_rng_seed": (None, [C.POINTER(orc_rng), C.c_uint32]),
            "orc_rng_next": (C.c_double, [C.POINTER(orc_rng)]),
            "orc_quantize_act": (None, [F32P, C.c_int, I8P, F32P, I32P]),
            "orc_row_bytes": (C.c_long, [C.c_int, C.c_long]),
            "orc_unpack_scale_min_k4": (None, [U8P, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
            "orc_dequant_row": (C.c_int, [C.c_int, U8P, C.c_long, C.c_long, F32P]),
            "orc_quantize_q8_0": (None, [F32P, C.c_long, U8P]),
            "orc_quantize_q4_0": (None, [F32P, C.c_long, U8P]),
            "orc_set_threads": (None, [C.c_int]),
            "orc_matvec": (C.c_int, [C.c_int, U8P, C.c_long, C.c_long, F32P, I8P, F32P, I32P, F32P]),
            "orc_rmsnorm": (None, [F32P, F32P, F32P, C.c_double, C.c_int]),
            "orc_softmax": (None, [F32P, C.c_int]),
            "orc_silu": (C.c_double, [C.c_double]),
            "orc_rope_tables": (None, [C.c_int, C.c_double, C.c_int, F32P, F32P, F32P]),
            "orc_apply_rope": (None, [F32P, C.c_int, C.c_int, C.c_int, C.c_int, F32P, F32P, C.c_int]),
            "orc_model_new": (C.c_void_p, [C.POINTER(orc_cfg), F32P]),
            "orc_model_set_global": (None, [C.c_void_p, C.c_int, C.c_long, C.c_long, U8P, C.c_int, U8P, F32P]),
            "orc_model_set_layer": (None, [C.c_void_p, C.c_int, F32P, F32P, F32P, F32P, F32P, F32P, F32P,
                                           C.POINTER(C.c_int), C.POINTER(U8P)]),
            "orc_model_set_layer_hybrid": (None, [C.c_void_p, C.c_int, F32P, F32P, F32P, F32P, F32P, F32P, F32P, F32P,
                                                  C.POINTER(C.c_int), C.POINTER(U8P)]),
            "orc_model_conv_state": (F32P, [C.c_void_p, C.POINTER(C.c_long)]),
            "orc_model_ssm_state": (F32P, [C.c_void_p, C.POINTER(C.c_long)]),
            "orc_sigmoid": (C.c_double, [C.c_double]),
            "orc_softplus": (C.c_double, [C.c_double]),
            "orc_conv_step": (None, [F32P, F32P, F32P, F32P, C.c_int, C.c_int]),
            "orc_l2norm_heads": (None, [F32P, C.c_int, C.c_int, C.c_double, C.c_double]),
            "orc_delta_rule_head": (None, [F32P, F32P, F32P, F32P, F32P, C.c_int, C.c_int, C.c_double, C.c_double]),
            "orc_gated_rmsnorm_head": (None, [F32P, F32P, F32P, C.c_int, C.c_double]),
            "orc_model_free": (None, [C.c_void_p]),
            "orc_model_pos": (C.c_int, [C.c_void_p]),
            "orc_model_truncate": (None, [C.c_void_p, C.c_int]),
            "orc_model_logits": (F32P, [C.c_void_p]),
            "orc_model_forward": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
            "orc_topk_select": (C.c_int, [F32P, C.c_int, C.c_int, I32P, F64P]),
            "orc_argmax": (C.c_int, [F32P, C.c_int]),
            "orc_distribution": (C.c_int, [C.POINTER(orc_sampler_opts), F32P, C.c_int, I32P, C.c_int, I32P, F64P, F64P,
                                           C.POINTER(C.c_int)]),
            "orc_draw": (C.c_int, [C.POINTER(orc_rng), I32P, F64P, C.c_int, C.c_double, C.c_int]),
            "orc_prob_of": (C.c_double, [I32P, F64P, C.c_int, C.c_double, C.c_int]),
            "orc_draw_residual": (C.c_int, [C.POINTER(orc_rng), I32P, F64P, C.c_int, C.c_double, C.c_int, I32P, F64P,
                                            C.c_int, C.c_double, F64P]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def p(a, t):
    return a.ctypes.data_as(C.POINTER(t))


def set_threads(n: int):
    lib().orc_set_threads(int(n))


# ------------------------------------------------------------------------------------------------ kernels
def f32_to_f16(x: float) -> int:
    return int(lib().orc_f32_to_f16(C.c_float(x)))


def f16_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(C.c_uint16(h)))


def quantize_act(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    q = np.zeros(n, np.int8)
    d = np.zeros(n // 32, np.float32)
    s = np.zeros(n // 32, np.int32)
    lib().orc_quantize_act(p(x, C.c_float), n, p(q, C.c_int8), p(d, C.c_float), p(s, C.c_int32))
    return q, d, s


def dequant(type_: int, raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        rc = lib().orc_dequant_row(type_, p(raw, C.c_uint8), cols, r, p(out[r], C.c_float))
        if rc:
            raise ValueError(f"unsupported type {type_}")
    return out


def matvec(type_: int, raw: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """matvec(W, new Act(x)) (src/compute/ref-kernels.js:127-302) for one activation vector."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    q, d, s = quantize_act(x) if cols % 32 == 0 else (np.zeros(cols, np.int8), np.zeros(1, np.float32), np.zeros(1, np.int32))
    y = np.zeros(rows, np.float32)
    rc = lib().orc_matvec(type_, p(raw, C.c_uint8), rows, cols, p(x, C.c_float), p(q, C.c_int8), p(d, C.c_float),
                          p(s, C.c_int32), p(y, C.c_float))
    if rc:
        raise ValueError(f"unsupported type {type_}")
    return y


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0(p(x, C.c_float), x.size, p(out, C.c_uint8))
    return out


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32 * 18, np.uint8)
    lib().orc_quantize_q4_0(p(x, C.c_float), x.size, p(out, C.c_uint8))
    return out


class Rng:
    """mulberry32 (src/util/rng.js:4-13)."""

    def __init__(self, seed: int):
        self.s = orc_rng()
        lib().orc_rng_seed(C.byref(self.s), seed & 0xFFFFFFFF)

    def __call__(self) -> float:
        return float(lib().orc_rng_next(C.byref(self.s)))

    @property
    def state(self):
        return int(self.s.a)


# ------------------------------------------------------------------------------------------------ sampler
class Dist:
    def __init__(self, ids, probs, total, greedy):
        self.ids, self.probs, self.total, self.greedy = ids, probs, total, greedy


class Sampler:
    """createSampler (src/sampling/sampler.js:81-155) over host logits."""

    def __init__(self, temperature=0.8, top_k=40, top_p=0.95, min_p=0.0, repeat_penalty=1.0, repeat_last_n=64,
                 presence_penalty=0.0, frequency_penalty=0.0, seed=1, argmax=False):
        self.o = orc_sampler_opts(temperature=-1.0 if argmax else temperature, topP=top_p, minP=min_p,
                                  repeatPenalty=1.0 if argmax else repeat_penalty,
                                  presence=0.0 if argmax else presence_penalty,
                                  frequency=0.0 if argmax else frequency_penalty, topK=top_k, repeatLastN=repeat_last_n)
        self.rng = Rng(seed)
        self.greedy = argmax or temperature <= 0
        # usesHistory (src/sampling/sampler.js:154): only penalties make the history matter
        self.uses_history = not argmax and (repeat_penalty != 1 or presence_penalty != 0 or frequency_penalty != 0)

    def distribution(self, logits: np.ndarray, history=()) -> Dist:
        l = np.ascontiguousarray(logits, dtype=np.float32).copy()
        n = l.size
        cap = n if (self.o.topK <= 0 or self.o.topK >= n) else self.o.topK
        ids = np.zeros(max(cap, 1), np.int32)
        probs = np.zeros(max(cap, 1), np.float64)
        total = C.c_double()
        greedy = C.c_int()
        h = np.ascontiguousarray(np.asarray(list(history), dtype=np.int32))
        keep = lib().orc_distribution(C.byref(self.o), p(l, C.c_float), n, p(h, C.c_int32) if len(h) else None, len(h),
                                      p(ids, C.c_int32), p(probs, C.c_double), C.byref(total), C.byref(greedy))
        return Dist(ids[:keep].copy(), probs[:keep].copy(), total.value, bool(greedy.value))

    def draw(self, d: Dist) -> int:
        return int(lib().orc_draw(C.byref(self.rng.s), p(d.ids, C.c_int32), p(d.probs, C.c_double), len(d.ids), d.total,
                                  1 if d.greedy else 0))

    def sample(self, logits, history=()) -> int:
        return self.draw(self.distribution(logits, history))

    def rand(self) -> float:
        return self.rng()


def prob_of(d: Dist, tok: int) -> float:
    return float(lib().orc_prob_of(p(d.ids, C.c_int32), p(d.probs, C.c_double), len(d.ids), d.total, int(tok)))


def draw_residual(s: Sampler, pd: Dist, qd: Dist, vocab: int) -> int:
    scratch = np.zeros(vocab, np.float64)
    return int(lib().orc_draw_residual(C.byref(s.rng.s), p(pd.ids, C.c_int32), p(pd.probs, C.c_double), len(pd.ids),
                                       pd.total, 1 if pd.greedy else 0, p(qd.ids, C.c_int32), p(qd.probs, C.c_double),
                                       len(qd.ids), qd.total, p(scratch, C.c_double)))


def topk_select(logits: np.ndarray, k: int):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(k, np.int32)
    vals = np.zeros(k, np.float64)
    n = lib().orc_topk_select(p(l, C.c_float), l.size, k, p(ids, C.c_int32), p(vals, C.c_double))
    return ids[:n], vals[:n]


# ------------------------------------------------------------------------------------------------ model
HYBRID_ARCHS = ("qwen35",)


class OracleModel:
    """RefModel (src/model/forward.js:100-257) and, for arch qwen35, Qwen35Model (src/model/forward-qwen35.js:158-342):
    single-token forward, f64 math, f32 storage; kv='f16' rounds the cache like the pool's js-kernel path. Hybrid models
    keep the recurrent state, its checkpoints (oracle.checkpoints) and truncate by restore + replay. Weights are
    memory-mapped from the GGUF file (zerollm_amd.gguf reader) or come from an ArraySource."""

    def __init__(self, path_or_gguf, ctx=2048, kv="f32", threads=1, max_checkpoints=None, checkpoint_every=0,
                 boundary_ids=()):
        from zerollm_amd import gguf as G  # the GGUF container parser (file format only)
        from .checkpoints import StateCheckpoints

        g = G.read_gguf(path_or_gguf) if isinstance(path_or_gguf, str) else path_or_gguf
        self.g = g
        a = g.get("general.architecture")
        if a not in ("llama", "qwen2", "qwen3") + HYBRID_ARCHS:
            raise ValueError(f"oracle: unsupported architecture {a}")
        self.hybrid = a in HYBRID_ARCHS
        n_embd = g.get(f"{a}.embedding_length")
        n_head = g.get(f"{a}.attention.head_count")
        n_head_kv = g.get(f"{a}.attention.head_count_kv", n_head)
        hd = g.get(f"{a}.attention.key_length", n_embd // n_head)
        toks = g.get("tokenizer.ggml.tokens")
        vocab = g.get(f"{a}.vocab_size") or (len(toks) if toks else g.tensor("token_embd.weight").dims[1])
        self.cfg = dict(nEmbd=n_embd, nLayer=g.get(f"{a}.block_count"), nFF=g.get(f"{a}.feed_forward_length"),
                        nHead=n_head, nHeadKv=n_head_kv, headDim=hd, nRot=g.get(f"{a}.rope.dimension_count", hd),
                        vocabSize=vocab, nCtxTrain=g.get(f"{a}.context_length"),
                        rmsEps=g.get(f"{a}.attention.layer_norm_rms_epsilon", 1e-5),
                        ropeBase=g.get(f"{a}.rope.freq_base", 10000.0))
        self.ctx = min(ctx, self.cfg["nCtxTrain"])
        hyb = {}
        if self.hybrid:
            # qwen35 layout (src/model/config.js:126-156)
            hyb = dict(hybrid=1, interval=g.get(f"{a}.full_attention_interval", 4), convK=g.get(f"{a}.ssm.conv_kernel"),
                       dk=g.get(f"{a}.ssm.state_size"), nK=g.get(f"{a}.ssm.group_count"),
                       nV=g.get(f"{a}.ssm.time_step_rank"))
            hyb["dv"] = g.get(f"{a}.ssm.inner_size") // hyb["nV"]
            self.cfg.update(hyb)
        c = orc_cfg(nEmbd=n_embd, nLayer=self.cfg["nLayer"], nFF=self.cfg["nFF"], nHead=n_head, nHeadKv=n_head_kv,
                    headDim=hd, nRot=self.cfg["nRot"], vocab=vocab, neox=0 if a == "llama" else 1, ctx=self.ctx,
                    kvF16=1 if kv == "f16" else 0, eps=float(self.cfg["rmsEps"]), ropeBase=float(self.cfg["ropeBase"]),
                    **hyb)
        self._keep = []
        rf = g.floats("rope_freqs.weight") if g.tensor("rope_freqs.weight") else None
        if rf is not None:
            rf = np.ascontiguousarray(rf)
            self._keep.append(rf)
        L = lib()
        L.orc_set_threads(threads)
        self.h = L.orc_model_new(C.byref(c), p(rf, C.c_float) if rf is not None else None)
        self.vocab = vocab

        def raw(name):
            d = g.data(name)
            self._keep.append(d)
            return d.ctypes.data_as(U8P)

        def vec(name):
            if not g.tensor(name):
                return None
            v = np.ascontiguousarray(g.floats(name))
            self._keep.append(v)
            return p(v, C.c_float)

        te = g.tensor("token_embd.weight")
        out = g.tensor("output.weight") or te
        L.orc_model_set_global(self.h, te.type, vocab, n_embd, raw("token_embd.weight"), out.type, raw(out.name),
                               vec("output_norm.weight"))
        for l in range(self.cfg["nLayer"]):
            pre = f"blk.{l}."
            if self.hybrid:
                rec = (l + 1) % hyb["interval"] != 0
                mix = ["attn_qkv", "attn_gate", "ssm_alpha", "ssm_beta", "ssm_out"] if rec else \
                    ["attn_q", "attn_k", "attn_v", "attn_output", None]
                names = mix + ["ffn_gate", "ffn_up", "ffn_down"]
                types = (C.c_int * 8)(*[g.tensor(pre + n + ".weight").type if n else 0 for n in names])
                datas = (U8P * 8)(*[raw(pre + n + ".weight") if n else None for n in names])
                L.orc_model_set_layer_hybrid(self.h, l, vec(pre + "attn_norm.weight"), vec(pre + "post_attention_norm.weight"),
                                             vec(pre + "attn_q_norm.weight"), vec(pre + "attn_k_norm.weight"),
                                             vec(pre + "ssm_conv1d.weight"), vec(pre + "ssm_dt.bias"), vec(pre + "ssm_a"),
                                             vec(pre + "ssm_norm.weight"), types, datas)
                continue
            names = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
            types = (C.c_int * 7)(*[g.tensor(pre + n + ".weight").type for n in names])
            datas = (U8P * 7)(*[raw(pre + n + ".weight") for n in names])
            L.orc_model_set_layer(self.h, l, vec(pre + "attn_norm.weight"), vec(pre + "ffn_norm.weight"),
                                  vec(pre + "attn_q_norm.weight"), vec(pre + "attn_k_norm.weight"),
                                  vec(pre + "attn_q.bias"), vec(pre + "attn_k.bias"), vec(pre + "attn_v.bias"), types, datas)
        self.tokens = []
        self.ck = StateCheckpoints(max_checkpoints, checkpoint_every, boundary_ids) if self.hybrid else None
        self.prev_no_logits = False

    @property
    def pos(self):
        return lib().orc_model_pos(self.h)

    # ---- hybrid models: the live recurrent state as numpy views (conv, ssm)
    def state(self):
        n1, n2 = C.c_long(), C.c_long()
        cp = lib().orc_model_conv_state(self.h, C.byref(n1))
        sp = lib().orc_model_ssm_state(self.h, C.byref(n2))
        return np.ctypeslib.as_array(cp, shape=(n1.value,)), np.ctypeslib.as_array(sp, shape=(n2.value,))

    def checkpoint(self):
        self.ck.save(self.pos, self.state())

    def mark_rollback(self):
        """markRollback (src/compute/pool.js:269): the rollback slot, hybrid models only."""
        if self.hybrid:
            self.ck.mark(self.pos, self.state())

    def truncate_plan(self, n):
        return self.ck.plan(n, self.pos) if self.hybrid else (min(n, self.pos), 0)

    def forward(self, token: int, logits=True):
        if self.hybrid and 0 <= token < self.vocab and self.pos < self.ctx:
            # checkpoint policy before the token (src/model/forward-qwen35.js:312-314)
            if self.ck.wants_before(self.pos, int(token), bool(logits), self.prev_no_logits):
                self.checkpoint()
            self.prev_no_logits = not logits
        rc = lib().orc_model_forward(self.h, int(token), 1 if logits else 0)
        if rc == -1:
            raise RuntimeError(f"context full ({self.ctx} tokens)")
        if rc == -2:
            raise RuntimeError(f"token id {token} out of range")
        self.tokens.append(int(token))
        if not logits:
            return None
        ptr = lib().orc_model_logits(self.h)
        return np.ctypeslib.as_array(ptr, shape=(self.vocab,)).copy()

    def truncate(self, n: int) -> int:
        """Positional for KV-cache models; hybrid models restore the nearest snapshot <= n and replay the tokens in
        between (Qwen35Model.truncate, src/model/forward-qwen35.js:284-300). Returns the tokens replayed."""
        if n >= self.pos:
            return 0
        n = max(0, n)
        if not self.hybrid:
            lib().orc_model_truncate(self.h, n)
            del self.tokens[n:]
            return 0
        frm, replay = self.ck.plan(n, self.pos)
        tail = self.tokens[frm:n]
        self.ck.drop_after(n)
        self.ck.restore(self.state(), frm)
        lib().orc_model_truncate(self.h, frm)
        del self.tokens[frm:]
        self.prev_no_logits = False
        for t in tail:
            self.forward(t, logits=False)
        if replay > 0:
            self.checkpoint()
        self.prev_no_logits = False
        return replay

    def reset(self):
        self.truncate(0)
        if self.hybrid:
            st = self.state()
            st[0][:] = 0
            st[1][:] = 0
            self.ck.clear()
            self.prev_no_logits = False

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ArraySource:
    """A GGUF-like view (get / tensor / data / floats) over in-memory raw tensors of a synthetic model spec
    (zerollm_amd.synth.ModelSpec), so the oracle can run a model that only exists in memory."""

    class _T:
        def __init__(self, name, type_, dims):
            self.name, self.type, self.dims = name, type_, dims

    def __init__(self, spec, arrays):
        a = spec.arch
        self.meta = {
            "general.architecture": a, f"{a}.embedding_length": spec.n_embd, f"{a}.attention.head_count": spec.n_head,
            f"{a}.attention.head_count_kv": spec.n_head_kv, f"{a}.attention.key_length": spec.head_dim,
            f"{a}.vocab_size": spec.vocab, f"{a}.block_count": spec.n_layer, f"{a}.feed_forward_length": spec.n_ff,
            f"{a}.rope.dimension_count": spec.head_dim, f"{a}.context_length": spec.ctx_train,
            f"{a}.attention.layer_norm_rms_epsilon": float(np.float32(spec.rms_eps)),
            f"{a}.rope.freq_base": float(np.float32(spec.rope_base)),
        }
        if getattr(spec, "hybrid", False):
            self.meta.update({
                f"{a}.rope.dimension_count": spec.n_rot, f"{a}.full_attention_interval": spec.interval,
                f"{a}.ssm.conv_kernel": spec.conv_k, f"{a}.ssm.state_size": spec.d_state,
                f"{a}.ssm.group_count": spec.n_group, f"{a}.ssm.time_step_rank": spec.dt_rank,
                f"{a}.ssm.inner_size": spec.d_inner,
            })
        self.arrays = arrays
        self.tensors = {t.name: self._T(t.name, t.type, t.dims) for t in spec.tensors}

    def get(self, k, default=None):
        return self.meta.get(k, default)

    def tensor(self, name):
        return self.tensors.get(name)

    def data(self, name):
        return self.arrays[name]

    def floats(self, name):
        return self.arrays[name].view(np.float32)
