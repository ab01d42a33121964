"""CPU baseline — benchmark and test infrastructure only (bench.py's cpu_baseline leg and tests/ use it; the product
never imports it).

SimdPoolModel: ctypes wrapper of oracle/pool_simd.c, a multi-threaded AVX-512 VNNI restatement of the reference's
worker-pool model (PoolModel, src/compute/pool.js:33-316): forward(token), forward_batch(tokens, logits) with up to
max_batch tokens per pass over the weights (forwardBatch, :145-160), positional truncate. Each pass computes exactly the
oracle's single-token arithmetic per token (tests/test_pool_simd.py pins every logit bit for bit against OracleModel),
so the speculative loop of oracle/spec.py runs on it unchanged and yields the same tokens, batch-verifying k + 1 rows in
one pass as the reference's speculative loop does with a pool (src/model/speculative.js:39-48). Llama / qwen2 / qwen3
architectures with an f16 KV cache (the benchmark's models); the formats Q8_0, Q4_K and Q6_K run the SIMD tiles, the
others the oracle's scalar rows on each thread's slice.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .oracle import F32P, I32P, U8P, lib, p

MAX_BATCH = 16


class ps_cfg(C.Structure):
    _fields_ = [("nEmbd", C.c_int), ("nLayer", C.c_int), ("nFF", C.c_int), ("nHead", C.c_int), ("nHeadKv", C.c_int),
                ("headDim", C.c_int), ("nRot", C.c_int), ("vocab", C.c_int), ("neox", C.c_int), ("ctx", C.c_int),
                ("eps", C.c_double), ("ropeBase", C.c_double)]


_sig_done = False


def _lib():
    global _sig_done
    L = lib()
    if not _sig_done:
        sig = {
            "ps_supported": (C.c_int, []),
            "ps_model_new": (C.c_void_p, [C.POINTER(ps_cfg), F32P, C.c_int]),
            "ps_model_set_global": (None, [C.c_void_p, C.c_int, U8P, C.c_int, U8P, F32P]),
            "ps_model_set_layer": (None, [C.c_void_p, C.c_int, F32P, F32P, F32P, F32P, F32P, F32P, F32P,
                                          C.POINTER(C.c_int), C.POINTER(U8P)]),
            "ps_model_free": (None, [C.c_void_p]),
            "ps_model_pos": (C.c_int, [C.c_void_p]),
            "ps_model_truncate": (None, [C.c_void_p, C.c_int]),
            "ps_model_logits": (F32P, [C.c_void_p]),
            "ps_model_forward": (C.c_int, [C.c_void_p, I32P, C.c_int, C.c_int]),
            "ps_matmul": (C.c_int, [C.c_int, U8P, C.c_long, C.c_long, C.c_int, F32P, F32P, C.c_int]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _sig_done = True
    return L


def supported() -> bool:
    """True when this CPU has AVX-512 F/BW/DQ/VL, AVX-512 VNNI and F16C."""
    return bool(_lib().ps_supported())


def cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def matmul(type_: int, raw: np.ndarray, rows: int, cols: int, X: np.ndarray, threads: int = 1) -> np.ndarray:
    """y[b] = W x_b for up to MAX_BATCH rows of X through the SIMD tiles (the oracle's matvec per row, bit for bit)."""
    raw = np.ascontiguousarray(raw, np.uint8)
    X = np.ascontiguousarray(X, np.float32)
    B = X.shape[0]
    y = np.zeros((B, rows), np.float32)
    rc = _lib().ps_matmul(type_, p(raw, C.c_uint8), rows, cols, B, p(X, C.c_float), p(y, C.c_float), threads)
    if rc:
        raise RuntimeError("ps_matmul: unsupported CPU, batch or shape")
    return y


class SimdPoolModel:
    """PoolModel's interface (src/compute/pool.js:33-316) over the SIMD restatement; weights from a GGUF file or an
    oracle.ArraySource."""

    max_batch = MAX_BATCH
    logits_batch = MAX_BATCH

    def __init__(self, path_or_gguf, ctx=2048, threads=16):
        from zerollm_amd import gguf as G  # the GGUF container parser (file format only)

        if not supported():
            raise RuntimeError(f"the SIMD pool restatement needs AVX-512 VNNI and F16C ({cpu_name()} lacks them)")
        g = G.read_gguf(path_or_gguf) if isinstance(path_or_gguf, str) else path_or_gguf
        a = g.get("general.architecture")
        if a not in ("llama", "qwen2", "qwen3"):
            raise ValueError(f"SIMD pool model: unsupported architecture {a}")
        n_embd = g.get(f"{a}.embedding_length")
        n_head = g.get(f"{a}.attention.head_count")
        n_head_kv = g.get(f"{a}.attention.head_count_kv", n_head)
        hd = g.get(f"{a}.attention.key_length", n_embd // n_head)
        toks = g.get("tokenizer.ggml.tokens")
        vocab = g.get(f"{a}.vocab_size") or (len(toks) if toks else g.tensor("token_embd.weight").dims[1])
        self.ctx = min(ctx, g.get(f"{a}.context_length"))
        self.vocab = vocab
        self.threads = int(threads)
        c = ps_cfg(nEmbd=n_embd, nLayer=g.get(f"{a}.block_count"), nFF=g.get(f"{a}.feed_forward_length"), nHead=n_head,
                   nHeadKv=n_head_kv, headDim=hd, nRot=g.get(f"{a}.rope.dimension_count", hd), vocab=vocab,
                   neox=0 if a == "llama" else 1, ctx=self.ctx,
                   eps=float(g.get(f"{a}.attention.layer_norm_rms_epsilon", 1e-5)),
                   ropeBase=float(g.get(f"{a}.rope.freq_base", 10000.0)))
        self._keep = []
        rf = g.floats("rope_freqs.weight") if g.tensor("rope_freqs.weight") else None
        if rf is not None:
            rf = np.ascontiguousarray(rf)
            self._keep.append(rf)
        L = _lib()
        self.h = L.ps_model_new(C.byref(c), p(rf, C.c_float) if rf is not None else None, self.threads)
        if not self.h:
            raise RuntimeError("ps_model_new failed")

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
        L.ps_model_set_global(self.h, te.type, raw("token_embd.weight"), out.type, raw(out.name),
                              vec("output_norm.weight"))
        for l in range(c.nLayer):
            pre = f"blk.{l}."
            names = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
            types = (C.c_int * 7)(*[g.tensor(pre + n + ".weight").type for n in names])
            datas = (U8P * 7)(*[raw(pre + n + ".weight") for n in names])
            L.ps_model_set_layer(self.h, l, vec(pre + "attn_norm.weight"), vec(pre + "ffn_norm.weight"),
                                 vec(pre + "attn_q_norm.weight"), vec(pre + "attn_k_norm.weight"),
                                 vec(pre + "attn_q.bias"), vec(pre + "attn_k.bias"), vec(pre + "attn_v.bias"), types,
                                 datas)
        self.tokens = []

    @property
    def pos(self):
        return _lib().ps_model_pos(self.h)

    def forward_batch(self, tokens, logits="last"):
        """forwardBatch (src/compute/pool.js:145-160): logits 'none' / False, 'last' / True, or 'all' (rows b * vocab)."""
        toks = np.ascontiguousarray([int(t) for t in tokens], np.int32)
        B = len(toks)
        want = {"none": 0, False: 0, "last": 1, True: 1, "all": 2}[logits]
        rc = _lib().ps_model_forward(self.h, p(toks, C.c_int32), B, want)
        if rc == -1:
            raise RuntimeError(f"context full ({self.ctx} tokens)")
        if rc == -2:
            raise RuntimeError(f"token id out of range in {list(toks)}")
        if rc == -3:
            raise RuntimeError(f"batch of {B} tokens (max {MAX_BATCH})")
        self.tokens.extend(int(t) for t in toks)
        if want == 0:
            return None
        rows = B if want == 2 else 1
        out = np.ctypeslib.as_array(_lib().ps_model_logits(self.h), shape=(rows * self.vocab,)).copy()
        return out.reshape(rows, self.vocab) if want == 2 else out

    def forward(self, token: int, logits=True):
        return self.forward_batch([token], logits="last" if logits else "none")

    def truncate(self, n: int) -> int:
        if n < self.pos:
            n = max(0, n)
            _lib().ps_model_truncate(self.h, n)
            del self.tokens[n:]
        return 0

    def reset(self):
        self.truncate(0)

    def close(self):
        if self.h:
            _lib().ps_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
