"""Synthetic random-init models of named shapes: tensor tables for the library's generator, GGUF files, HBM models.

Every matrix is std * N(0, 1) from a counter-based stream per tensor (seed = f(model seed, tensor name)), quantised
with this library's quantisers; norm weights are constant. The GPU and CPU generators produce identical bytes, so a
model built directly in HBM equals the GGUF file written from the same spec. Mirrors the role of zerollm's
make-tiny-gguf (tools/make-tiny-gguf.js:28-149) with the shapes of the benchmark configurations.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib, gguf
from ._lib import call

MASK64 = (1 << 64) - 1


def _mix(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def tensor_seed(model_seed: int, name: str) -> int:
    """Seed of a named tensor: FNV-1a of the name mixed with the model seed."""
    h = 1469598103934665603
    for b in name.encode():
        h ^= b
        h = (h * 1099511628211) & MASK64
    return _mix(h ^ ((model_seed * 0x9E3779B97F4A7C15) & MASK64))


@dataclass
class TensorSpec:
    name: str
    type: int
    rows: int
    cols: int
    seed: int = 0
    std: float = 0.02
    src_cols: int = 0
    col0: int = 0
    fill: bool = False
    fill_value: float = 1.0

    @property
    def dims(self):
        return [self.cols] if self.rows == 1 else [self.cols, self.rows]

    @property
    def nbytes(self):
        return gguf.tensor_bytes(self.type, self.dims)

    def c(self) -> _lib.zl_synth_tensor:
        return _lib.zl_synth_tensor(name=self.name.encode(), type=self.type, rows=self.rows, cols=self.cols, seed=self.seed,
                                    std=self.std, src_cols=self.src_cols or self.cols, col0=self.col0,
                                    fill=1 if self.fill else 0, fill_value=self.fill_value)


@dataclass
class ModelSpec:
    arch: str
    n_embd: int
    n_layer: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_ff: int
    vocab: int
    ctx_train: int
    rope_base: float = 1e6
    rms_eps: float = 1e-6
    name: str = "synthetic"
    tensors: list = field(default_factory=list)

    def config(self) -> _lib.zl_config:
        return _lib.zl_config(arch={"llama": 0, "qwen2": 1, "qwen3": 2}[self.arch], n_ctx_train=self.ctx_train,
                              n_embd=self.n_embd, n_layer=self.n_layer, n_ff=self.n_ff, n_head=self.n_head,
                              n_head_kv=self.n_head_kv, head_dim=self.head_dim, n_rot=self.head_dim, vocab=self.vocab,
                              rms_eps=self.rms_eps, rope_base=self.rope_base, neox=0 if self.arch == "llama" else 1,
                              qk_norm=1 if self.arch == "qwen3" else 0, qkv_bias=0,
                              tied=0 if any(t.name == "output.weight" for t in self.tensors) else 1, has_rope_freqs=0)

    @property
    def weight_bytes(self) -> int:
        """Quantised matrix bytes streamed by one pass (layers + output head; the embedding is one row per token)."""
        return sum(t.nbytes for t in self.tensors if t.rows > 1 and t.name != "token_embd.weight")


def build_spec(arch, n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, vocab, ctx_train, types, seed, std=0.02,
               embd_from=None, name="synthetic", norm_value=1.0) -> ModelSpec:
    """types: dict with keys embd, output, q, k, v, o, gate, up, down (ggml type ids).
    embd_from: (seed, src_cols) to take token_embd / output values from another model's tensors (their first n_embd
    columns), e.g. a draft that shares the target's embedding and output head."""
    s = ModelSpec(arch, n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, vocab, ctx_train, name=name)
    qd, kvd = n_head * head_dim, n_head_kv * head_dim

    def mat(nm, key, rows, cols):
        if embd_from and nm in ("token_embd.weight", "output.weight"):
            src_seed, src_cols = embd_from
            s.tensors.append(TensorSpec(nm, types[key], rows, cols, tensor_seed(src_seed, nm), std, src_cols, 0))
        else:
            s.tensors.append(TensorSpec(nm, types[key], rows, cols, tensor_seed(seed, nm), std))

    def vec(nm, n):
        s.tensors.append(TensorSpec(nm, gguf.F32, 1, n, fill=True, fill_value=norm_value))

    mat("token_embd.weight", "embd", vocab, n_embd)
    vec("output_norm.weight", n_embd)
    mat("output.weight", "output", vocab, n_embd)
    for l in range(n_layer):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", n_embd)
        mat(p + "attn_q.weight", "q", qd, n_embd)
        mat(p + "attn_k.weight", "k", kvd, n_embd)
        mat(p + "attn_v.weight", "v", kvd, n_embd)
        mat(p + "attn_output.weight", "o", n_embd, qd)
        if arch == "qwen3":
            vec(p + "attn_q_norm.weight", head_dim)
            vec(p + "attn_k_norm.weight", head_dim)
        vec(p + "ffn_norm.weight", n_embd)
        mat(p + "ffn_gate.weight", "gate", n_ff, n_embd)
        mat(p + "ffn_up.weight", "up", n_ff, n_embd)
        mat(p + "ffn_down.weight", "down", n_embd, n_ff)
    return s


def all_type(t):
    return dict(embd=t, output=t, q=t, k=t, v=t, o=t, gate=t, up=t, down=t)


# Q4_K_M mix as llama.cpp names it: Q6_K for attn_v, ffn_down and the output head, Q4_K elsewhere
# (the same rule as zerollm's generator, tools/make-tiny-gguf.js:71)
Q4_K_M = dict(embd=gguf.Q4_K, output=gguf.Q6_K, q=gguf.Q4_K, k=gguf.Q4_K, v=gguf.Q6_K, o=gguf.Q4_K, gate=gguf.Q4_K,
              up=gguf.Q4_K, down=gguf.Q6_K)


def tiny_pair(seed=1, draft_layers=2, quant=gguf.Q8_0):
    """Tiny qwen3 target (4 layers, d 512, 8/4 heads, hd 64, FFN 1536, vocab 32000, theta 1e6, all Q8_0, norms 1.0)
    and a draft made of its first 2 layers plus the same embedding / output head (same seed, so identical tensors)."""
    kw = dict(arch="qwen3", n_embd=512, n_head=8, n_head_kv=4, head_dim=64, n_ff=1536, vocab=32000, ctx_train=2048,
              types=all_type(quant), seed=seed)
    return build_spec(n_layer=4, name="tiny-target", **kw), build_spec(n_layer=draft_layers, name="tiny-draft", **kw)


def qwen3_8b_pair(seed=8, draft_seed=6, ctx_train=32768):
    """Qwen3-8B-shaped Q4_K_M target and Qwen3-0.6B-shaped Q8_0 draft. The draft's embedding and output head are the
    target's N(0, 0.02) values restricted to the first 1024 input columns, quantised to Q8_0."""
    t = build_spec("qwen3", 4096, 36, 32, 8, 128, 12288, 151936, ctx_train, Q4_K_M, seed, name="qwen3-8b-shaped")
    d = build_spec("qwen3", 1024, 28, 16, 8, 128, 3072, 151936, ctx_train, all_type(gguf.Q8_0), draft_seed,
                   embd_from=(seed, 4096), name="qwen3-0.6b-shaped")
    return t, d


def tensor_bytes(t: TensorSpec, use_device=False) -> np.ndarray:
    """Raw ggml bytes (or F32 values) of one synthetic tensor."""
    out = np.empty(t.nbytes, dtype=np.uint8)
    ct = t.c()
    call("zl_synth_tensor_bytes", C.byref(ct), 1 if use_device else 0, out.ctypes.data_as(C.c_void_p))
    return out


def write_gguf(path: str, spec: ModelSpec, use_device=False):
    """Write the synthetic model as a GGUF file with the metadata zerollm's loader reads (src/model/config.js:275-325)."""
    a = spec.arch
    U32, F32, STR, ARR, I32 = gguf.UINT32, gguf.FLOAT32, gguf.STRING, gguf.ARRAY, gguf.INT32
    M = gguf.MetaKV
    tokens = [f"<t{i}>" for i in range(spec.vocab)]
    meta = [
        M("general.architecture", STR, a), M("general.name", STR, spec.name),
        M(f"{a}.context_length", U32, spec.ctx_train), M(f"{a}.embedding_length", U32, spec.n_embd),
        M(f"{a}.block_count", U32, spec.n_layer), M(f"{a}.feed_forward_length", U32, spec.n_ff),
        M(f"{a}.attention.head_count", U32, spec.n_head), M(f"{a}.attention.head_count_kv", U32, spec.n_head_kv),
        M(f"{a}.attention.layer_norm_rms_epsilon", F32, spec.rms_eps), M(f"{a}.rope.freq_base", F32, spec.rope_base),
        M(f"{a}.rope.dimension_count", U32, spec.head_dim),
        M(f"{a}.attention.key_length", U32, spec.head_dim), M(f"{a}.attention.value_length", U32, spec.head_dim),
        M("tokenizer.ggml.model", STR, "gpt2"),
        M("tokenizer.ggml.tokens", ARR, tokens, STR),
        M("tokenizer.ggml.token_type", ARR, [1] * spec.vocab, I32),
    ]
    tensors = [(t.name, t.dims, t.type, tensor_bytes(t, use_device)) for t in spec.tensors]
    gguf.write_gguf(path, meta, tensors)


def build_on_device(spec: ModelSpec, ctx=None, kv="f32", max_batch=16, logits_batch=None):
    from .model import HipModel
    return HipModel.from_synth(spec.config(), [t.c() for t in spec.tensors], ctx=ctx, kv=kv, max_batch=max_batch,
                               logits_batch=logits_batch)
