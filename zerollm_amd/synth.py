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


def seeded_ids(n: int, seed: int, vocab: int) -> list:
    """n token ids floor(mulberry32(seed)() * vocab), the reference's seeded prompts (src/util/rng.js:4-13)."""
    a = seed & 0xFFFFFFFF
    out = []
    for _ in range(n):
        a = (a + 0x6D2B79F5) & 0xFFFFFFFF
        t = ((a ^ (a >> 15)) * (a | 1)) & 0xFFFFFFFF
        t ^= (t + (((t ^ (t >> 7)) * (t | 61)) & 0xFFFFFFFF)) & 0xFFFFFFFF
        out.append(int(((t ^ (t >> 14)) & 0xFFFFFFFF) / 4294967296.0 * vocab))
    return out


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
    fill: int = 0  # 1 constant fill_value, 2 fill_value + std * N(0, 1), 3 fill_value then std from element src_cols
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
                                    fill=int(self.fill), fill_value=self.fill_value)


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
    # qwen35 hybrid layout: layer l is a Gated DeltaNet layer unless (l + 1) % interval == 0
    n_rot: int = 0
    interval: int = 0
    conv_k: int = 0
    d_state: int = 0
    n_group: int = 0
    dt_rank: int = 0
    d_inner: int = 0

    @property
    def hybrid(self) -> bool:
        return self.arch == "qwen35"

    def config(self) -> _lib.zl_config:
        return _lib.zl_config(arch={"llama": 0, "qwen2": 1, "qwen3": 2, "qwen35": 3}[self.arch],
                              n_ctx_train=self.ctx_train, n_embd=self.n_embd, n_layer=self.n_layer, n_ff=self.n_ff,
                              n_head=self.n_head, n_head_kv=self.n_head_kv, head_dim=self.head_dim,
                              n_rot=self.n_rot or self.head_dim, vocab=self.vocab, rms_eps=self.rms_eps,
                              rope_base=self.rope_base, neox=0 if self.arch == "llama" else 1,
                              qk_norm=1 if self.arch in ("qwen3", "qwen35") else 0, qkv_bias=0,
                              tied=0 if any(t.name == "output.weight" for t in self.tensors) else 1, has_rope_freqs=0,
                              hybrid=1 if self.hybrid else 0, full_attn_interval=self.interval,
                              ssm_conv_kernel=self.conv_k, ssm_d_state=self.d_state, ssm_n_group=self.n_group,
                              ssm_dt_rank=self.dt_rank, ssm_d_inner=self.d_inner)

    @property
    def weight_bytes(self) -> int:
        """Quantised matrix bytes streamed by one pass (layers + output head; the embedding is one row per token, but
        with tied embeddings it is also the output head)."""
        tied = not any(t.name == "output.weight" for t in self.tensors)
        return sum(t.nbytes for t in self.tensors if t.rows > 1 and (tied or t.name != "token_embd.weight"))


def build_spec(arch, n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, vocab, ctx_train, types, seed, std=0.02,
               embd_from=None, name="synthetic", norm_value=1.0, layer_std=None) -> ModelSpec:
    """types: dict with keys embd, output, q, k, v, o, gate, up, down (ggml type ids).
    embd_from: (seed, src_cols) to take token_embd / output values from another model's tensors (their first n_embd
    columns), e.g. a draft that shares the target's embedding and output head.
    layer_std: std of the per-layer matrices (default std); a smaller value keeps the residual stream close to the
    embedding, so a draft made of the first layers agrees with the target more often."""
    lstd = std if layer_std is None else layer_std
    s = ModelSpec(arch, n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, vocab, ctx_train, name=name)
    qd, kvd = n_head * head_dim, n_head_kv * head_dim

    def mat(nm, key, rows, cols):
        if embd_from and nm in ("token_embd.weight", "output.weight"):
            src_seed, src_cols = embd_from
            s.tensors.append(TensorSpec(nm, types[key], rows, cols, tensor_seed(src_seed, nm), std, src_cols, 0))
        else:
            sd = std if nm in ("token_embd.weight", "output.weight") else lstd
            s.tensors.append(TensorSpec(nm, types[key], rows, cols, tensor_seed(seed, nm), sd))

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


def build_qwen35_spec(n_embd, n_layer, n_head, n_head_kv, head_dim, n_rot, n_ff, vocab, ctx_train, types, seed,
                      interval=4, conv_k=4, d_state=128, n_group=16, dt_rank=32, std=0.02, name="qwen35-synthetic",
                      rope_base=1e7, layer_type=None):
    """A qwen35 (Gated DeltaNet + gated attention) model with the tensor set of a real Qwen3.5 file
    (test-fixtures/qwen35-4b-tensors.txt), tied output. types keys: embd, qkv, z, ab, ssm_out, q, k, v, o, gate, up,
    down; layer_type(l, key) may override a key's type per layer. Matrices are std * N(0, 1); the F32 vectors follow
    the reference's synthetic generator's ranges (tools/make-synth-qwen35.js:41-44): norms 1 + 0.05 N,
    ssm_a = -(0.7 + 0.1 N) < 0, dt bias 0.5 N, conv 0.3 N."""
    d_inner = dt_rank * d_state
    s = ModelSpec("qwen35", n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, vocab, ctx_train, rope_base=rope_base,
                  name=name, n_rot=n_rot, interval=interval, conv_k=conv_k, d_state=d_state, n_group=n_group,
                  dt_rank=dt_rank, d_inner=d_inner)
    qd, kvd = n_head * head_dim, n_head_kv * head_dim
    conv_dim = 2 * n_group * d_state + d_inner

    def mat(nm, key, rows, cols):
        ty = types[key]
        if layer_type and nm.startswith("blk."):
            ty = layer_type(int(nm.split(".")[1]), key) or ty
        s.tensors.append(TensorSpec(nm, ty, rows, cols, tensor_seed(seed, nm), std))

    def vec(nm, n, mean, sd, rows=1):
        s.tensors.append(TensorSpec(nm, gguf.F32, rows, n, tensor_seed(seed, nm), sd, fill=2, fill_value=mean))

    mat("token_embd.weight", "embd", vocab, n_embd)
    vec("output_norm.weight", n_embd, 1.0, 0.05)
    for l in range(n_layer):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", n_embd, 1.0, 0.05)
        vec(p + "post_attention_norm.weight", n_embd, 1.0, 0.05)
        if (l + 1) % interval != 0:
            mat(p + "attn_qkv.weight", "qkv", conv_dim, n_embd)
            mat(p + "attn_gate.weight", "z", d_inner, n_embd)
            mat(p + "ssm_alpha.weight", "ab", dt_rank, n_embd)
            mat(p + "ssm_beta.weight", "ab", dt_rank, n_embd)
            vec(p + "ssm_conv1d.weight", conv_k, 0.0, 0.3, rows=conv_dim)
            vec(p + "ssm_dt.bias", dt_rank, 0.0, 0.5)
            vec(p + "ssm_a", dt_rank, -0.7, 0.1)
            vec(p + "ssm_norm.weight", d_state, 1.0, 0.05)
            mat(p + "ssm_out.weight", "ssm_out", n_embd, d_inner)
        else:
            mat(p + "attn_q.weight", "q", 2 * qd, n_embd)
            mat(p + "attn_k.weight", "k", kvd, n_embd)
            mat(p + "attn_v.weight", "v", kvd, n_embd)
            mat(p + "attn_output.weight", "o", n_embd, qd)
            vec(p + "attn_q_norm.weight", head_dim, 1.0, 0.05)
            vec(p + "attn_k_norm.weight", head_dim, 1.0, 0.05)
        mat(p + "ffn_gate.weight", "gate", n_ff, n_embd)
        mat(p + "ffn_up.weight", "up", n_ff, n_embd)
        mat(p + "ffn_down.weight", "down", n_embd, n_ff)
    return s


# Q4_K_M mix of the real Qwen3.5-4B file (test-fixtures/qwen35-4b-tensors.txt): Q5_K attn_qkv and ssm_out, Q8_0 ssm_alpha
# and ssm_beta, Q6_K token_embd, attn_v and ffn_down, Q4_K elsewhere
QWEN35_Q4_K_M = dict(embd=gguf.Q6_K, qkv=gguf.Q5_K, z=gguf.Q4_K, ab=gguf.Q8_0, ssm_out=gguf.Q5_K, q=gguf.Q4_K,
                     k=gguf.Q4_K, v=gguf.Q6_K, o=gguf.Q4_K, gate=gguf.Q4_K, up=gguf.Q4_K, down=gguf.Q6_K)


def _use_more_bits(i, n):
    """llama.cpp's Q4_K_M rule for the layers that keep more bits: the first and last eighth, and every third between."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


# layers whose attn_v is Q6_K in the real Qwen3.5-4B-Q4_K_M file (the other attention layers: Q4_K)
QWEN35_4B_V_Q6K = {3, 7, 11, 15, 27}


def _qwen35_4b_layer_type(l, key):
    if key == "down":
        return gguf.Q6_K if _use_more_bits(l, 32) else gguf.Q4_K
    if key == "v":
        return gguf.Q6_K if l in QWEN35_4B_V_Q6K else gguf.Q4_K
    return None


def qwen35_types(t):
    return dict(embd=t, qkv=t, z=t, ab=t, ssm_out=t, q=t, k=t, v=t, o=t, gate=t, up=t, down=t)


def tiny_qwen35(seed=35, quant="q8_0", n_layer=4, interval=2):
    """Tiny qwen35 model for parity tests: d 256, 4 layers (DeltaNet, attention, DeltaNet, attention), 4/2 heads of
    64 with 32 rotary dims, FFN 512, vocab 2048, DeltaNet 2 key / 4 value heads of 64, conv kernel 4."""
    types = QWEN35_Q4_K_M if quant == "q4_k_m" else qwen35_types({"q8_0": gguf.Q8_0, "f32": gguf.F32}[quant])
    return build_qwen35_spec(256, n_layer, 4, 2, 64, 32, 512, 2048, 4096, types, seed, interval=interval, d_state=64,
                             n_group=2, dt_rank=4, name=f"tiny-qwen35-{quant}")


def qwen35_4b(seed=354, ctx_train=262144):
    """Qwen3.5-4B-shaped hybrid target with the real file's tensor set and Q4_K_M mix: 32 layers (every 4th gated
    attention), d 2560, 16/4 heads of 256 with 64 rotary dims, FFN 9216, vocab 248320, DeltaNet 16 key / 32 value heads
    of 128, conv kernel 4, tied output; ffn_down and attn_v types per layer as in the real file."""
    return build_qwen35_spec(2560, 32, 16, 4, 256, 64, 9216, 248320, ctx_train, QWEN35_Q4_K_M, seed,
                             name="qwen35-4b-shaped", layer_type=_qwen35_4b_layer_type)


def all_type(t):
    return dict(embd=t, output=t, q=t, k=t, v=t, o=t, gate=t, up=t, down=t)


# Q4_K_M mix as llama.cpp names it: Q6_K for attn_v, ffn_down and the output head, Q4_K elsewhere
# (the same rule as zerollm's generator, tools/make-tiny-gguf.js:71)
Q4_K_M = dict(embd=gguf.Q4_K, output=gguf.Q6_K, q=gguf.Q4_K, k=gguf.Q4_K, v=gguf.Q6_K, o=gguf.Q4_K, gate=gguf.Q4_K,
              up=gguf.Q4_K, down=gguf.Q6_K)


def tiny_pair(seed=1, draft_layers=2, quant=gguf.Q8_0, layer_std=None, n_embd=512):
    """Tiny qwen3 target (4 layers, d 512, 8/4 heads, hd 64, FFN 1536, vocab 32000, theta 1e6, all Q8_0, norms 1.0)
    and a draft made of its first 2 layers plus the same embedding / output head (same seed, so identical tensors).
    layer_std: see build_spec; n_embd: another model width (the heads stay 8 / 4 of 64)."""
    kw = dict(arch="qwen3", n_embd=n_embd, n_head=8, n_head_kv=4, head_dim=64, n_ff=1536, vocab=32000, ctx_train=2048,
              types=all_type(quant), seed=seed, layer_std=layer_std)
    return build_spec(n_layer=4, name="tiny-target", **kw), build_spec(n_layer=draft_layers, name="tiny-draft", **kw)


def qwen3_8b_pair(seed=8, draft_seed=6, ctx_train=32768):
    """Qwen3-8B-shaped Q4_K_M target and Qwen3-0.6B-shaped Q8_0 draft. The draft's embedding and output head are the
    target's N(0, 0.02) values restricted to the first 1024 input columns, quantised to Q8_0."""
    t = build_spec("qwen3", 4096, 36, 32, 8, 128, 12288, 151936, ctx_train, Q4_K_M, seed, name="qwen3-8b-shaped")
    d = build_spec("qwen3", 1024, 28, 16, 8, 128, 3072, 151936, ctx_train, all_type(gguf.Q8_0), draft_seed,
                   embd_from=(seed, 4096), name="qwen3-0.6b-shaped")
    return t, d


def qwen3_8b_close_pair(layer_std=0.0003, tail=0.01, seed=8, draft_seed=6, ctx_train=32768):
    """The headline pair's shapes, formats and bytes, made to agree: small per-layer matrices (layer_std) keep both
    residual streams close to the token embedding, and the target's output norm weighs the 3072 embedding columns its
    draft does not have by `tail` (1.0 on the first 1024), so the target's head mostly sees what the draft's head sees.
    The reference's generator builds agreeing pairs the same way, by damping what the draft lacks
    (tools/make-tiny-gguf.js:22-23, 80-81: fadeAfter / fade)."""
    t = build_spec("qwen3", 4096, 36, 32, 8, 128, 12288, 151936, ctx_train, Q4_K_M, seed, name="qwen3-8b-shaped-close",
                   layer_std=layer_std)
    for i, ts in enumerate(t.tensors):
        if ts.name == "output_norm.weight":
            t.tensors[i] = TensorSpec("output_norm.weight", gguf.F32, 1, 4096, std=tail, src_cols=1024, fill=3,
                                      fill_value=1.0)
    d = build_spec("qwen3", 1024, 28, 16, 8, 128, 3072, 151936, ctx_train, all_type(gguf.Q8_0), draft_seed,
                   embd_from=(seed, 4096), name="qwen3-0.6b-shaped-close", layer_std=layer_std)
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
    ]
    if spec.hybrid:
        meta[-3] = M(f"{a}.rope.dimension_count", U32, spec.n_rot)
        meta += [
            M(f"{a}.full_attention_interval", U32, spec.interval), M(f"{a}.ssm.conv_kernel", U32, spec.conv_k),
            M(f"{a}.ssm.state_size", U32, spec.d_state), M(f"{a}.ssm.group_count", U32, spec.n_group),
            M(f"{a}.ssm.time_step_rank", U32, spec.dt_rank), M(f"{a}.ssm.inner_size", U32, spec.d_inner),
        ]
    meta += [
        M("tokenizer.ggml.model", STR, "gpt2"),
        M("tokenizer.ggml.tokens", ARR, tokens, STR),
        M("tokenizer.ggml.token_type", ARR, [1] * spec.vocab, I32),
    ]
    tensors = [(t.name, t.dims, t.type, tensor_bytes(t, use_device)) for t in spec.tensors]
    gguf.write_gguf(path, meta, tensors)


def build_on_device(spec: ModelSpec, ctx=None, kv="f32", max_batch=16, logits_batch=None, **ck):
    """The model generated directly in HBM; ck: the hybrid checkpoint options of HipModel."""
    from .model import HipModel
    return HipModel.from_synth(spec.config(), [t.c() for t in spec.tensors], ctx=ctx, kv=kv, max_batch=max_batch,
                               logits_batch=logits_batch, **ck)
