"""CPU tests of the host side: the C-ABI library loads and exports every symbol the header declares (no compute calls
without a GPU), the GGUF reader/writer round trip, and the synthetic generator and quantisers."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle import oracle as O
from zerollm_amd import _lib, gguf as G, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "zerollm_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(zl_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = C.CDLL(_lib.LIB_PATH)
    names = header_functions()
    assert len(names) >= 30
    for n in names:
        assert hasattr(L, n), n
    # and the Python binding covers them all
    bound = {s[0] for s in _lib.SIGNATURES}
    assert set(names) <= bound, set(names) - bound


def test_errors_without_gpu_are_reported_not_crashing():
    """A bad path fails with a status code and a message (no GPU is touched before the file is parsed)."""
    h = C.c_void_p()
    o = _lib.zl_model_opts()
    rc = _lib.lib().zl_model_load(b"/nonexistent/x.gguf", C.byref(o), C.byref(h))
    assert rc != 0
    assert _lib.lib().zl_last_error()


@pytest.mark.parametrize("opts,msg", [
    (dict(top_k=40, repeat_last_n=65), "repeat_last_n must be 0..64 on the GPU sampler"),
])
def test_sampler_options_the_device_does_not_take_are_refused(opts, msg):
    """A repetition window above the device history's 64 ids is refused with a message before any device call
    (every topK is taken: 0 and values above 256 keep full candidate lists)."""
    o = _lib.zl_sampler_opts(temperature=0.8, top_p=0.95, min_p=0.0, repeat_penalty=1.0, presence_penalty=0.0,
                             frequency_penalty=0.0, top_k=opts["top_k"], repeat_last_n=opts.get("repeat_last_n", 64),
                             seed=1, greedy_argmax=0)
    h = C.c_void_p()
    rc = _lib.lib().zl_sampler_create(C.byref(o), C.byref(h))
    assert rc != 0
    assert msg in _lib.lib().zl_last_error().decode()


def test_gguf_round_trip(tmp_path):
    M = G.MetaKV
    meta = [M("general.architecture", G.STRING, "qwen3"), M("qwen3.block_count", G.UINT32, 2),
            M("qwen3.attention.layer_norm_rms_epsilon", G.FLOAT32, 1e-6), M("x.arr", G.ARRAY, [1, 2, 3], G.INT32),
            M("x.strs", G.ARRAY, ["a", "bc"], G.STRING), M("x.b", G.BOOL, True), M("x.f64", G.FLOAT64, 0.125)]
    a = np.arange(64, dtype=np.float32)
    b = np.arange(34 * 4, dtype=np.uint8)
    p = str(tmp_path / "t.gguf")
    G.write_gguf(p, meta, [("a", [64], G.F32, a), ("b", [128], G.Q8_0, b)], alignment=64)
    g = G.read_gguf(p)
    assert g.get("general.architecture") == "qwen3" and g.get("qwen3.block_count") == 2
    assert g.get("qwen3.attention.layer_norm_rms_epsilon") == float(np.float32(1e-6))
    assert g.get("x.arr") == [1, 2, 3] and g.get("x.strs") == ["a", "bc"] and g.get("x.b") is True
    assert g.alignment == 64 and g.data_start % 64 == 0
    assert (g.floats("a") == a).all() and (np.asarray(g.data("b")) == b).all()
    assert g.tensor("b").abs_offset % 64 == 0


def test_gguf_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGML" + b"\0" * 20)
    with pytest.raises(ValueError, match="not a GGUF file"):
        G.read_gguf(str(p))
    p.write_bytes(b"GGUF" + (3).to_bytes(4, "little") + (1).to_bytes(8, "little") + (0).to_bytes(8, "little"))
    with pytest.raises(ValueError):
        G.read_gguf(str(p))


def test_synth_is_deterministic_and_normal():
    t = synth.TensorSpec("w", G.F32, 64, 1024, seed=42, std=1.0)
    a = synth.tensor_bytes(t).view(np.float32)
    b = synth.tensor_bytes(t).view(np.float32)
    assert (a == b).all()
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1) < 0.02
    # kurtosis of a normal is 3; tails present
    k = ((a - a.mean()) ** 4).mean() / a.var() ** 2
    assert abs(k - 3) < 0.15 and np.abs(a).max() > 3.5
    # a column window of a wider tensor takes the same deviates
    w = synth.TensorSpec("w", G.F32, 64, 256, seed=42, std=1.0, src_cols=1024, col0=0)
    assert (synth.tensor_bytes(w).view(np.float32).reshape(64, 256) == a.reshape(64, 1024)[:, :256]).all()


@pytest.mark.parametrize("type_,tol", [(G.Q8_0, 0.51 / 127), (G.Q4_K, 1.02 / 15), (G.Q5_K, 1.02 / 31), (G.Q6_K, 1.01 / 32),
                                       (G.Q5_0, 1.01 / 16), (G.Q4_0, 1.01 / 8)])
def test_quantisers_round_trip(type_, tol):
    """The library's quantisers against the oracle's dequantisation of what they write: error within half a step
    (the K-quant affine step is range/qmax with range <= 2*amax; Q4_0/Q5_0/Q6_K map +max exactly and clamp -max)."""
    rows, cols = 16, 512
    f = synth.TensorSpec("w", G.F32, rows, cols, seed=7, std=0.02)
    x = synth.tensor_bytes(f).view(np.float32).reshape(rows, cols)
    q = synth.TensorSpec("w", type_, rows, cols, seed=7, std=0.02)
    y = O.dequant(type_, synth.tensor_bytes(q), rows, cols)
    amax = np.abs(x).max()
    assert np.abs(x - y).max() <= tol * amax * 1.05 + 1e-6, np.abs(x - y).max() / amax
    if type_ == G.Q8_0:
        # Q8_0 follows the reference's quantizeQ8_0 exactly
        assert (synth.tensor_bytes(q) == O.quantize_q8_0(x.reshape(-1))).all()
    if type_ == G.Q4_0:
        assert (synth.tensor_bytes(q) == O.quantize_q4_0(x.reshape(-1))).all()


def test_named_configs():
    t, d = synth.tiny_pair()
    assert t.weight_bytes == 30777344 and d.weight_bytes == 24092672
    names_t = {x.name: x for x in t.tensors}
    names_d = {x.name: x for x in d.tensors}
    # the tiny draft is the target's first 2 layers and the same head: identical tensor specs
    for n, x in names_d.items():
        assert names_t[n] == x
    T, D = synth.qwen3_8b_pair()
    assert T.weight_bytes == 4923568128 and D.weight_bytes == 633233408
    e_t = {x.name: x for x in T.tensors}["output.weight"]
    e_d = {x.name: x for x in D.tensors}["output.weight"]
    assert e_d.seed == e_t.seed and e_d.src_cols == 4096 and e_d.cols == 1024 and e_d.type == G.Q8_0


def test_seeded_ids_are_mulberry32_prompts():
    """The package's seeded prompt ids equal floor(mulberry32(seed)() * vocab) of the oracle's restatement."""
    from oracle import oracle as O
    from zerollm_amd import synth

    r = O.Rng(2024)
    assert synth.seeded_ids(300, 2024, 151936) == [int(r() * 151936) for _ in range(300)]


class _Meta:
    """The get() view of GGUF metadata that vocabFingerprint reads."""

    def __init__(self, tokens, types, arch="qwen3", vocab=None):
        self.m = {"tokenizer.ggml.tokens": tokens, "tokenizer.ggml.token_type": types, "general.architecture": arch}
        if vocab is not None:
            self.m[f"{arch}.vocab_size"] = vocab

    def get(self, k, default=None):
        return self.m.get(k, default)


def test_vocab_fingerprint_and_mismatch_messages():
    """vocabFingerprint / vocabMismatch (src/model/speculative.js:256-283): sha256 over each token string and a NUL,
    then '#<n types>:' and '<type>,' per token; the three mismatch messages, token strings quoted as JSON."""
    import hashlib

    from zerollm_amd.speculative import vocab_fingerprint, vocab_mismatch

    a = _Meta(["a", "b"], [1, 1])
    fp = vocab_fingerprint(a)
    assert fp == {"size": 2, "hash": hashlib.sha256(b"a\0b\0#2:1,1,").hexdigest()}
    assert vocab_mismatch(a, _Meta(["a", "b"], [1, 1])) is None
    assert vocab_mismatch(a, _Meta(["a"], [1])) == (
        "the draft model has a vocabulary of 1 tokens but the target has 2: speculative decoding needs two models of "
        "the same family with the same tokenizer (e.g. Qwen3-0.6B for Qwen3-8B)")
    assert vocab_mismatch(a, _Meta(["a", "cé"], [1, 1])) == (
        "the draft model's tokenizer differs from the target's (first difference at token id 1: \"b\" vs \"cé\"): "
        "speculative decoding needs the same vocabulary")
    assert vocab_mismatch(a, _Meta(["a", "b"], [1, 3])) == (
        "the draft model's tokenizer differs from the target's (the token types differ): speculative decoding needs "
        "the same vocabulary")
    assert vocab_mismatch(_Meta(["a", "b"], [1, 1], vocab=2), _Meta(["a", "b"], [1, 1], vocab=3)) == \
        "the models disagree on the logits vocabulary size (2 vs 3)"


def test_synthetic_pair_files_share_a_vocabulary(tmp_path):
    from zerollm_amd.speculative import vocab_mismatch

    t, d = synth.tiny_pair()
    tp, dp = str(tmp_path / "t.gguf"), str(tmp_path / "d.gguf")
    synth.write_gguf(tp, t)
    synth.write_gguf(dp, d)
    assert vocab_mismatch(G.read_gguf(tp), G.read_gguf(dp)) is None
