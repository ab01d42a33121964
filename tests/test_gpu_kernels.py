"""GPU kernel parity through the C ABI: synthetic weights, repack + dequantisation, activation quantisation and the
GEMV family against the oracle (bit-exact where the reference's arithmetic allows it)."""
import base64
import ctypes as C
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from zerollm_amd import _lib, gguf as G, synth
from zerollm_amd._lib import call, ptr

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant-vectors.json")
QTYPES = [G.Q8_0, G.Q4_0, G.Q5_0, G.Q4_K, G.Q5_K, G.Q6_K]


class Mat:
    def __init__(self, type_, raw, rows, cols):
        self.h = C.c_void_p()
        raw = np.ascontiguousarray(raw, np.uint8)
        call("zl_mat_upload", type_, raw.ctypes.data_as(C.c_void_p), rows, cols, C.byref(self.h))
        self.rows, self.cols = rows, cols

    def dequant(self):
        out = np.zeros((self.rows, self.cols), np.float32)
        call("zl_mat_dequant", self.h, 0, self.rows, ptr(out, C.c_float))
        return out

    def gemv(self, X):
        X = np.ascontiguousarray(X, np.float32)
        M = X.shape[0]
        y = np.zeros((M, self.rows), np.float32)
        call("zl_mat_gemv", self.h, ptr(X, C.c_float), M, ptr(y, C.c_float))
        return y

    def free(self):
        call("zl_mat_free", self.h)


def rand_blocks(type_, rows, cols, seed):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=rows * G.row_size(type_, cols), dtype=np.uint8)
    _, bs, ts = G.TYPE_INFO[type_]
    blk = raw.reshape(-1, ts)
    f16 = lambda v: np.frombuffer(np.float16(v).tobytes(), np.uint8)
    for i in range(blk.shape[0]):
        d = 0.01 * (0.5 + rng.random())
        if type_ == G.Q6_K:
            blk[i, 208:210] = f16(d / 50)
        else:
            blk[i, 0:2] = f16(d)
            if type_ in (G.Q4_K, G.Q5_K):
                blk[i, 2:4] = f16(d * 2)
    return raw


@pytest.mark.parametrize("type_", [G.F32, G.Q8_0, G.Q4_0, G.Q5_0, G.Q4_K, G.Q5_K, G.Q6_K])
def test_device_synth_equals_host_synth(gpu, type_):
    t = synth.TensorSpec("x", type_, 37, 512, seed=1234567, std=0.02)
    a = synth.tensor_bytes(t, use_device=False)
    b = synth.tensor_bytes(t, use_device=True)
    assert (a == b).all()


@pytest.mark.parametrize("name", ["Q5_0", "Q4_K", "Q5_K", "Q6_K"])
def test_dequant_golden_vectors(gpu, name):
    v = json.load(open(GOLD))[name]
    raw = np.frombuffer(base64.b64decode(v["raw"]), np.uint8)
    t = {"Q5_0": G.Q5_0, "Q4_K": G.Q4_K, "Q5_K": G.Q5_K, "Q6_K": G.Q6_K}[name]
    m = Mat(t, raw, v["rows"], v["cols"])
    got = m.dequant()
    m.free()
    want = O.dequant(t, raw, v["rows"], v["cols"])
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), "repacked dequantisation must be bit-exact with the reference's"


@pytest.mark.parametrize("type_", QTYPES)
@pytest.mark.parametrize("cols", [256, 1024, 96])
def test_dequant_random_blocks_bit_exact(gpu, type_, cols):
    if cols % G.TYPE_INFO[type_][1]:
        pytest.skip("not a whole number of blocks")
    raw = rand_blocks(type_, 19, cols, 7)
    m = Mat(type_, raw, 19, cols)
    got = m.dequant()
    m.free()
    want = O.dequant(type_, raw, 19, cols)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


def test_quant_act_bit_exact(gpu):
    rng = np.random.default_rng(3)
    M, K = 5, 4096
    x = (rng.normal(0, 1, (M, K)) * rng.choice([1e-3, 1, 30], (M, K))).astype(np.float32)
    x[0, :32] = 0
    x[1, 32:64] = np.array([127] + [0.5, -0.5, 1.5, -1.5, 2.5, -2.5] + [0] * 25, np.float32)
    q = np.zeros((M, K), np.int8)
    d = np.zeros((M, K // 32), np.float32)
    s = np.zeros((M, K // 32), np.int32)
    call("zl_quant_act", ptr(x, C.c_float), K, M, ptr(q, C.c_int8), ptr(d, C.c_float), ptr(s, C.c_int32))
    for t in range(M):
        wq, wd, ws = O.quantize_act(x[t])
        assert (q[t] == wq).all() and (d[t].view(np.uint32) == wd.view(np.uint32)).all() and (s[t] == ws).all()


def _check_gemv(type_, rows, cols, Ms, seed, raw=None):
    raw = rand_blocks(type_, rows, cols, seed) if raw is None else raw
    m = Mat(type_, raw, rows, cols)
    rng = np.random.default_rng(seed + 1)
    X = rng.normal(0, 1, (max(Ms), cols)).astype(np.float32)
    want = np.stack([O.matvec(type_, raw, rows, cols, X[t]) for t in range(max(Ms))])
    ys = {}
    for M in Ms:
        y = m.gemv(X[:M])
        ys[M] = y
        exact = (y.view(np.uint32) == want[:M].view(np.uint32)).mean()
        rel = np.abs(y - want[:M]).max() / (np.abs(want[:M]).max() + 1e-30)
        # f64 combine in a different summation order than the reference: bit-identical f32 results except for rare
        # last-place rounding differences
        assert exact >= 0.999, (M, exact)
        assert rel <= 1e-6, (M, rel)
    m.free()
    # batched == token by token, bit for bit (the per-(row, token) arithmetic does not depend on M)
    one = ys[min(Ms)]
    for M in Ms:
        assert (ys[M][:min(Ms)].view(np.uint32) == one.view(np.uint32)).all()
    return ys


@pytest.mark.parametrize("type_", QTYPES)
@pytest.mark.parametrize("cols", [512, 1024, 1536, 4096])
def test_gemv_matches_oracle(gpu, type_, cols):
    """1..9 tokens on the GEMV kernels, 10..64 on the GEMM (Q8_0, Q4_K, Q5_K, Q6_K: one launch of up to 64 tokens by
    default); every token's row equals its single-token row bit for bit and the oracle's."""
    if cols % G.TYPE_INFO[type_][1]:
        pytest.skip("not a whole number of blocks")
    _check_gemv(type_, 300, cols, [1, 2, 5, 9, 16, 17, 32, 33, 64], seed=cols + type_)


@pytest.mark.parametrize("maxm", ["64", "48", "16", "0"])
@pytest.mark.parametrize("type_", [G.Q8_0, G.Q4_K, G.Q5_K, G.Q6_K])
def test_gemm_launch_widths_give_the_same_bits(gpu, monkeypatch, type_, maxm):
    """The GEMM at every token-group count (ZEROLLM_GEMM_MAXM = 64: one launch of 64 tokens, four groups of 16; 48:
    three groups; 16: one; 0: the GEMV kernels alone) gives the rows of single-token launches bit for bit, and the
    oracle's."""
    monkeypatch.setenv("ZEROLLM_GEMM_MAXM", maxm)
    print(f"case gemm width {maxm} type {type_}", flush=True)
    _check_gemv(type_, 200, 2048, [1, 10, 16, 31, 48, 64], seed=7 + type_)


def float_raw(type_, rows, cols, seed):
    """Raw F32 / F16 / BF16 rows of N(0, 0.05) values (BF16: the top half of the f32 bits, as ggml truncates)."""
    w = np.random.default_rng(seed).normal(0, 0.05, (rows, cols)).astype(np.float32)
    if type_ == G.F32:
        return w.view(np.uint8).ravel()
    if type_ == G.F16:
        return w.astype(np.float16).view(np.uint8).ravel()
    return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).ravel()


@pytest.mark.parametrize("type_", [G.F32, G.F16, G.BF16])
@pytest.mark.parametrize("cols", [512, 1536])
def test_gemv_float_weights_match_oracle(gpu, type_, cols):
    """Float weights take the f32 activations, not their int8 quantisation (src/compute/ref-kernels.js:278-299)."""
    _check_gemv(type_, 200, cols, [1, 2, 5, 9, 17], seed=cols + type_, raw=float_raw(type_, 200, cols, cols + type_))


@pytest.mark.parametrize("type_", [G.Q8_0, G.Q4_0, G.Q5_0])
def test_gemv_odd_block_count(gpu, type_):
    """cols = 96: the last 64-value slab is half padding."""
    _check_gemv(type_, 70, 96, [1, 3, 8], seed=5)


def test_gemv_batched_rows_equal_single_token(gpu):
    raw = rand_blocks(G.Q4_K, 1024, 4096, 11)
    m = Mat(G.Q4_K, raw, 1024, 4096)
    X = np.random.default_rng(2).normal(0, 1, (17, 4096)).astype(np.float32)
    full = m.gemv(X)
    for t in (0, 4, 9, 16):
        single = m.gemv(X[t:t + 1])
        assert (single[0].view(np.uint32) == full[t].view(np.uint32)).all()
    m.free()


# the verify-width microbenchmark's projection shapes (Qwen3-8B): attn_q / attn_output, attn_k, attn_v, ffn_gate /
# ffn_up, ffn_down, the output head
C2_SHAPES = [(4096, 4096, G.Q4_K), (1024, 4096, G.Q4_K), (1024, 4096, G.Q6_K), (12288, 4096, G.Q4_K),
             (4096, 12288, G.Q6_K), (151936, 4096, G.Q6_K)]


@pytest.mark.parametrize("N,K,type_", C2_SHAPES)
def test_gemv_projection_shapes_synthetic(gpu, N, K, type_):
    """Projection shapes with this library's quantised N(0, 0.02) weights, at M = k + 1 in {1, 2, 5, 9, 17} and the
    prefill chunks M = 16, 32, 64: the first and the last 96 rows against the oracle, every M's first row equal to the
    single-token row bit for bit (M = 16, 17, 32 and 64 are one GEMM launch each; the other rows are covered by the same
    kernels through the model tests)."""
    t = synth.TensorSpec("w", type_, N, K, seed=99 + N, std=0.02)
    raw = synth.tensor_bytes(t, use_device=True)
    print(f"case gemv {N}x{K} type {type_}", flush=True)
    m = Mat(type_, raw, N, K)
    X = np.random.default_rng(N).normal(0, 1, (64, K)).astype(np.float32)
    rows = 96
    rb = G.row_size(type_, K)
    heads = [(0, raw[:rows * rb]), (N - rows, raw[(N - rows) * rb:])]
    want = {r0: np.stack([O.matvec(type_, sub, rows, K, X[i]) for i in range(64)]) for r0, sub in heads}
    for M in (1, 2, 5, 9, 16, 17, 32, 64):
        y = m.gemv(X[:M])
        for r0, _ in heads:
            got, w = y[:, r0:r0 + rows], want[r0][:M]
            assert (got.view(np.uint32) == w.view(np.uint32)).mean() >= 0.999, (M, r0)
            assert np.abs(got - w).max() <= 1e-6 * np.abs(w).max(), (M, r0)
        if M > 1:
            assert (y[:1].view(np.uint32) == first.view(np.uint32)).all(), M
        else:
            first = y[:1].copy()
    m.free()
