"""The no-allocation GEMV entry point (zl_mat_gemv_noalloc: static device work space, device inputs and outputs)
against zl_mat_gemv on the same matrices and rows: the same kernels, so the same bits. Two calls in a row, the second
with a smaller input, then a call on a caller's stream, and the size limits."""
import ctypes as C

import numpy as np
import pytest

from zerollm_amd import _lib, gguf as G
from zerollm_amd._lib import call, ptr

pytestmark = pytest.mark.gpu


class Hip:
    """Device buffers from the HIP runtime the library itself links (libamdhip64.so.7), for this test only."""

    H2D, D2H = 1, 2

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so.7")
        self.L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.L.hipFree.argtypes = [C.c_void_p]
        self.L.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.L.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.L.hipStreamDestroy.argtypes = [C.c_void_p]

    def ok(self, rc):
        assert rc == 0, f"HIP error {rc}"

    def upload(self, a):
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        self.ok(self.L.hipMalloc(C.byref(p), a.nbytes))
        self.ok(self.L.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), a.nbytes, self.H2D))
        return p

    def alloc(self, nbytes):
        p = C.c_void_p()
        self.ok(self.L.hipMalloc(C.byref(p), nbytes))
        return p

    def download(self, p, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        self.ok(self.L.hipMemcpy(out.ctypes.data_as(C.c_void_p), p, out.nbytes, self.D2H))
        return out

    def free(self, p):
        self.ok(self.L.hipFree(p))


def synth_mat(type_, rows, cols, seed):
    h = C.c_void_p()
    call("zl_mat_synth", type_, rows, cols, seed, 0.02, 1, C.byref(h))
    return h


def gemv_alloc(h, X, rows):
    y = np.zeros((X.shape[0], rows), np.float32)
    call("zl_mat_gemv", h, ptr(X, C.c_float), X.shape[0], ptr(y, C.c_float))
    return y


def gemv_noalloc(hip, h, X, rows, stream=None):
    dx = hip.upload(X)
    dy = hip.alloc(X.shape[0] * rows * 4)
    call("zl_mat_gemv_noalloc", h, dx, X.shape[0], dy, stream)
    if stream is not None:
        hip.ok(hip.L.hipStreamSynchronize(stream))
    y = hip.download(dy, (X.shape[0], rows))
    hip.free(dx)
    hip.free(dy)
    return y


def test_noalloc_gemv_equals_gemv_two_calls_then_a_caller_stream(gpu):
    hip = Hip()
    rng = np.random.default_rng(5)
    # 1: ffn_down shape, Q6_K, 16 tokens (two token chunks, split-K partials and counters in the static array)
    a = synth_mat(G.Q6_K, 4096, 12288, 71)
    Xa = rng.normal(0, 1, (16, 12288)).astype(np.float32)
    print("case noalloc Q6_K 4096x12288 M=16", flush=True)
    ya = gemv_noalloc(hip, a, Xa, 4096)
    assert (ya.view(np.uint32) == gemv_alloc(a, Xa, 4096).view(np.uint32)).all()
    # 2: a smaller input right after: attn_k shape, Q4_K, 5 tokens (the matrix-core path)
    b = synth_mat(G.Q4_K, 1024, 4096, 72)
    Xb = rng.normal(0, 1, (5, 4096)).astype(np.float32)
    print("case noalloc Q4_K 1024x4096 M=5", flush=True)
    yb = gemv_noalloc(hip, b, Xb, 1024)
    assert (yb.view(np.uint32) == gemv_alloc(b, Xb, 1024).view(np.uint32)).all()
    # 3: the first matrix again with 3 tokens, enqueued on the caller's stream
    s = C.c_void_p()
    hip.ok(hip.L.hipStreamCreate(C.byref(s)))
    print("case noalloc Q6_K M=3 on a caller stream", flush=True)
    yc = gemv_noalloc(hip, a, Xa[:3], 4096, stream=s)
    hip.ok(hip.L.hipStreamDestroy(s))
    assert (yc.view(np.uint32) == ya[:3].view(np.uint32)).all()
    call("zl_mat_free", a)
    call("zl_mat_free", b)


def test_noalloc_gemv_float_and_q8_rows(gpu):
    """Float weights read the f32 copy of the rows from the static array; Q8_0 single-token rows."""
    hip = Hip()
    rng = np.random.default_rng(6)
    for type_, rows, cols, M in ((G.Q8_0, 3072, 1024, 1), (G.F32, 300, 512, 4)):
        if type_ == G.F32:
            w = rng.normal(0, 0.05, (rows, cols)).astype(np.float32)
            h = C.c_void_p()
            call("zl_mat_upload", type_, w.ctypes.data_as(C.c_void_p), rows, cols, C.byref(h))
        else:
            h = synth_mat(type_, rows, cols, 73)
        X = rng.normal(0, 1, (M, cols)).astype(np.float32)
        print(f"case noalloc type {type_} {rows}x{cols} M={M}", flush=True)
        y = gemv_noalloc(hip, h, X, rows)
        assert (y.view(np.uint32) == gemv_alloc(h, X, rows).view(np.uint32)).all()
        call("zl_mat_free", h)


def test_noalloc_gemv_rejects_sizes_beyond_the_static_array(gpu):
    h = synth_mat(G.Q8_0, 64, 512, 74)
    dummy = C.c_void_p(16)  # never dereferenced: the size check fails first
    with pytest.raises(_lib.ZLError, match="at most 16 tokens of at most 16384 values"):
        call("zl_mat_gemv_noalloc", h, dummy, 17, dummy, None)
    call("zl_mat_free", h)
    w = synth_mat(G.Q8_0, 64, 16384 + 64, 75)
    with pytest.raises(_lib.ZLError, match="at most 16 tokens of at most 16384 values"):
        call("zl_mat_gemv_noalloc", w, dummy, 1, dummy, None)
    call("zl_mat_free", w)
