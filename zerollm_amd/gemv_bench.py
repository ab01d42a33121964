"""Verify-width k-quant GEMV microbenchmark at Qwen3-8B projection shapes (zerollm's tools/kbench.mjs plays this role for
the WASM kernels).

For each N x K matrix (Q4_K: attn_q/o, attn_k, ffn_gate/up; Q6_K: attn_v, ffn_down, output head) and M tokens, distinct
synthetic copies of the matrix totalling at least 512 MB (beyond the 256 MB MALL) are built in HBM, and `iters` launches
cycle through them, timed with HIP events on the library's stream. Reports weight GB/s (GGUF block bytes / time) and
the fraction of the 8 TB/s HBM peak. Activations are device-resident.

    python -m zerollm_amd.gemv_bench [--m 1,2,5,9,17] [--shapes all|name,...] [--min-mb 512] [--json out.json]
                                     [--iters N] [--copy-mb MB]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import sys

from . import _lib
from .gguf import Q4_K, Q6_K, Q8_0, row_size

HBM_PEAK = 8.0e12

# (name, type, N rows, K cols)
SHAPES = [
    ("q_o_4096x4096_q4k", Q4_K, 4096, 4096),
    ("k_1024x4096_q4k", Q4_K, 1024, 4096),
    ("v_1024x4096_q6k", Q6_K, 1024, 4096),
    ("gate_up_12288x4096_q4k", Q4_K, 12288, 4096),
    ("down_4096x12288_q6k", Q6_K, 4096, 12288),
    ("output_151936x4096_q6k", Q6_K, 151936, 4096),
    ("draft_qkv_4096x1024_q8_0", Q8_0, 4096, 1024),
    ("draft_gate_up_6144x1024_q8_0", Q8_0, 6144, 1024),
    ("draft_down_1024x3072_q8_0", Q8_0, 1024, 3072),
]


def weight_bytes(t, rows, cols):
    return rows * row_size(t, cols)


def copy_calibration(mb):
    """A kernel of known traffic, against which FETCH_SIZE / WRITE_SIZE counter readings are scaled: through the HIP
    runtime the library links (libamdhip64), hipMemset writes `mb` MiB (the runtime's fill kernel) and a
    device-to-device hipMemcpy then reads `mb` MiB and writes `mb` MiB (the runtime's copy kernel)."""
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hip.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipFree.argtypes = [C.c_void_p]
    n = mb << 20
    a, b = C.c_void_p(), C.c_void_p()
    for rc in (hip.hipMalloc(C.byref(a), n), hip.hipMalloc(C.byref(b), n), hip.hipMemset(a, 1, n),
               hip.hipMemcpy(b, a, n, 3), hip.hipDeviceSynchronize(), hip.hipFree(a), hip.hipFree(b)):
        if rc != 0:
            raise RuntimeError(f"copy calibration: HIP error {rc}")
    print(f"copy calibration: fill of {n} B written, then a copy of {n} B read and {n} B written", flush=True)


def run(shapes, ms_list, min_mb=512, target_ms=40.0, seed=7, iters=None):
    _lib.call("zl_init", 0)
    results = []
    for name, t, n, k in shapes:
        wb = weight_bytes(t, n, k)
        copies = max(1, -(-min_mb * 1024 * 1024 // wb))
        h = C.c_void_p()
        _lib.call("zl_mat_synth", t, n, k, seed, 0.02, copies, C.byref(h))
        try:
            for m in ms_list:
                ms = C.c_float()
                if iters is None:
                    _lib.call("zl_mat_gemv_time", h, m, max(8, copies), C.byref(ms))  # warm-up and estimate
                    n_it = min(2000, max(copies, int(target_ms / max(ms.value, 1e-4))))
                else:
                    n_it = iters
                _lib.call("zl_mat_gemv_time", h, m, n_it, C.byref(ms))
                gbs = wb / (ms.value * 1e-3) / 1e9
                r = {"shape": name, "type": {Q4_K: "Q4_K", Q6_K: "Q6_K", Q8_0: "Q8_0"}[t], "N": n, "K": k, "M": m,
                     "weight_bytes": wb, "copies": copies, "iters": n_it, "us": round(ms.value * 1e3, 2),
                     "GBps": round(gbs, 1), "frac_hbm": round(gbs * 1e9 / HBM_PEAK, 4)}
                results.append(r)
                print(f"{name:30s} M={m:2d}  {r['us']:9.2f} us  {gbs:8.1f} GB/s  {100 * r['frac_hbm']:5.1f}% of HBM peak",
                      flush=True)
        finally:
            _lib.call("zl_mat_free", h)
    return results


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--m", default="1,2,5,9,17")
    ap.add_argument("--shapes", default="all")
    ap.add_argument("--min-mb", type=int, default=512)
    ap.add_argument("--json", default=None)
    ap.add_argument("--iters", type=int, default=None,
                    help="timed launches per shape and M (default: about 40 ms worth); every call first launches each "
                         "copy once eagerly, cache-cold, which is what counter runs read")
    ap.add_argument("--copy-mb", type=int, default=0, help="first run a plain copy of this many MiB (counter scaling)")
    a = ap.parse_args(argv)
    if a.copy_mb:
        copy_calibration(a.copy_mb)
    ms_list = [int(x) for x in a.m.split(",")]
    shapes = SHAPES if a.shapes == "all" else [s for s in SHAPES if s[0] in a.shapes.split(",")]
    res = run(shapes, ms_list, a.min_mb, iters=a.iters)
    if a.json:
        with open(a.json, "w") as f:
            json.dump(res, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
