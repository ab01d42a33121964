"""Hybrid (qwen35) verify-window benchmark: a Qwen3.5-4B-shaped Q4_K_M target (Gated DeltaNet + gated attention, the real
file's tensor set) in HBM, a seeded 2048-token prefix prefilled, then cycles of the speculative-decoding target side:
markRollback (recurrent-state snapshot), one 5-token verify pass with logits for every row, and truncate to the accepted
length, as generateSpeculative drives a hybrid target (src/model/speculative.js:185, 226; src/compute/pool.js:269,
278-294). The verify pass captures the recurrent state after each of its tokens, so the truncate copies the captured
state where the reference restores the snapshot and replays the accepted tokens (ZEROLLM_STATE_CAPTURE=0: restore +
replay).

Checks on the way (size-independent, exact): the verify rows equal five single-token passes, and a model rolled back to
the accepted length holds the same recurrent state as one that only ran those tokens. Prints one JSON line.

    python -m zerollm_amd.hybrid_bench [--prefix 2048] [--cycles 20] [--accept 2]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import sys
import time

import numpy as np

from . import model as M
from . import synth
from ._lib import call

HBM_PEAK = 8.0e12


def sync(m):
    buf = np.empty(m.cfg["vocabSize"], np.float32)
    call("zl_model_logits", m._h, 0, 1, buf.ctypes.data_as(C.POINTER(C.c_float)))


def prefill(m, ids, logits_last=True):
    for i in range(0, len(ids), m.max_batch):
        chunk = ids[i:i + m.max_batch]
        last = i + m.max_batch >= len(ids)
        m.forward_batch(chunk, logits="last" if (last and logits_last) else "none", copy=False)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--prefix", type=int, default=2048)
    ap.add_argument("--cycles", type=int, default=20)
    ap.add_argument("--accept", type=int, default=2, help="drafts accepted per cycle (the rest rolled back)")
    ap.add_argument("--k", type=int, default=4)
    a = ap.parse_args(argv)
    M.init(0)
    spec = synth.qwen35_4b()
    B = a.k + 1
    t0 = time.perf_counter()
    m = synth.build_on_device(spec, ctx=a.prefix + 2 * B * (a.cycles + 4), kv="f16")
    print(f"model built in HBM in {time.perf_counter() - t0:.1f}s: {m.weight_bytes / 1e9:.3f} GB/pass, recurrent state "
          f"{m.state_bytes / 1e6:.1f} MB", file=sys.stderr, flush=True)
    prefix = synth.seeded_ids(a.prefix, 3535, spec.vocab)
    t0 = time.perf_counter()
    prefill(m, prefix)
    sync(m)
    print(f"prefill {a.prefix} tokens: {time.perf_counter() - t0:.2f}s, checkpoints {m.checkpoint_positions}",
          file=sys.stderr, flush=True)

    # exact checks at the full shapes
    ver = synth.seeded_ids(B, 77, spec.vocab)
    m.mark_rollback()
    rows = m.forward_batch(ver, logits="all").copy()
    state_after_verify = m.recurrent_state()
    m.truncate(a.prefix)
    seq = np.stack([m.forward(t).copy() for t in ver])
    batched_equals_sequential = bool((rows.view(np.uint32) == seq.view(np.uint32)).all())
    st = m.recurrent_state()
    state_equal = bool((st[0] == state_after_verify[0]).all() and (st[1] == state_after_verify[1]).all())
    m.truncate(a.prefix + a.accept)
    rolled = m.recurrent_state()
    ref = synth.build_on_device(spec, ctx=a.prefix + 2 * B, kv="f16")
    prefill(ref, prefix + ver[:a.accept], logits_last=False)
    rs = ref.recurrent_state()
    rollback_exact = bool((rolled[0] == rs[0]).all() and (rolled[1] == rs[1]).all())
    ref.close()
    m.truncate(a.prefix)
    print(f"checks: batched==sequential {batched_equals_sequential}, state {state_equal}, rollback {rollback_exact}",
          file=sys.stderr, flush=True)

    # timed (a): verify pass + return to the rollback snapshot (a 5-token pass, then one state copy of state_bytes)
    P = a.prefix
    for _ in range(3):
        m.forward_batch(ver, logits="all", copy=False)
        m.truncate(P)
    sync(m)
    t0 = time.perf_counter()
    for _ in range(a.cycles):
        m.forward_batch(ver, logits="all", copy=False)
        m.truncate(P)
    sync(m)
    verify_ms = (time.perf_counter() - t0) * 1e3 / a.cycles
    # timed (b): whole target-side cycles as generateSpeculative drives a hybrid target: markRollback (snapshot), verify,
    # truncate to the accepted length (the captured state, or restore + replay of the accepted tokens; a checkpoint there)
    t0 = time.perf_counter()
    for c in range(a.cycles):
        m.mark_rollback()
        m.forward_batch(synth.seeded_ids(B, 1000 + c, spec.vocab), logits="all", copy=False)
        m.truncate(m.pos - B + a.accept)
    sync(m)
    cycle_ms = (time.perf_counter() - t0) * 1e3 / a.cycles
    wb = m.weight_bytes
    line = {
        "metric": "qwen35 hybrid verify window: 5-token verify pass ms and weight-stream fraction of HBM peak",
        "workload": f"Qwen3.5-4B-shaped Q4_K_M hybrid (32 layers: 24 Gated DeltaNet, 8 gated attention; d 2560; vocab "
                    f"248320 tied), {a.prefix}-token seeded prefix, f16 KV, verify width {B}",
        "verify_ms": round(verify_ms, 3), "weight_bytes_per_pass": wb,
        "verify_weight_GBps": round(wb / (verify_ms * 1e-3) / 1e9, 1),
        "verify_frac_hbm": round(wb / (verify_ms * 1e-3) / HBM_PEAK, 4),
        "note_verify": "includes one device copy of the recurrent state (restore from the rollback snapshot)",
        "cycle_ms": round(cycle_ms, 3), "accepted_per_cycle": a.accept,
        "note_cycle": ("markRollback snapshot + verify pass (capturing the state after each token) + copy of the captured "
                       "state at the accepted length + checkpoint" if m.captures else
                       "markRollback snapshot + verify pass + restore + replay pass of the accepted tokens + checkpoint"),
        "state_bytes": m.state_bytes, "checks": {"batched_equals_sequential": batched_equals_sequential,
                                                 "verify_state_equals_sequential": state_equal,
                                                 "rollback_equals_fresh": rollback_exact},
    }
    m.close()
    print(json.dumps(line), flush=True)
    return 0 if (batched_equals_sequential and state_equal and rollback_exact) else 1


if __name__ == "__main__":
    sys.exit(main())
