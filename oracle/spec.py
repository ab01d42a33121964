"""ORACLE — test infrastructure only. generateSpeculative (src/model/speculative.js:100-240) over oracle models, greedy:
the draft proposes k tokens one forward at a time, the target checks them one forward at a time (RefModel has no
batched pass: forwardRows falls back to sequential forwards, src/model/speculative.js:42-47). Used as the CPU baseline
leg of bench.py and as a reference stream in tests."""
from __future__ import annotations

import time

import numpy as np


def common_prefix(a, b):
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


def speculative_greedy(target, draft, seq, k, max_tokens, deadline=None):
    """Continue `seq` (its last token pending; both models hold seq[:-1]) by up to max_tokens greedy tokens.
    Returns (emitted, cycles). Stops early at `deadline` (time.perf_counter value) after a whole cycle."""
    seq = list(seq)
    out = []
    cycles = 0
    while len(out) < max_tokens:
        if deadline is not None and time.perf_counter() > deadline:
            break
        kk = max(0, min(k, max_tokens - len(out) - 1))
        draft.truncate(min(common_prefix(draft.tokens, seq), len(seq) - 1))
        drafted = []
        if kk:
            logits = None
            for t in seq[draft.pos:]:
                logits = draft.forward(t)
            for j in range(kk):
                x = int(np.argmax(logits))
                drafted.append(x)
                if j == kk - 1:
                    break
                logits = draft.forward(x)
        rows = [target.forward(t) for t in [seq[-1]] + drafted]
        a = 0
        tok = -1
        for j in range(len(drafted)):
            t = int(np.argmax(rows[j]))
            if t == drafted[j]:
                a += 1
                continue
            tok = t
            break
        if a == len(drafted):
            tok = int(np.argmax(rows[len(drafted)]))
        emit = drafted[:a] + [tok]
        for e in emit:
            seq.append(e)
            out.append(e)
            if len(out) >= max_tokens:
                break
        target.truncate(min(common_prefix(target.tokens, seq), len(seq) - 1))
        cycles += 1
    return out, cycles
