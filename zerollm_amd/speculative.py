"""Speculative decoding on the GPU: generateSpeculative (src/model/speculative.js:100-240) with the cycle's device work
(draft proposals, the (k+1)-token verification pass, acceptance / residual / bonus draws) in one library call per cycle.

The loop bookkeeping stays on the host exactly as the reference writes it: kk, the draft's KV reuse and feed, emission
through stop / max / context checks, and truncation of both models. Only accepted token ids cross from the GPU.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import time

import numpy as np

from . import _lib
from ._lib import call, ptr
from .generate import common_prefix, prefill_tokens
from .model import verify_limit
from .sampler import HipSampler

DEFAULT_DRAFT_K = 3  # src/model/speculative.js:248


def generate_speculative(target, draft, prompt_ids, k=4, max_tokens=256, sample=None, stop_ids=(), signal=None,
                         stats=None, penalize_prompt=True, on_prefill_progress=None, cycle_log=None):
    """Yield token ids after prompt_ids using `draft` to propose k tokens per cycle and `target` to verify them.
    Same contract as generateSpeculative: greedy output equals plain greedy decoding; sampled output has the target's
    distribution; stats gets promptTokens, cachedTokens, prefillMs, decodeMs, generated, stopReason and
    speculative = {k, cycles, drafted, accepted, acceptRate, tokensPerCycle, cycleMs, acceptedHist, effectiveTps}.
    cycle_log (not in the reference): a list that receives one (kk, drafted, accepted, token) tuple per cycle, the
    decisions the device took."""
    if sample is None:
        sample = HipSampler(argmax=True)
    greedy = sample.greedy
    stop = list(stop_ids or ())
    stop_set = set(stop)
    mx = max_tokens
    stats = stats if stats is not None else {}
    k_max = max(1, int(k))
    n0 = len(prompt_ids)
    if n0 == 0:
        raise ValueError("empty prompt")
    if n0 >= target.ctx:
        raise ValueError(f"prompt is {n0} tokens but the context window is {target.ctx}; shorten it or raise --ctx")
    if n0 >= draft.ctx:
        raise ValueError(f"prompt is {n0} tokens but the draft model's context window is {draft.ctx}; give the draft model at least the target's context")
    V = target.cfg["vocabSize"]
    if draft.cfg["vocabSize"] != V:
        raise ValueError(f"draft vocabulary ({draft.cfg['vocabSize']}) differs from the target's ({V})")
    t_limit = verify_limit(target)
    if t_limit < 2:
        raise ValueError("speculative decoding needs a target that can verify at least 2 tokens per pass (raise maxBatch)")
    prompt_ids = list(prompt_ids)

    # ---- prefill everything but the last prompt token on both models (:117-143)
    body = prompt_ids[:-1]
    reuse = min(common_prefix(target.tokens, prompt_ids), n0 - 1)
    target.truncate(reuse)
    d_reuse = min(common_prefix(draft.tokens, body), len(body))
    draft.truncate(d_reuse)
    stats.update(promptTokens=n0, cachedTokens=reuse, generated=0, stopReason="length")
    spec = stats["speculative"] = {"k": k_max, "cycles": 0, "drafted": 0, "accepted": 0, "acceptRate": 0.0,
                                   "tokensPerCycle": 0.0, "cycleMs": 0.0, "draftMs": 0.0, "verifyMs": 0.0, "otherMs": 0.0,
                                   "acceptedHist": [0] * (k_max + 1), "draftCachedTokens": d_reuse, "draftPrefillMs": 0.0}
    t0 = time.perf_counter()
    t_todo, d_todo = len(body) - reuse, len(body) - d_reuse
    prog = on_prefill_progress
    _, aborted = prefill_tokens(target, body, start=reuse, want_logits=False, signal=signal,
                                on_progress=(lambda d, _n: prog(d, t_todo + d_todo)) if prog else None)
    if not aborted:
        td = time.perf_counter()
        _, aborted = prefill_tokens(draft, body, start=d_reuse, want_logits=False, signal=signal,
                                    on_progress=(lambda d, _n: prog(t_todo + d, t_todo + d_todo)) if prog else None)
        spec["draftPrefillMs"] = (time.perf_counter() - td) * 1e3
    stats["prefillMs"] = (time.perf_counter() - t0) * 1e3
    if aborted:
        stats["stopReason"] = "aborted"
        return
    stats["prefilled"] = n0 - reuse

    seq = list(prompt_ids)
    need_hist = sample.uses_history

    def hist_of(full, n):
        if not need_hist:
            return []
        return full[n0:n] if penalize_prompt is False else full[:n]

    res = _lib.zl_spec_result()
    stop_arr = np.ascontiguousarray(np.asarray(stop[:64], dtype=np.int32))
    generated = 0
    t_dec = time.perf_counter()
    try:
        while generated < mx:
            if signal is not None and getattr(signal, "aborted", False):
                stats["stopReason"] = "aborted"
                break
            pending = seq[-1]
            kk = min(k_max, mx - generated - 1, target.ctx - len(seq), t_limit - 1, draft.ctx - len(seq) + 1)
            kk = max(0, kk)
            feed = []
            if kk > 0:
                draft.truncate(min(common_prefix(draft.tokens, seq), len(seq) - 1))
                feed = seq[draft.pos:]
                # draft.markRollback after feedLogits (src/model/speculative.js:168) happens inside zl_spec_cycle
            target.mark_rollback()
            feed_arr = np.ascontiguousarray(np.asarray(feed, dtype=np.int32))
            h = hist_of(seq, len(seq))
            hist_arr = np.ascontiguousarray(np.asarray(h[-64:], dtype=np.int32))
            tc = time.perf_counter()
            call("zl_spec_cycle", target._h, draft._h, sample._h, ptr(feed_arr, C.c_int32) if len(feed_arr) else None,
                 len(feed_arr), int(pending), int(kk), ptr(stop_arr, C.c_int32) if len(stop_arr) else None, len(stop_arr),
                 ptr(hist_arr, C.c_int32) if len(hist_arr) else None, len(hist_arr), C.byref(res))
            t_after = time.perf_counter()
            spec["cycleMs"] += (t_after - tc) * 1e3
            spec["draftMs"] += res.ms_draft
            spec["verifyMs"] += res.ms_total - res.ms_draft
            kk = res.kk
            drafted = list(res.drafted[:kk])
            a = res.accepted
            tok = res.token
            spec["cycles"] += 1
            spec["drafted"] += kk
            spec["accepted"] += a
            spec["acceptedHist"][a] += 1
            if cycle_log is not None:
                cycle_log.append((kk, tuple(drafted), a, tok))
            # ---- emit and roll back (:212-226)
            emit = drafted[:a] + [tok]
            done = False
            for e in emit:
                if signal is not None and getattr(signal, "aborted", False):
                    stats["stopReason"] = "aborted"
                    done = True
                    break
                if e in stop_set:
                    stats["stopReason"] = "stop"
                    done = True
                    break
                idx = len(seq)
                seq.append(e)
                yield e
                generated += 1
                stats["generated"] = generated
                if generated >= mx:
                    done = True
                    break
                if idx >= target.ctx:
                    stats["stopReason"] = "context"
                    done = True
                    break
            target.truncate(min(common_prefix(target.tokens, seq), len(seq) - 1))
            spec["otherMs"] += (time.perf_counter() - t_after) * 1e3
            if done:
                break
    finally:
        if not target.closed:
            target.truncate(common_prefix(target.tokens, seq))
        if not draft.closed:
            draft.truncate(common_prefix(draft.tokens, seq))
        stats["decodeMs"] = (time.perf_counter() - t_dec) * 1e3
        spec["acceptRate"] = spec["accepted"] / spec["drafted"] if spec["drafted"] else 0.0
        spec["tokensPerCycle"] = generated / spec["cycles"] if spec["cycles"] else 0.0
        spec["effectiveTps"] = generated * 1000.0 / stats["decodeMs"] if stats["decodeMs"] > 0 else 0.0


generateSpeculative = generate_speculative


def vocab_fingerprint(g):
    """vocabFingerprint (src/model/speculative.js:256-264): size and sha256 over token strings and types."""
    tokens = g.get("tokenizer.ggml.tokens", []) or []
    types = g.get("tokenizer.ggml.token_type", []) or []
    h = hashlib.sha256()
    for t in tokens:
        h.update(str(t).encode("utf-8"))
        h.update(b"\0")
    h.update(f"#{len(types)}:".encode())
    for t in types:
        h.update(f"{t},".encode())
    return {"size": len(tokens), "hash": h.hexdigest()}


def vocab_mismatch(target, draft):
    """Why `draft` cannot draft for `target` (GGUF files), or None (src/model/speculative.js:271-283)."""
    a = vocab_fingerprint(target)
    b = vocab_fingerprint(draft)
    if a["size"] != b["size"]:
        return (f"the draft model has a vocabulary of {b['size']} tokens but the target has {a['size']}: speculative decoding "
                "needs two models of the same family with the same tokenizer (e.g. Qwen3-0.6B for Qwen3-8B)")
    if a["hash"] != b["hash"]:
        ta = target.get("tokenizer.ggml.tokens", []) or []
        tb = draft.get("tokenizer.ggml.tokens", []) or []
        i = 0
        while i < len(ta) and i < len(tb) and ta[i] == tb[i]:
            i += 1
        # JSON.stringify of the two token strings, as the reference formats them
        detail = (f" (first difference at token id {i}: {json.dumps(ta[i], ensure_ascii=False)} vs "
                  f"{json.dumps(tb[i], ensure_ascii=False) if i < len(tb) else 'undefined'})") if i < len(ta) \
            else " (the token types differ)"
        return f"the draft model's tokenizer differs from the target's{detail}: speculative decoding needs the same vocabulary"
    arch_a = target.get("general.architecture")
    arch_b = draft.get("general.architecture")
    va = target.get(f"{arch_a}.vocab_size")
    vb = draft.get(f"{arch_b}.vocab_size")
    if va is not None and vb is not None and va != vb:
        return f"the models disagree on the logits vocabulary size ({va} vs {vb})"
    return None
