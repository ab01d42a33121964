"""ORACLE — test infrastructure only (tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it; the
product never imports it).

generateSpeculative (src/model/speculative.js:100-240) restated over oracle models: any object with forward(token,
logits=True) -> f32 logits | None, truncate(n), tokens, pos, ctx and (optionally) mark_rollback(). A model with a batched
pass (forward_batch(tokens, logits) and max_batch, as oracle.pool.SimdPoolModel) is driven as the reference drives a
PoolModel: prefill and feedLogits in chunks of max_batch (src/model/generate.js:15-31, src/model/speculative.js:51-61) and
the k + 1 verify rows in one pass (forwardRows, :39-48; verifyLimit, :25-28). The single-token oracle models fall back
to one forward per token, as the reference does for RefModel. Both the greedy path and speculative sampling are
restated, with the single mulberry32 stream of the sampler consumed in the reference's order: draft draws x_1..x_kk
(:173), then the accept uniforms (:203), then one residual draw (:204, drawResidual :75-87) or one bonus draw (:207-209).
"""
from __future__ import annotations

import time

import numpy as np

from . import oracle as O


def common_prefix(a, b):
    """commonPrefix (src/model/generate.js:34-39)."""
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


class Argmax:
    """The plain argmax sampler generate() uses when none is passed (src/model/generate.js:4-8): first maximum."""

    greedy = True
    uses_history = False

    def sample(self, logits, history=()):
        return int(np.argmax(logits))


def _is_argmax(sample):
    return isinstance(sample, Argmax)


def _batched(model):
    return hasattr(model, "forward_batch")


def verify_limit(model):
    """verifyLimit (src/model/speculative.js:25-28): rows one verify pass can carry; infinite without a batched pass."""
    if not _batched(model):
        return float("inf")
    return min(model.max_batch, getattr(model, "logits_batch", model.max_batch))


def feed(model, ids, want_logits):
    """prefillTokens / feedLogits (src/model/generate.js:15-31, src/model/speculative.js:51-61): ids in chunks of the
    model's batch (1 without a batched pass); returns the last token's logits when asked."""
    logits = None
    chunk = max(1, model.max_batch) if _batched(model) else 1
    i = 0
    while i < len(ids):
        end = min(len(ids), i + chunk)
        last = want_logits and end == len(ids)
        if chunk > 1:
            logits = model.forward_batch(ids[i:end], logits="last" if last else "none")
        else:
            logits = model.forward(ids[i], logits=last)
        i = end
    return logits


def forward_rows(model, tokens):
    """forwardRows (src/model/speculative.js:39-48): per-position logits of every token, in one pass when it fits."""
    if _batched(model) and len(tokens) <= verify_limit(model):
        return list(model.forward_batch(tokens, logits="all"))
    return [model.forward(t) for t in tokens]


def speculative(target, draft, prompt_ids, k=4, max_tokens=256, sample=None, stop_ids=(), penalize_prompt=True,
                t_limit=None, cycle_log=None, stats=None, deadline=None):
    """Yield the token ids generateSpeculative yields after prompt_ids (src/model/speculative.js:100-240).

    sample: an oracle.Sampler (createSampler) or None / Argmax() for plain greedy. t_limit: verifyLimit(target) by
    default (Infinity for the single-token oracle models, :26-28); the caller may pass the device model's limit so both
    run the same kk sequence. cycle_log: a list that receives one
    (kk, drafted, accepted, token) tuple per cycle. deadline: a time.perf_counter() value after which no new cycle
    starts (bench sampling only)."""
    sample = sample if sample is not None else Argmax()
    greedy = _is_argmax(sample) or bool(sample.greedy)
    stop = set(stop_ids or ())
    mx = max_tokens
    stats = stats if stats is not None else {}
    k_max = max(1, int(k))
    n0 = len(prompt_ids)
    if n0 == 0:
        raise ValueError("empty prompt")
    if n0 >= target.ctx:
        raise ValueError(f"prompt is {n0} tokens but the context window is {target.ctx}; shorten it or raise --ctx")
    if n0 >= draft.ctx:
        raise ValueError(f"prompt is {n0} tokens but the draft model's context window is {draft.ctx}; give the draft "
                         "model at least the target's context")
    t_limit = verify_limit(target) if t_limit is None else t_limit
    prompt_ids = [int(t) for t in prompt_ids]

    # ---- prefill everything but the last prompt token on both models (:117-143)
    body = prompt_ids[:-1]
    reuse = min(common_prefix(target.tokens, prompt_ids), n0 - 1)
    target.truncate(reuse)
    d_reuse = min(common_prefix(draft.tokens, body), len(body))
    draft.truncate(d_reuse)
    feed(target, body[reuse:], False)
    feed(draft, body[d_reuse:], False)
    spec = stats["speculative"] = {"k": k_max, "cycles": 0, "drafted": 0, "accepted": 0,
                                   "acceptedHist": [0] * (k_max + 1)}
    stats["generated"] = 0
    stats["stopReason"] = "length"

    seq = list(prompt_ids)
    need_hist = not _is_argmax(sample) and bool(sample.uses_history)

    def hist_of(full, n):
        if not need_hist:
            return []
        return full[n0:n] if penalize_prompt is False else full[:n]

    generated = 0
    try:
        while generated < mx:
            if deadline is not None and time.perf_counter() > deadline:
                stats["stopReason"] = "deadline"
                break
            pending = seq[-1]
            kk = min(k_max, mx - generated - 1, target.ctx - len(seq), t_limit - 1, draft.ctx - len(seq) + 1)
            kk = max(0, int(kk))
            # -- draft (:163-179)
            drafted, qd = [], []
            if kk > 0:
                draft.truncate(min(common_prefix(draft.tokens, seq), len(seq) - 1))
                dl = feed(draft, seq[draft.pos:], True)  # feedLogits (:51-61)
                if hasattr(draft, "mark_rollback"):
                    draft.mark_rollback()
                for j in range(kk):
                    h = hist_of(seq + drafted, len(seq) + j)
                    if greedy:
                        x = sample.sample(dl, h)
                    else:
                        d = sample.distribution(dl, h)
                        x = sample.draw(d)
                        qd.append(d)
                    drafted.append(x)
                    if x in stop or j == kk - 1:
                        break
                    dl = draft.forward(x)
                kk = len(drafted)
            # -- verify: one pass over [pending, x_1..x_kk] (:182-190)
            if hasattr(target, "mark_rollback"):
                target.mark_rollback()
            rows = forward_rows(target, [pending] + drafted)
            full = seq + drafted
            # -- accept / reject (:192-209)
            a, tok = 0, -1
            for j in range(kk):
                h = hist_of(full, len(seq) + j)
                if greedy:
                    t = sample.sample(rows[j], h)
                    if t == drafted[j]:
                        a += 1
                        continue
                    tok = t
                    break
                pd = sample.distribution(rows[j], h)
                px = O.prob_of(pd, drafted[j])
                qx = O.prob_of(qd[j], drafted[j])
                if sample.rand() * qx < px:
                    a += 1
                    continue
                tok = O.draw_residual(sample, pd, qd[j], len(rows[j]))
                break
            if a == kk:
                tok = sample.sample(rows[kk], hist_of(full, len(seq) + kk))
            spec["cycles"] += 1
            spec["drafted"] += kk
            spec["accepted"] += a
            spec["acceptedHist"][a] += 1
            if cycle_log is not None:
                cycle_log.append((kk, tuple(drafted), a, tok))
            # -- emit and roll back (:211-226)
            done = False
            for e in drafted[:a] + [tok]:
                if e in stop:
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
            if done:
                break
    finally:
        target.truncate(common_prefix(target.tokens, seq))
        draft.truncate(common_prefix(draft.tokens, seq))
        spec["acceptRate"] = spec["accepted"] / spec["drafted"] if spec["drafted"] else 0.0
        spec["tokensPerCycle"] = generated / spec["cycles"] if spec["cycles"] else 0.0


def plain(model, prompt_ids, max_tokens, sample=None, stop_ids=(), penalize_prompt=True, stats=None):
    """generate() (src/model/generate.js:41-96) over an oracle model, one token per forward: the stream that greedy
    speculative decoding must reproduce."""
    sample = sample if sample is not None else Argmax()
    stop = set(stop_ids or ())
    stats = stats if stats is not None else {}
    prompt_ids = [int(t) for t in prompt_ids]
    n0 = len(prompt_ids)
    if n0 == 0:
        raise ValueError("empty prompt")
    if n0 >= model.ctx:
        raise ValueError(f"prompt is {n0} tokens but the context window is {model.ctx}; shorten it or raise --ctx")
    reuse = min(common_prefix(model.tokens, prompt_ids), n0 - 1)
    model.truncate(reuse)
    logits = None
    for i, t in enumerate(prompt_ids[reuse:]):
        logits = model.forward(t, logits=reuse + i == n0 - 1)
    history = list(prompt_ids)
    stats["stopReason"] = "length"
    for n in range(max_tokens):
        tok = sample.sample(logits, history[n0:] if penalize_prompt is False else history)
        if tok in stop:
            stats["stopReason"] = "stop"
            break
        yield tok
        history.append(tok)
        if n + 1 >= max_tokens:
            break
        if model.pos >= model.ctx:
            stats["stopReason"] = "context"
            break
        logits = model.forward(tok)


def speculative_greedy(target, draft, seq, k, max_tokens, deadline=None):
    """Greedy speculative decoding continuing `seq` whose body both models already hold (bench.py's CPU leg).
    Returns (emitted, cycles)."""
    st = {}
    out = list(speculative(target, draft, seq, k=k, max_tokens=max_tokens, deadline=deadline, stats=st))
    return out, st["speculative"]["cycles"]
