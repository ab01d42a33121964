"""Token generation helpers around the model interface (src/model/generate.js:4-96)."""
from __future__ import annotations

import time


def common_prefix(a, b) -> int:
    """Length of the common prefix of two token lists (src/model/generate.js:34-39)."""
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


def prefill_tokens(model, ids, start=0, want_logits=True, signal=None, on_progress=None, copy=True):
    """Feed ids[start:] in chunks of model.max_batch (src/model/generate.js:18-31). Returns (logits, aborted).
    copy=False keeps the last chunk's logits on the device (HipModel only)."""
    chunk = max(1, getattr(model, "max_batch", 1)) if hasattr(model, "forward_batch") else 1
    logits = None
    i = start
    while i < len(ids):
        if signal is not None and getattr(signal, "aborted", False):
            return None, True
        end = min(len(ids), i + chunk)
        last = want_logits and end == len(ids)
        if chunk > 1 or not copy:
            logits = model.forward_batch(ids[i:end], logits=bool(last), **({} if copy else {"copy": False}))
        else:
            logits = model.forward(ids[i], logits=bool(last))
        i = end
        if on_progress:
            on_progress(i - start, len(ids) - start)
    return logits, False


def generate(model, prompt_ids, max_tokens=256, sample=None, stop_ids=(), signal=None, stats=None, penalize_prompt=True):
    """Plain decoding (src/model/generate.js:55-96): yields token ids; the sampler runs on the device over the model's
    logits row, so only ids cross to the host. sample=None is greedy argmax."""
    from .sampler import HipSampler

    if sample is None:
        sample = HipSampler(argmax=True)
    stop = set(stop_ids or ())
    stats = stats if stats is not None else {}
    if len(prompt_ids) == 0:
        raise ValueError("empty prompt")
    if len(prompt_ids) >= model.ctx:
        raise ValueError(f"prompt is {len(prompt_ids)} tokens but the context window is {model.ctx}; shorten it or raise --ctx")
    reuse = min(common_prefix(model.tokens, prompt_ids), len(prompt_ids) - 1)
    model.truncate(reuse)
    stats.update(promptTokens=len(prompt_ids), cachedTokens=reuse, generated=0, stopReason="length")
    t0 = time.perf_counter()
    _, aborted = prefill_tokens(model, list(prompt_ids), start=reuse, want_logits=True, signal=signal, copy=False)
    if aborted:
        stats["stopReason"] = "aborted"
        stats["prefillMs"] = (time.perf_counter() - t0) * 1e3
        return
    stats["prefillMs"] = (time.perf_counter() - t0) * 1e3
    history = list(prompt_ids)
    t1 = time.perf_counter()
    try:
        n = 0
        while n < max_tokens:
            if signal is not None and getattr(signal, "aborted", False):
                stats["stopReason"] = "aborted"
                break
            hist = history[len(prompt_ids):] if penalize_prompt is False else history
            tok = sample.sample(model, 0, hist if sample.uses_history else ())
            if tok in stop:
                stats["stopReason"] = "stop"
                break
            yield tok
            history.append(tok)
            n += 1
            stats["generated"] = n
            if n >= max_tokens:
                break
            if model.pos >= model.ctx:
                stats["stopReason"] = "context"
                break
            model.forward_batch([tok], logits="last", copy=False)
    finally:
        stats["decodeMs"] = (time.perf_counter() - t1) * 1e3
