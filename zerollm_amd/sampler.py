"""Device sampler: createSampler (src/sampling/sampler.js:81-155) with distribution() and draw() running on the GPU
over a model's logits rows. Only token ids (or, for tests, the sparse distribution) come back to the host."""
from __future__ import annotations

import ctypes as C
import random
import time
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import call, ptr


@dataclass
class TokenDist:
    """zerollm's TokenDist (src/sampling/sampler.js:52-62): ids[i] has probability probs[i] / total."""
    ids: np.ndarray
    probs: np.ndarray
    total: float
    greedy: bool


class HipSampler:
    """createSampler(options). Defaults as the library's (src/sampling/sampler.js:82-90): temperature 0.8, topK 40,
    topP 0.95, minP 0, no penalties, repeatLastN 64, seed from the clock. argmax=True gives the plain argmax sampler
    that generate()/generateSpeculative() use when no sampler is passed (src/model/generate.js:4-8)."""

    def __init__(self, temperature=0.8, top_k=40, top_p=0.95, min_p=0.0, repeat_penalty=1.0, repeat_last_n=64,
                 presence_penalty=0.0, frequency_penalty=0.0, seed=None, argmax=False):
        if seed is None:
            seed = (int(time.time() * 1000) ^ random.getrandbits(32)) & 0xFFFFFFFF
        self.temperature = float(temperature)
        self.top_k = int(top_k)
        self.greedy = argmax or self.temperature <= 0
        self.uses_history = (repeat_penalty != 1 or presence_penalty != 0 or frequency_penalty != 0) and not argmax
        self.repeat_last_n = int(repeat_last_n)
        o = _lib.zl_sampler_opts(temperature=self.temperature, top_p=float(top_p), min_p=float(min_p),
                                 repeat_penalty=float(repeat_penalty), presence_penalty=float(presence_penalty),
                                 frequency_penalty=float(frequency_penalty), top_k=self.top_k,
                                 repeat_last_n=int(repeat_last_n), seed=int(seed) & 0xFFFFFFFF, greedy_argmax=1 if argmax else 0)
        self._h = C.c_void_p()
        call("zl_sampler_create", C.byref(o), C.byref(self._h))
        self.closed = False

    @staticmethod
    def _hist(history):
        h = np.ascontiguousarray(np.asarray(list(history) if history is not None else [], dtype=np.int32))
        return (ptr(h, C.c_int32) if len(h) else None), len(h), h

    def distribution(self, model, row: int = 0, history=()) -> TokenDist:
        hp, nh, keep = self._hist(history)
        cap = int(model._logits.shape[1])  # a full candidate list (top_k 0) keeps up to the vocabulary
        ids = np.zeros(cap, np.int32)
        probs = np.zeros(cap, np.float64)
        n = C.c_int()
        total = C.c_double()
        greedy = C.c_int()
        call("zl_distribution", self._h, model._h, int(row), hp, nh, ptr(ids, C.c_int32), ptr(probs, C.c_double), cap,
             C.byref(n), C.byref(total), C.byref(greedy))
        return TokenDist(ids[:n.value].copy(), probs[:n.value].copy(), total.value, bool(greedy.value))

    def sample(self, model, row: int = 0, history=()) -> int:
        """sample(logits, history) = draw(distribution(logits, history)), on the model's logits row `row`."""
        hp, nh, keep = self._hist(history)
        tok = C.c_int32()
        call("zl_sample", self._h, model._h, int(row), hp, nh, C.byref(tok))
        return int(tok.value)

    __call__ = sample

    @property
    def rng_state(self) -> int:
        s = C.c_uint32()
        call("zl_sampler_get_rng", self._h, C.byref(s))
        return int(s.value)

    @rng_state.setter
    def rng_state(self, v: int):
        call("zl_sampler_set_rng", self._h, int(v) & 0xFFFFFFFF)

    def close(self):
        if not self.closed:
            self.closed = True
            call("zl_sampler_free", self._h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def create_sampler(**opts) -> HipSampler:
    return HipSampler(**opts)


createSampler = create_sampler
