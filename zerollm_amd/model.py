"""HipModel: the reference's model interface (PoolModel, src/compute/pool.js:24-316) backed by the HIP library.

Same members and semantics: forward / forward_batch with logits False|True|'none'|'last'|'all', truncate (positional
KV bookkeeping; restore + replay for hybrid models), mark_rollback, reset, close (idempotent), and the fields tokens, pos,
ctx, cfg, max_batch,
logits_batch, kernels ('hip'), kv. Errors carry the reference's messages ("context full (N tokens)", "token id X out of
range", "batch of B tokens (max M)", "model is closed"). Returned logits are a view over model-owned host memory that
is valid until the next call, as the reference's are (src/compute/pool.js:133, 143).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import ZLError, call, lib, ptr

ARCH_NAMES = {0: "llama", 1: "qwen2", 2: "qwen3", 3: "qwen35"}


def _opts(ctx, kv, max_batch, logits_batch, max_checkpoints=None, checkpoint_every=0, boundary_ids=()):
    """PoolModel.create options; the last three are the hybrid checkpoint policy (src/model/state-checkpoints.js:18-35):
    max_checkpoints None = the default 6, 0 = none."""
    if kv not in ("f32", "f16"):
        raise ValueError(f'kv must be f32 or f16 (got "{kv}")')
    ids = (C.c_int32 * max(1, len(boundary_ids)))(*boundary_ids)
    o = _lib.zl_model_opts(ctx=int(ctx or 0), kv_f16=1 if kv == "f16" else 0, max_batch=int(max_batch or 16),
                           logits_batch=int(logits_batch or 0),
                           max_checkpoints=0 if max_checkpoints is None else (-1 if max_checkpoints == 0 else int(max_checkpoints)),
                           checkpoint_every=int(checkpoint_every or 0), boundary_ids=ids, n_boundary=len(boundary_ids))
    o._ids = ids  # kept alive with the struct
    return o


class HipModel:
    kernels = "hip"

    def __init__(self, handle, kv):
        self._h = handle
        self.kv = kv
        c = _lib.zl_config()
        call("zl_model_config", self._h, C.byref(c))
        self._cfgs = c
        self.cfg = {
            "arch": ARCH_NAMES[c.arch], "nCtxTrain": c.n_ctx_train, "nEmbd": c.n_embd, "nLayer": c.n_layer, "nFF": c.n_ff,
            "nHead": c.n_head, "nHeadKv": c.n_head_kv, "headDim": c.head_dim, "nRot": c.n_rot, "rmsEps": c.rms_eps,
            "ropeBase": c.rope_base, "ropeType": "neox" if c.neox else "norm", "vocabSize": c.vocab,
            "qkNorm": bool(c.qk_norm), "qkvBias": bool(c.qkv_bias), "tiedEmbeddings": bool(c.tied),
            "hasRopeFreqs": bool(c.has_rope_freqs), "hybrid": bool(c.hybrid),
        }
        if c.hybrid:
            # qwen35 layout (src/model/config.js:126-156)
            self.cfg["layerIsRecurrent"] = [(l + 1) % c.full_attn_interval != 0 for l in range(c.n_layer)]
            self.cfg["ssm"] = {"convKernel": c.ssm_conv_kernel, "headKDim": c.ssm_d_state,
                               "headVDim": c.ssm_d_inner // c.ssm_dt_rank, "nKHeads": c.ssm_n_group,
                               "nVHeads": c.ssm_dt_rank, "innerSize": c.ssm_d_inner,
                               "convDim": 2 * c.ssm_n_group * c.ssm_d_state + c.ssm_d_inner}
        info = _lib.zl_model_info()
        call("zl_model_info_get", self._h, C.byref(info))
        self.ctx = info.ctx
        self.max_batch = info.max_batch
        self.logits_batch = info.logits_batch
        self.weight_bytes = info.weight_bytes
        self.device_bytes = info.device_bytes
        self.state_bytes = info.state_bytes
        self.captures = info.state_capture_slots > 0  # rollbacks inside a verify window copy a captured state
        self.closed = False
        self._logits = np.empty((self.logits_batch, c.vocab), dtype=np.float32)

    # ---- construction
    @classmethod
    def load(cls, path: str, ctx=None, kv="f32", max_batch=16, logits_batch=None, **ck) -> "HipModel":
        """PoolModel.create over a GGUF file (src/compute/pool.js:33-121). ck: max_checkpoints, checkpoint_every,
        boundary_ids (hybrid models)."""
        h = C.c_void_p()
        o = _opts(ctx, kv, max_batch, logits_batch, **ck)
        call("zl_model_load", path.encode(), C.byref(o), C.byref(h))
        return cls(h, kv)

    @classmethod
    def from_synth(cls, cfg: "_lib.zl_config", tensors, ctx=None, kv="f32", max_batch=16, logits_batch=None,
                   **ck) -> "HipModel":
        """A synthetic model generated in HBM (see zerollm_amd.synth)."""
        h = C.c_void_p()
        o = _opts(ctx, kv, max_batch, logits_batch, **ck)
        arr = (_lib.zl_synth_tensor * len(tensors))(*tensors)
        call("zl_model_synth", C.byref(cfg), arr, len(tensors), C.byref(o), C.byref(h))
        return cls(h, kv)

    # ---- state
    @property
    def pos(self) -> int:
        return lib().zl_model_pos(self._h) if not self.closed else 0

    @property
    def tokens(self) -> list:
        if self.closed:
            return []
        n = lib().zl_model_tokens(self._h, None, 0)
        buf = (C.c_int32 * max(n, 1))()
        lib().zl_model_tokens(self._h, buf, n)
        return list(buf[:n])

    def _check_open(self):
        if self.closed:
            raise ZLError(5, "model is closed")

    # ---- passes
    def forward(self, token: int, logits=True):
        """Run one token at the next position (src/compute/pool.js:135)."""
        return self.forward_batch([token], logits=logits)

    def forward_batch(self, tokens, logits=None, copy=True):
        """Run several tokens at consecutive positions in one pass over the weights (src/compute/pool.js:145-160).
        logits: False/'none' -> None; True/'last'/None -> vocab floats of the last token; 'all' -> B x vocab.
        copy=False leaves the logits on the device only (for the device sampler) and returns None."""
        self._check_open()
        want = 0 if logits is False or logits == "none" else 2 if logits == "all" else 1
        toks = np.ascontiguousarray(np.asarray(list(tokens), dtype=np.int32))
        B = len(toks)
        out = self._logits if (want and copy) else None
        call("zl_forward", self._h, ptr(toks, C.c_int32) if B else None, B, want, ptr(out, C.c_float) if out is not None else None)
        if out is None:
            return None
        if want == 2:
            return self._logits[:B]
        return self._logits[0] if want else None

    def truncate(self, n: int) -> int:
        """Roll back to n positions (src/compute/pool.js:278-294): positional KV is bookkeeping; a hybrid model restores
        the nearest recurrent-state snapshot and replays the tokens in between. Returns the tokens replayed."""
        if n >= self.pos:
            return 0
        self._check_open()
        r = C.c_int()
        call("zl_truncate", self._h, max(0, int(n)), C.byref(r))
        return r.value

    def truncate_plan(self, n: int):
        """truncatePlan (src/compute/pool.js:256): (from, replay)."""
        f, r = C.c_int(), C.c_int()
        call("zl_truncate_plan", self._h, int(n), C.byref(f), C.byref(r))
        return f.value, r.value

    @property
    def checkpoint_positions(self) -> list:
        if self.closed:
            return []
        n = lib().zl_model_checkpoints(self._h, None, 0)
        buf = (C.c_int32 * max(n, 1))()
        lib().zl_model_checkpoints(self._h, buf, n)
        return list(buf[:n])

    def recurrent_state(self):
        """getRecurrentState (src/compute/pool.js:259): (conv, ssm) float32 arrays in the reference's layout."""
        c = self.cfg
        s = c["ssm"]
        n_rec = sum(c["layerIsRecurrent"])
        conv = np.zeros(n_rec * s["convDim"] * (s["convKernel"] - 1), np.float32)
        ssm = np.zeros(n_rec * s["nVHeads"] * s["headVDim"] * s["headKDim"], np.float32)
        call("zl_model_recurrent_state", self._h, ptr(conv, C.c_float), ptr(ssm, C.c_float))
        return conv, ssm

    def mark_rollback(self):
        """markRollback (src/compute/pool.js:269): snapshot of a hybrid model's recurrent state; no-op otherwise."""
        if not self.closed:
            call("zl_mark_rollback", self._h)

    def reset(self):
        self._check_open()
        call("zl_reset", self._h)

    def close(self):
        """Release the model (idempotent, src/compute/pool.js:302-316)."""
        if self.closed:
            return
        self.closed = True
        call("zl_model_free", self._h)
        self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # camelCase aliases of the reference's member names
    forwardBatch = forward_batch
    markRollback = mark_rollback
    truncatePlan = truncate_plan

    @property
    def maxBatch(self):
        return self.max_batch

    @property
    def logitsBatch(self):
        return self.logits_batch

    # ---- timing probe
    PROBE = {"qkv": 0, "wo": 1, "gate_up": 2, "down": 3, "output": 4}

    def probe_gemv(self, which: str, M: int, iters: int):
        """(ms per launch, weight bytes per launch) of one GEMV of the pass, launched back to back over the layers."""
        ms = C.c_float()
        b = C.c_int64()
        call("zl_probe_gemv", self._h, self.PROBE[which], int(M), int(iters), C.byref(ms), C.byref(b))
        return ms.value, b.value


def verify_limit(model) -> int:
    """verifyLimit (src/model/speculative.js:25-28)."""
    if not hasattr(model, "forward_batch"):
        return 1 << 30
    return min(getattr(model, "max_batch", 1), getattr(model, "logits_batch", getattr(model, "max_batch", 1)))


def init(device: int = 0):
    call("zl_init", int(device))


def device_info():
    d = _lib.zl_device_info()
    call("zl_device_query", C.byref(d))
    return {"name": d.name.decode(), "compute_units": d.compute_units, "hbm_bytes": d.hbm_bytes,
            "lds_per_block": d.lds_per_block, "clock_khz": d.clock_khz, "mem_clock_khz": d.mem_clock_khz,
            "mem_bus_width": d.mem_bus_width}
