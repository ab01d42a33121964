"""ctypes binding of libzerollm_hip.so (the C ABI in include/zerollm_hip.h).

There is no fallback: if the library is missing or cannot load, importing the model/sampler classes raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzerollm_hip.so")

ZL_OK = 0
ERRORS = {1: "argument", 2: "HIP", 3: "format", 4: "unsupported", 5: "state", 6: "context", 7: "token", 8: "batch", 9: "io"}


class ZLError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class zl_device_info(C.Structure):
    _fields_ = [("name", C.c_char * 128), ("compute_units", C.c_int), ("hbm_bytes", C.c_int64), ("lds_per_block", C.c_int),
                ("clock_khz", C.c_int), ("mem_clock_khz", C.c_int), ("mem_bus_width", C.c_int)]


class zl_model_opts(C.Structure):
    _fields_ = [("ctx", C.c_int), ("kv_f16", C.c_int), ("max_batch", C.c_int), ("logits_batch", C.c_int),
                ("max_checkpoints", C.c_int), ("checkpoint_every", C.c_int), ("boundary_ids", C.POINTER(C.c_int32)),
                ("n_boundary", C.c_int)]


class zl_config(C.Structure):
    _fields_ = [("arch", C.c_int), ("n_ctx_train", C.c_int), ("n_embd", C.c_int), ("n_layer", C.c_int), ("n_ff", C.c_int),
                ("n_head", C.c_int), ("n_head_kv", C.c_int), ("head_dim", C.c_int), ("n_rot", C.c_int), ("vocab", C.c_int),
                ("rms_eps", C.c_float), ("rope_base", C.c_float), ("neox", C.c_int), ("qk_norm", C.c_int),
                ("qkv_bias", C.c_int), ("tied", C.c_int), ("has_rope_freqs", C.c_int), ("hybrid", C.c_int),
                ("full_attn_interval", C.c_int), ("ssm_conv_kernel", C.c_int), ("ssm_d_state", C.c_int),
                ("ssm_n_group", C.c_int), ("ssm_dt_rank", C.c_int), ("ssm_d_inner", C.c_int)]


class zl_model_info(C.Structure):
    _fields_ = [("ctx", C.c_int), ("max_batch", C.c_int), ("logits_batch", C.c_int), ("kv_f16", C.c_int),
                ("weight_bytes", C.c_int64), ("device_bytes", C.c_int64), ("state_bytes", C.c_int64),
                ("state_capture_slots", C.c_int)]


class zl_synth_tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64), ("seed", C.c_uint64),
                ("std", C.c_double), ("src_cols", C.c_int64), ("col0", C.c_int64), ("fill", C.c_int), ("fill_value", C.c_float)]


class zl_sampler_opts(C.Structure):
    _fields_ = [("temperature", C.c_double), ("top_p", C.c_double), ("min_p", C.c_double), ("repeat_penalty", C.c_double),
                ("presence_penalty", C.c_double), ("frequency_penalty", C.c_double), ("top_k", C.c_int),
                ("repeat_last_n", C.c_int), ("seed", C.c_uint32), ("greedy_argmax", C.c_int)]


class zl_spec_result(C.Structure):
    _fields_ = [("kk", C.c_int), ("accepted", C.c_int), ("token", C.c_int), ("drafted", C.c_int32 * 64), ("ms_total", C.c_float),
                ("ms_draft", C.c_float)]


P = C.c_void_p
I32P = C.POINTER(C.c_int32)
F32P = C.POINTER(C.c_float)
F64P = C.POINTER(C.c_double)

# (name, restype, argtypes) for every exported symbol
SIGNATURES = [
    ("zl_last_error", C.c_char_p, []),
    ("zl_init", C.c_int, [C.c_int]),
    ("zl_device_query", C.c_int, [C.POINTER(zl_device_info)]),
    ("zl_model_load", C.c_int, [C.c_char_p, C.POINTER(zl_model_opts), C.POINTER(P)]),
    ("zl_model_config", C.c_int, [P, C.POINTER(zl_config)]),
    ("zl_model_info_get", C.c_int, [P, C.POINTER(zl_model_info)]),
    ("zl_model_free", C.c_int, [P]),
    ("zl_forward", C.c_int, [P, I32P, C.c_int, C.c_int, F32P]),
    ("zl_truncate", C.c_int, [P, C.c_int, C.POINTER(C.c_int)]),
    ("zl_truncate_plan", C.c_int, [P, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    ("zl_mark_rollback", C.c_int, [P]),
    ("zl_model_checkpoints", C.c_int, [P, I32P, C.c_int]),
    ("zl_model_recurrent_state", C.c_int, [P, F32P, F32P]),
    ("zl_reset", C.c_int, [P]),
    ("zl_model_pos", C.c_int, [P]),
    ("zl_model_tokens", C.c_int, [P, I32P, C.c_int]),
    ("zl_model_logits", C.c_int, [P, C.c_int, C.c_int, F32P]),
    ("zl_synth_tensor_bytes", C.c_int, [C.POINTER(zl_synth_tensor), C.c_int, P]),
    ("zl_model_synth", C.c_int, [C.POINTER(zl_config), C.POINTER(zl_synth_tensor), C.c_int, C.POINTER(zl_model_opts), C.POINTER(P)]),
    ("zl_sampler_create", C.c_int, [C.POINTER(zl_sampler_opts), C.POINTER(P)]),
    ("zl_sampler_free", C.c_int, [P]),
    ("zl_sampler_get_rng", C.c_int, [P, C.POINTER(C.c_uint32)]),
    ("zl_sampler_set_rng", C.c_int, [P, C.c_uint32]),
    ("zl_sampler_cycle_graphs", C.c_int, [P, C.POINTER(C.c_int)]),
    ("zl_sample", C.c_int, [P, P, C.c_int, I32P, C.c_int, I32P]),
    ("zl_distribution", C.c_int, [P, P, C.c_int, I32P, C.c_int, I32P, F64P, C.c_int, C.POINTER(C.c_int), F64P, C.POINTER(C.c_int)]),
    ("zl_spec_cycle", C.c_int, [P, P, P, I32P, C.c_int, C.c_int32, C.c_int, I32P, C.c_int, I32P, C.c_int, C.POINTER(zl_spec_result)]),
    ("zl_mat_upload", C.c_int, [C.c_int, P, C.c_int64, C.c_int64, C.POINTER(P)]),
    ("zl_mat_synth", C.c_int, [C.c_int, C.c_int64, C.c_int64, C.c_uint64, C.c_double, C.c_int, C.POINTER(P)]),
    ("zl_mat_free", C.c_int, [P]),
    ("zl_mat_dequant", C.c_int, [P, C.c_int64, C.c_int64, F32P]),
    ("zl_mat_gemv", C.c_int, [P, F32P, C.c_int, F32P]),
    ("zl_mat_gemv_time", C.c_int, [P, C.c_int, C.c_int, F32P]),
    ("zl_mat_gemv_noalloc", C.c_int, [P, P, C.c_int, P, P]),
    ("zl_quant_act", C.c_int, [F32P, C.c_int64, C.c_int, C.POINTER(C.c_int8), F32P, I32P]),
    ("zl_probe_gemv", C.c_int, [P, C.c_int, C.c_int, C.c_int, F32P, C.POINTER(C.c_int64)]),
]

_lib = None


def lib():
    """The loaded library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ZLError(4, f"{LIB_PATH} is not built: run `python -m zerollm_amd.build` (the HIP path has no fallback)")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int):
    if rc != ZL_OK:
        msg = lib().zl_last_error().decode("utf-8", errors="replace")
        raise ZLError(rc, msg or f"zerollm_hip error {rc} ({ERRORS.get(rc, '?')})")


def call(name: str, *args):
    check(getattr(lib(), name)(*args))


def ptr(arr, ctype):
    """ctypes pointer to a contiguous numpy array."""
    return arr.ctypes.data_as(C.POINTER(ctype))
