"""ctypes binding of the C ABI in include/citlali_hip.h (libcitlali_hip.so).

The library is built in-tree by ``make -C citlali-llm-engine_amd`` (or
``__graft_entry__.build()``).  Loading fails loudly when it is missing: there
is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_longlong, c_size_t, c_uint64, c_void_p

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
HIP_LIB_PATH = os.path.join(LIB_DIR, "libcitlali_hip.so")
HOST_LIB_PATH = os.path.join(LIB_DIR, "libcitlali.so")

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3


class CitlaliError(RuntimeError):
    """An entry point returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


# (name, restype, argtypes) for every function of include/citlali_hip.h
_P = c_void_p
class Norm(ctypes.Structure):
    """citlali_hip_norm: residual add + RMSNorm feeding a GEMV."""
    _fields_ = [("delta", c_void_p), ("weight", c_void_p), ("sum_out", c_void_p), ("eps", c_float)]


SIGNATURES = [
    ("citlali_hip_last_error", c_char_p, []),
    ("citlali_hip_abi_version", c_int, []),
    ("citlali_hip_init", c_int, [c_int]),
    ("citlali_hip_device_count", c_int, [POINTER(c_int)]),
    ("citlali_hip_set_stream", c_int, [_P]),
    ("citlali_hip_get_stream", _P, []),
    ("citlali_hip_synchronize", c_int, []),
    ("citlali_hip_malloc", c_int, [POINTER(c_void_p), c_size_t]),
    ("citlali_hip_free", c_int, [_P]),
    ("citlali_hip_memcpy_h2d", c_int, [_P, _P, c_size_t]),
    ("citlali_hip_memcpy_d2h", c_int, [_P, _P, c_size_t]),
    ("citlali_hip_memcpy_d2d", c_int, [_P, _P, c_size_t]),
    ("citlali_hip_zero", c_int, [_P, c_size_t]),
    ("citlali_hip_matvec_q4k", c_int, [_P, _P, _P, c_int, c_int]),
    ("citlali_hip_matvec_q4k_to_float", c_int, [_P, _P, _P, c_int, c_int]),
    ("citlali_hip_matvec_q6k", c_int, [_P, _P, _P, c_int, c_int]),
    ("citlali_hip_matvec_q6k_to_float", c_int, [_P, _P, _P, c_int, c_int]),
    ("citlali_hip_embed_q6k", c_int, [_P, c_int32, _P, c_int]),
    ("citlali_hip_attention", c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int]),
    ("citlali_hip_attention_batched", c_int,
     [_P, _P, _P, c_longlong, _P, c_int, c_int, c_int, c_int, c_int, _P, c_size_t, _P]),
    ("citlali_hip_attention_workspace_bytes", c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    ("citlali_hip_release_workspace", c_int, []),
    ("citlali_hip_store_kv", c_int, [_P, _P, _P, _P, c_int, c_int]),
    ("citlali_hip_dequant_q4k_f16", c_int, [_P, c_uint64, _P]),
    ("citlali_hip_dequant_q6k_f16", c_int, [_P, c_uint64, _P]),
    ("citlali_hip_embed", c_int, [_P, c_int32, _P, c_int]),
    ("citlali_hip_copy", c_int, [_P, _P, c_int]),
    ("citlali_hip_add_inplace", c_int, [_P, _P, c_int]),
    ("citlali_hip_add_bias_inplace", c_int, [_P, _P, c_int]),
    ("citlali_hip_rms_norm", c_int, [_P, _P, _P, c_int, c_float]),
    ("citlali_hip_rms_norm_heads", c_int, [_P, _P, _P, c_int, c_int, c_float]),
    ("citlali_hip_matvec_fp16", c_int, [_P, _P, _P, c_int, c_int]),
    ("citlali_hip_matvec_fp16_to_float", c_int, [_P, _P, _P, c_int, c_int]),
    ("citlali_hip_swiglu", c_int, [_P, _P, _P, c_int]),
    ("citlali_hip_rope", c_int, [_P, c_int, c_int, c_int, c_float]),
    ("citlali_hip_argmax", c_int, [_P, c_int, _P]),
    ("citlali_hip_stream_read", c_int, [_P, c_size_t, _P]),
    ("citlali_hip_add_rms_norm", c_int, [_P, _P, _P, _P, c_int, c_float]),
    ("citlali_hip_qk_norm_rope_store", c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_float, c_float, _P,
                                               _P]),
    ("citlali_hip_matvec_gate_up_swiglu", c_int, [c_int, _P, _P, _P, _P, c_int, c_int]),
    ("citlali_hip_matvec_group", c_int, [c_int, POINTER(c_int), POINTER(c_void_p), _P, POINTER(c_void_p),
                                         POINTER(c_int), c_int]),
    ("citlali_hip_attention_noalloc", c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int]),
    ("citlali_hip_attention_plan_length", c_int, [c_int, c_int]),
    ("citlali_hip_attention_plan_info", c_int, [c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    ("citlali_hip_argmax_advance", c_int, [_P, c_int, _P, _P, c_int]),
    ("citlali_hip_embed_q6k_at", c_int, [_P, _P, c_int, _P, c_int]),
    ("citlali_hip_embed_at", c_int, [_P, _P, c_int, _P, c_int]),
    ("citlali_hip_qk_norm_rope_store_at", c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, _P, c_int, c_float,
                                                  c_float, _P, _P]),
    ("citlali_hip_qk_norm_rope_store_attention", c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, _P, c_int,
                                                         c_int, c_float, c_float, _P, _P, _P, c_size_t, _P]),
    ("citlali_hip_stream_create", c_int, [POINTER(c_void_p)]),
    ("citlali_hip_stream_destroy", c_int, [_P]),
    ("citlali_hip_graph_begin", c_int, []),
    ("citlali_hip_graph_end", c_int, [POINTER(c_void_p)]),
    ("citlali_hip_graph_launch", c_int, [_P]),
    ("citlali_hip_graph_destroy", c_int, [_P]),
    ("citlali_hip_matvec_group_norm", c_int, [c_int, POINTER(c_int), POINTER(c_void_p), _P, POINTER(Norm),
                                              POINTER(c_void_p), POINTER(c_int), c_int]),
    ("citlali_hip_matvec_gate_up_swiglu_norm", c_int, [c_int, _P, _P, _P, POINTER(Norm), _P, c_int, c_int]),
    ("citlali_hip_matvec_norm", c_int, [c_int, _P, _P, POINTER(Norm), _P, c_int, c_int, c_int]),
    ("citlali_hip_set_kernel_timing", c_int, [_P, _P]),
    ("citlali_hip_set_dispatch_timing", c_int, [POINTER(c_void_p), POINTER(c_void_p), c_int]),
    ("citlali_hip_dispatch_timing_count", c_int, [POINTER(c_int)]),
    ("citlali_hip_event_create", c_int, [POINTER(c_void_p)]),
    ("citlali_hip_event_record", c_int, [_P]),
    ("citlali_hip_event_synchronize", c_int, [_P]),
    ("citlali_hip_event_elapsed_ms", c_int, [_P, _P, POINTER(c_float)]),
    ("citlali_hip_event_destroy", c_int, [_P]),
]

_lib = None


def load() -> ctypes.CDLL:
    """Loads libcitlali_hip.so (once) and declares every signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(HIP_LIB_PATH):
        raise ImportError(
            f"{HIP_LIB_PATH} is not built; run `make -C {PKG_DIR}` or __graft_entry__.build()")
    lib = ctypes.CDLL(HIP_LIB_PATH)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().citlali_hip_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    if status != OK:
        raise CitlaliError(status, last_error())


def call(name: str, *args) -> None:
    """Calls an int-returning entry point and raises CitlaliError on failure."""
    check(getattr(load(), name)(*args))
