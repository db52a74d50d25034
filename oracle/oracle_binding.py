"""ctypes bindings of oracle/liboracle.so (the CPU restatement) and of
oracle/_ref/libcitlali_ref.so (the reference's own host routines, compiled
from /root/reference).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by the cpu_baseline leg of bench.py -- never by the product."""
from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_float, c_int, c_int32, c_size_t, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libcitlali_ref.so")

_P = c_void_p


def _p(a: np.ndarray) -> c_void_p:
    return a.ctypes.data_as(c_void_p)


class Oracle:
    SIGS = {
        "orc_f2h": (ctypes.c_uint16, [c_float]),
        "orc_h2f": (c_float, [ctypes.c_uint16]),
        "orc_f2h_rne": (ctypes.c_uint16, [c_float]),
        "orc_f2h_array": (None, [_P, c_size_t, _P]),
        "orc_f2h_rne_array": (None, [_P, c_size_t, _P]),
        "orc_h2f_array": (None, [_P, c_size_t, _P]),
        "orc_dequant_q4k_f16": (None, [_P, c_uint64, _P]),
        "orc_dequant_q6k_f16": (None, [_P, c_uint64, _P]),
        "orc_dequant_q4k_f32": (None, [_P, c_uint64, _P]),
        "orc_dequant_q6k_f32": (None, [_P, c_uint64, _P]),
        "orc_matvec_q4k": (None, [_P, _P, _P, c_int, c_int, c_int]),
        "orc_matvec_q6k": (None, [_P, _P, _P, c_int, c_int, c_int]),
        "orc_matvec_q4k_f16dot": (None, [_P, _P, _P, c_int, c_int, c_int]),
        "orc_matvec_q6k_f16dot": (None, [_P, _P, _P, c_int, c_int, c_int]),
        "orc_matvec_f16": (None, [_P, _P, _P, c_int, c_int, c_int]),
        "orc_embed_q6k": (None, [_P, c_int32, _P, c_int]),
        "orc_attention": (None, [_P, _P, _P, c_int, c_int, c_int, c_int, _P]),
        "orc_attention_f32": (None, [_P, _P, _P, c_int, c_int, c_int, c_int, _P, c_int]),
        "orc_rms_norm": (None, [_P, _P, _P, c_int, c_float]),
        "orc_rms_norm_heads": (None, [_P, _P, _P, c_int, c_int, c_float]),
        "orc_rope": (None, [_P, c_int, c_int, c_int, c_float]),
        "orc_swiglu": (None, [_P, _P, _P, c_int]),
        "orc_add_inplace": (None, [_P, _P, c_int]),
        "orc_store_kv": (None, [_P, _P, _P, _P, c_int, c_int]),
        "orc_argmax": (c_int32, [_P, c_int]),
        "orc_num_threads": (c_int, []),
    }

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        self.lib = ctypes.CDLL(path)
        for name, (res, args) in self.SIGS.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    # fp16
    def f2h(self, f) -> np.ndarray:
        f = np.ascontiguousarray(f, dtype=np.float32)
        out = np.empty(f.shape, np.uint16)
        self.lib.orc_f2h_array(_p(f), f.size, _p(out))
        return out

    def f2h_rne(self, f) -> np.ndarray:
        f = np.ascontiguousarray(f, dtype=np.float32)
        out = np.empty(f.shape, np.uint16)
        self.lib.orc_f2h_rne_array(_p(f), f.size, _p(out))
        return out

    def h2f(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.orc_h2f_array(_p(h), h.size, _p(out))
        return out

    # dequant
    def dequant_f16(self, kind: str, blocks: np.ndarray, count: int) -> np.ndarray:
        out = np.empty(count, np.uint16)
        getattr(self.lib, f"orc_dequant_{kind}_f16")(_p(np.ascontiguousarray(blocks)), count, _p(out))
        return out

    def dequant_f32(self, kind: str, blocks: np.ndarray, count: int) -> np.ndarray:
        out = np.empty(count, np.float32)
        getattr(self.lib, f"orc_dequant_{kind}_f32")(_p(np.ascontiguousarray(blocks)), count, _p(out))
        return out

    # GEMV
    def matvec(self, kind: str, w: np.ndarray, x: np.ndarray, in_f: int, out_f: int, nthreads: int = 0) -> np.ndarray:
        y = np.empty(out_f, np.float64)
        getattr(self.lib, f"orc_matvec_{kind}")(_p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(x)), _p(y),
                                                in_f, out_f, nthreads)
        return y

    def matvec_f16dot(self, kind: str, w, x, in_f, out_f, nthreads=0) -> np.ndarray:
        y = np.empty(out_f, np.float32)
        getattr(self.lib, f"orc_matvec_{kind}_f16dot")(_p(w), _p(x), _p(y), in_f, out_f, nthreads)
        return y

    def embed_q6k(self, table, token_id: int, hidden: int) -> np.ndarray:
        out = np.empty(hidden, np.uint16)
        self.lib.orc_embed_q6k(_p(table), token_id, _p(out), hidden)
        return out

    def attention(self, q, kc, vc, position, heads, kv_heads, head_dim) -> np.ndarray:
        out = np.empty(heads * head_dim, np.float64)
        self.lib.orc_attention(_p(q), _p(kc), _p(vc), position, heads, kv_heads, head_dim, _p(out))
        return out

    def attention_f32(self, q, kc, vc, position, heads, kv_heads, head_dim, nthreads=0) -> np.ndarray:
        out = np.empty(heads * head_dim, np.float32)
        self.lib.orc_attention_f32(_p(q), _p(kc), _p(vc), position, heads, kv_heads, head_dim, _p(out), nthreads)
        return out


    # the rest of forward_token (all fp16 bit patterns in and out)
    def rms_norm(self, x, w, eps) -> np.ndarray:
        x, w = np.ascontiguousarray(x, np.uint16), np.ascontiguousarray(w, np.uint16)
        out = np.empty_like(x)
        self.lib.orc_rms_norm(_p(x), _p(w), _p(out), x.size, eps)
        return out

    def rms_norm_heads(self, x, w, heads, head_dim, eps) -> np.ndarray:
        x, w = np.ascontiguousarray(x, np.uint16), np.ascontiguousarray(w, np.uint16)
        out = np.empty_like(x)
        self.lib.orc_rms_norm_heads(_p(x), _p(w), _p(out), heads, head_dim, eps)
        return out

    def rope(self, x, heads, head_dim, position, theta) -> np.ndarray:
        out = np.array(x, np.uint16, copy=True)
        self.lib.orc_rope(_p(out), heads, head_dim, position, theta)
        return out

    def swiglu(self, g, u) -> np.ndarray:
        g, u = np.ascontiguousarray(g, np.uint16), np.ascontiguousarray(u, np.uint16)
        out = np.empty_like(g)
        self.lib.orc_swiglu(_p(g), _p(u), _p(out), g.size)
        return out

    def add(self, t, d) -> np.ndarray:
        out = np.array(t, np.uint16, copy=True)
        d = np.ascontiguousarray(d, np.uint16)
        self.lib.orc_add_inplace(_p(out), _p(d), out.size)
        return out

    def store_kv(self, k, v, kc, vc, position) -> tuple:
        k, v = np.ascontiguousarray(k, np.uint16), np.ascontiguousarray(v, np.uint16)
        kc, vc = np.array(kc, np.uint16, copy=True), np.array(vc, np.uint16, copy=True)
        self.lib.orc_store_kv(_p(k), _p(v), _p(kc), _p(vc), position, k.size)
        return kc, vc

    def argmax(self, logits) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        return int(self.lib.orc_argmax(_p(logits), logits.size))


class RefLib:
    """The reference's own host fp16 and dequant routines (oracle/_ref)."""

    def __init__(self, path: str = REF_SO):
        self.lib = ctypes.CDLL(path)
        self.lib.ref_f2h_array.argtypes = [_P, c_uint64, _P]
        self.lib.ref_h2f_array.argtypes = [_P, c_uint64, _P]
        self.lib.ref_bf16_to_half_array.argtypes = [_P, c_uint64, _P]
        self.lib.ref_dequant_q4k.argtypes = [_P, c_uint64, c_uint64, _P]
        self.lib.ref_dequant_q6k.argtypes = [_P, c_uint64, c_uint64, _P]
        self.lib.ref_tensor_nbytes.argtypes = [ctypes.c_uint32, c_uint64]
        self.lib.ref_tensor_nbytes.restype = c_uint64
        self.lib.ref_matvec_dequant_dot.argtypes = [c_int, _P, _P, _P, c_int, c_int, c_int]
        self.lib.ref_matvec_dequant_dot.restype = None
        self.lib.ref_matvec_f16_dot.argtypes = [_P, _P, _P, c_int, c_int, c_int]
        self.lib.ref_matvec_f16_dot.restype = None

    @classmethod
    def try_load(cls):
        return cls() if os.path.exists(REF_SO) else None

    def f2h(self, f) -> np.ndarray:
        f = np.ascontiguousarray(f, dtype=np.float32)
        out = np.empty(f.shape, np.uint16)
        self.lib.ref_f2h_array(_p(f), f.size, _p(out))
        return out

    def h2f(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.ref_h2f_array(_p(h), h.size, _p(out))
        return out

    def dequant(self, kind: str, blocks: np.ndarray, count: int) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        out = np.empty(count, np.uint16)
        getattr(self.lib, f"ref_dequant_{kind}")(_p(blocks), blocks.size, count, _p(out))
        return out

    def matvec_dequant_dot(self, kind: str, w, x, in_f: int, out_f: int, nthreads: int) -> np.ndarray:
        """CPU baseline (i): the reference's dequant of each row, then an fp32 dot."""
        y = np.empty(out_f, np.float32)
        self.lib.ref_matvec_dequant_dot(12 if kind == "q4k" else 14, _p(w), _p(x), _p(y), in_f, out_f, nthreads)
        return y

    def matvec_f16_dot(self, wf16, x, in_f: int, out_f: int, nthreads: int) -> np.ndarray:
        """CPU baseline (ii): the fp32 dot over rows dequantised beforehand."""
        y = np.empty(out_f, np.float32)
        self.lib.ref_matvec_f16_dot(_p(wf16), _p(x), _p(y), in_f, out_f, nthreads)
        return y
