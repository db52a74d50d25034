"""Device memory and thin call wrappers over the C ABI.

DeviceArray mirrors the reference's DeviceBuffer (tensor.h:10-54): it owns
one device allocation, copies from/to host numpy arrays and frees on close.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


class DeviceArray:
    def __init__(self, nbytes: int):
        lib = _lib.load()
        p = ctypes.c_void_p()
        _lib.check(lib.citlali_hip_malloc(ctypes.byref(p), ctypes.c_size_t(int(nbytes))))
        self.ptr = p.value or 0
        self.nbytes = int(nbytes)

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(arr.nbytes)
        d.upload(arr)
        return d

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload exceeds the allocation")
        _lib.call("citlali_hip_memcpy_h2d", ctypes.c_void_p(self.ptr + offset), arr.ctypes.data_as(ctypes.c_void_p),
                  ctypes.c_size_t(arr.nbytes))

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download exceeds the allocation")
        _lib.call("citlali_hip_memcpy_d2h", out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr + offset),
                  ctypes.c_size_t(out.nbytes))
        return out

    def zero(self) -> None:
        _lib.call("citlali_hip_zero", ctypes.c_void_p(self.ptr), ctypes.c_size_t(self.nbytes))

    def at(self, offset: int) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.ptr + offset)

    @property
    def vp(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.ptr)

    def close(self) -> None:
        if self.ptr:
            _lib.load().citlali_hip_free(ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# GGUF type codes of the GEMV weight kinds
_GGUF_TYPE = {"q4k": 12, "q6k": 14, "fp16": 1}

def synchronize() -> None:
    _lib.call("citlali_hip_synchronize")


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        _lib.check(_lib.load().citlali_hip_event_create(ctypes.byref(p)))
        self.h = p

    def record(self) -> None:
        _lib.call("citlali_hip_event_record", self.h)

    def synchronize(self) -> None:
        _lib.call("citlali_hip_event_synchronize", self.h)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _lib.check(_lib.load().citlali_hip_event_elapsed_ms(self.h, end.h, ctypes.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            _lib.load().citlali_hip_event_destroy(self.h)
        except Exception:
            pass


class KernelTimer:
    """Kernel-own time of the library calls made inside `with timer:` (the
    first kernel's start to the last kernel's end, stamped by the dispatch).
    Use `ms()` after the stream has passed the calls."""

    def __init__(self):
        self.start, self.stop = Event(), Event()

    def __enter__(self):
        _lib.call("citlali_hip_set_kernel_timing", self.start.h, self.stop.h)
        return self

    def __exit__(self, *exc):
        _lib.call("citlali_hip_set_kernel_timing", ctypes.c_void_p(0), ctypes.c_void_p(0))
        return False

    def ms(self) -> float:
        self.stop.synchronize()
        return self.start.elapsed_ms(self.stop)


class DispatchTimer:
    """Each kernel's own time for the library calls made inside `with
    timer:`, stamped by its own dispatch (at most `n` kernels; more raise on
    exit).  `each_ms()` lists them in launch order, `ms()` is their sum: the
    kernels' durations without the gaps between them.  Use after the stream
    has passed the calls."""

    def __init__(self, n: int = 4):
        self.starts = [Event() for _ in range(n)]
        self.stops = [Event() for _ in range(n)]
        self.count = 0

    def __enter__(self):
        n = len(self.starts)
        arr = ctypes.c_void_p * n
        _lib.call("citlali_hip_set_dispatch_timing", arr(*[e.h for e in self.starts]),
                  arr(*[e.h for e in self.stops]), n)
        return self

    def __exit__(self, *exc):
        c = ctypes.c_int()
        _lib.call("citlali_hip_dispatch_timing_count", ctypes.byref(c))
        _lib.call("citlali_hip_set_dispatch_timing", None, None, 0)
        self.count = c.value
        if exc[0] is None and self.count > len(self.starts):
            raise RuntimeError(f"DispatchTimer: {self.count} kernels launched, {len(self.starts)} event pairs")
        return False

    def each_ms(self) -> list:
        out = []
        for i in range(self.count):
            self.stops[i].synchronize()
            out.append(self.starts[i].elapsed_ms(self.stops[i]))
        return out

    def ms(self) -> float:
        return sum(self.each_ms())


def _vp(x) -> ctypes.c_void_p:
    if isinstance(x, DeviceArray):
        return x.vp
    if isinstance(x, ctypes.c_void_p):
        return x
    return ctypes.c_void_p(int(x))


def matvec(kind: str, w, x, y, in_features: int, out_features: int, f32_out: bool = False) -> None:
    """kind in {"q4k", "q6k", "fp16"}; y fp16 unless f32_out."""
    name = {("q4k", False): "citlali_hip_matvec_q4k", ("q4k", True): "citlali_hip_matvec_q4k_to_float",
            ("q6k", False): "citlali_hip_matvec_q6k", ("q6k", True): "citlali_hip_matvec_q6k_to_float",
            ("fp16", False): "citlali_hip_matvec_fp16", ("fp16", True): "citlali_hip_matvec_fp16_to_float"}[
        (kind, bool(f32_out))]
    _lib.call(name, _vp(w), _vp(x), _vp(y), int(in_features), int(out_features))


def attention(q, k_cache, v_cache, scores, out, position: int, max_context: int, heads: int, kv_heads: int,
              head_dim: int) -> None:
    _lib.call("citlali_hip_attention", _vp(q), _vp(k_cache), _vp(v_cache),
              _vp(scores) if scores is not None else ctypes.c_void_p(0), _vp(out), int(position), int(max_context),
              int(heads), int(kv_heads), int(head_dim))


def attention_noalloc(q, k_cache, v_cache, out, position: int, max_context: int, heads: int, kv_heads: int,
                      head_dim: int) -> None:
    """citlali_hip_attention with the split partials in the library's static
    per-GPU scratch: allocates nothing."""
    _lib.call("citlali_hip_attention_noalloc", _vp(q), _vp(k_cache), _vp(v_cache), _vp(out), int(position),
              int(max_context), int(heads), int(kv_heads), int(head_dim))


def attention_workspace_bytes(max_positions_bound: int, nseq: int, heads: int, kv_heads: int, head_dim: int) -> int:
    return int(_lib.load().citlali_hip_attention_workspace_bytes(int(max_positions_bound), int(nseq), int(heads),
                                                                 int(kv_heads), int(head_dim)))


def attention_batched(q, k_cache, v_cache, seq_stride: int, positions, max_positions_bound: int, nseq: int,
                      heads: int, kv_heads: int, head_dim: int, workspace, workspace_bytes: int, out) -> None:
    _lib.call("citlali_hip_attention_batched", _vp(q), _vp(k_cache), _vp(v_cache), ctypes.c_longlong(seq_stride),
              _vp(positions), int(max_positions_bound), int(nseq), int(heads), int(kv_heads), int(head_dim),
              _vp(workspace) if workspace is not None else ctypes.c_void_p(0), ctypes.c_size_t(workspace_bytes),
              _vp(out))


def embed_q6k(table, token_id: int, out, hidden: int) -> None:
    _lib.call("citlali_hip_embed_q6k", _vp(table), ctypes.c_int32(token_id), _vp(out), int(hidden))


def dequant_f16(kind: str, w, count: int, out) -> None:
    name = "citlali_hip_dequant_q4k_f16" if kind == "q4k" else "citlali_hip_dequant_q6k_f16"
    _lib.call(name, _vp(w), ctypes.c_uint64(count), _vp(out))


# ---- the rest of forward_token (kernels.h:8-37 launchers) ----------------
def rms_norm(x, w, out, n: int, eps: float) -> None:
    _lib.call("citlali_hip_rms_norm", _vp(x), _vp(w), _vp(out), int(n), ctypes.c_float(eps))


def rms_norm_heads(x, w, out, heads: int, head_dim: int, eps: float) -> None:
    _lib.call("citlali_hip_rms_norm_heads", _vp(x), _vp(w), _vp(out), int(heads), int(head_dim),
              ctypes.c_float(eps))


def rope(data, heads: int, head_dim: int, position: int, theta: float) -> None:
    _lib.call("citlali_hip_rope", _vp(data), int(heads), int(head_dim), int(position), ctypes.c_float(theta))


def swiglu(gate, up, out, n: int) -> None:
    _lib.call("citlali_hip_swiglu", _vp(gate), _vp(up), _vp(out), int(n))


def add_inplace(target, delta, n: int) -> None:
    _lib.call("citlali_hip_add_inplace", _vp(target), _vp(delta), int(n))


def add_bias_inplace(target, bias, n: int) -> None:
    _lib.call("citlali_hip_add_bias_inplace", _vp(target), _vp(bias), int(n))


def store_kv(k, v, k_cache, v_cache, position: int, kv_size: int) -> None:
    _lib.call("citlali_hip_store_kv", _vp(k), _vp(v), _vp(k_cache), _vp(v_cache), int(position), int(kv_size))


def embed(table, token_id: int, out, hidden: int) -> None:
    _lib.call("citlali_hip_embed", _vp(table), ctypes.c_int32(token_id), _vp(out), int(hidden))


def copy(src, dst, n: int) -> None:
    _lib.call("citlali_hip_copy", _vp(src), _vp(dst), int(n))


def argmax(logits, n: int, out_index) -> None:
    """Index of the first largest finite value of `n` fp32 logits, written to
    the device int32 `out_index` (0 when none is finite)."""
    _lib.call("citlali_hip_argmax", _vp(logits), int(n), _vp(out_index))


# ---- fused forward_token steps (same results as the separate launches) ----
def add_rms_norm(x, delta, w, out, n: int, eps: float) -> None:
    _lib.call("citlali_hip_add_rms_norm", _vp(x), _vp(delta), _vp(w), _vp(out), int(n), ctypes.c_float(eps))


def qk_norm_rope_store(q, k, v, q_norm, k_norm, heads: int, kv_heads: int, head_dim: int, position: int,
                       theta: float, eps: float, k_cache, v_cache) -> None:
    null = ctypes.c_void_p(0)
    _lib.call("citlali_hip_qk_norm_rope_store", _vp(q), _vp(k), _vp(v), _vp(q_norm) if q_norm is not None else null,
              _vp(k_norm) if k_norm is not None else null, int(heads), int(kv_heads), int(head_dim), int(position),
              ctypes.c_float(theta), ctypes.c_float(eps), _vp(k_cache), _vp(v_cache))


def matvec_gate_up_swiglu(kind: str, w_gate, w_up, x, act, in_features: int, out_features: int) -> None:
    _lib.call("citlali_hip_matvec_gate_up_swiglu", _GGUF_TYPE[kind], _vp(w_gate), _vp(w_up), _vp(x),
              _vp(act), int(in_features), int(out_features))


def matvec_group(kinds, weights, x, outputs, out_features, in_features: int) -> None:
    """One launch of up to three Q4_K/Q6_K GEMVs that read `x`."""
    n = len(kinds)
    types = (ctypes.c_int * n)(*[_GGUF_TYPE[k] for k in kinds])
    ws = (ctypes.c_void_p * n)(*[w.ptr for w in weights])
    ys = (ctypes.c_void_p * n)(*[y.ptr for y in outputs])
    rows = (ctypes.c_int * n)(*[int(r) for r in out_features])
    _lib.call("citlali_hip_matvec_group", n, types, ws, _vp(x), ys, rows, int(in_features))


# ---- replayable decode steps: inputs read from device memory --------------
def attention_plan_length(length: int, max_context: int) -> int:
    return int(_lib.load().citlali_hip_attention_plan_length(int(length), int(max_context)))


def attention_plan_info(max_positions_bound: int, nseq: int, heads: int, kv_heads: int,
                        head_dim: int) -> tuple[int, int]:
    """(chunk, n_splits) of the batched attention plan for this bound."""
    chunk, n = ctypes.c_int(0), ctypes.c_int(0)
    _lib.check(_lib.load().citlali_hip_attention_plan_info(int(max_positions_bound), int(nseq), int(heads),
                                                           int(kv_heads), int(head_dim), ctypes.byref(chunk),
                                                           ctypes.byref(n)))
    return chunk.value, n.value


def argmax_advance(logits, n: int, state, tokens, capacity: int) -> None:
    """argmax, then tokens[step] = pick, token = pick, position += 1, step += 1
    in the device int32 state {token, position, step, 0}."""
    _lib.call("citlali_hip_argmax_advance", _vp(logits), int(n), _vp(state),
              _vp(tokens) if tokens is not None else ctypes.c_void_p(0), int(capacity))


def embed_q6k_at(table, token, vocab: int, out, hidden: int) -> None:
    _lib.call("citlali_hip_embed_q6k_at", _vp(table), _vp(token), int(vocab), _vp(out), int(hidden))


def embed_at(table, token, vocab: int, out, hidden: int) -> None:
    _lib.call("citlali_hip_embed_at", _vp(table), _vp(token), int(vocab), _vp(out), int(hidden))


def qk_norm_rope_store_at(q, k, v, q_norm, k_norm, heads: int, kv_heads: int, head_dim: int, position,
                          max_positions: int, theta: float, eps: float, k_cache, v_cache) -> None:
    null = ctypes.c_void_p(0)
    _lib.call("citlali_hip_qk_norm_rope_store_at", _vp(q), _vp(k), _vp(v),
              _vp(q_norm) if q_norm is not None else null, _vp(k_norm) if k_norm is not None else null, int(heads),
              int(kv_heads), int(head_dim), _vp(position), int(max_positions), ctypes.c_float(theta),
              ctypes.c_float(eps), _vp(k_cache), _vp(v_cache))


def qk_norm_rope_store_attention(q, k, v, q_norm, k_norm, heads: int, kv_heads: int, head_dim: int, position,
                                 plan_length: int, max_context: int, theta: float, eps: float, k_cache, v_cache,
                                 workspace, workspace_bytes: int, out) -> None:
    """qk_norm_rope_store(_at) + attention(_batched) in one launch; `position`
    is an int (scalar form) or a device int32 (then plan_length is the
    bucket)."""
    null = ctypes.c_void_p(0)
    scalar = isinstance(position, int)
    _lib.call("citlali_hip_qk_norm_rope_store_attention", _vp(q), _vp(k), _vp(v),
              _vp(q_norm) if q_norm is not None else null, _vp(k_norm) if k_norm is not None else null, int(heads),
              int(kv_heads), int(head_dim), int(position) if scalar else 0, null if scalar else _vp(position),
              int(plan_length), int(max_context), ctypes.c_float(theta), ctypes.c_float(eps), _vp(k_cache),
              _vp(v_cache), _vp(workspace) if workspace is not None else null, ctypes.c_size_t(workspace_bytes),
              _vp(out))


class Stream:
    """A HIP stream of the library (citlali_hip_stream_create)."""

    def __init__(self):
        h = ctypes.c_void_p()
        _lib.call("citlali_hip_stream_create", ctypes.byref(h))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            _lib.call("citlali_hip_stream_destroy", self.handle)
            self.handle = None


def set_stream(stream) -> None:
    _lib.check(_lib.load().citlali_hip_set_stream(stream.handle if stream is not None else None))


class Graph:
    """Launches captured on the library stream (citlali_hip_graph_begin/end)."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def capture(fn) -> "Graph":
        _lib.call("citlali_hip_graph_begin")
        try:
            fn()
        except BaseException:
            h = ctypes.c_void_p()   # end the capture; drop what it made
            if _lib.load().citlali_hip_graph_end(ctypes.byref(h)) == _lib.OK and h:
                _lib.load().citlali_hip_graph_destroy(h)
            raise
        h = ctypes.c_void_p()
        _lib.call("citlali_hip_graph_end", ctypes.byref(h))
        return Graph(h)

    def launch(self) -> None:
        _lib.call("citlali_hip_graph_launch", self.handle)

    def close(self) -> None:
        if self.handle:
            _lib.call("citlali_hip_graph_destroy", self.handle)
            self.handle = None


# ---- GEMVs with the residual add + RMSNorm prologue -------------------------
def _norm(delta, weight, sum_out, eps):
    nv = lambda a: a.ptr if a is not None else None
    return _lib.Norm(nv(delta), nv(weight), nv(sum_out), float(eps))


def matvec_group_norm(kinds, weights, x, delta, weight, sum_out, eps, outputs, out_features, in_features) -> None:
    n = len(kinds)
    types = (ctypes.c_int * n)(*[_GGUF_TYPE[k] for k in kinds])
    ws = (ctypes.c_void_p * n)(*[w.ptr for w in weights])
    ys = (ctypes.c_void_p * n)(*[y.ptr for y in outputs])
    rows = (ctypes.c_int * n)(*[int(r) for r in out_features])
    nrm = _norm(delta, weight, sum_out, eps)
    _lib.call("citlali_hip_matvec_group_norm", n, types, ws, _vp(x), ctypes.byref(nrm), ys, rows, int(in_features))


def matvec_gate_up_swiglu_norm(kind, w_gate, w_up, x, delta, weight, sum_out, eps, act, in_features: int,
                               out_features: int) -> None:
    nrm = _norm(delta, weight, sum_out, eps)
    _lib.call("citlali_hip_matvec_gate_up_swiglu_norm", _GGUF_TYPE[kind], _vp(w_gate), _vp(w_up), _vp(x),
              ctypes.byref(nrm), _vp(act), int(in_features), int(out_features))


def matvec_norm(kind, w, x, delta, weight, sum_out, eps, y, in_features: int, out_features: int,
                f32_out: bool = False) -> None:
    nrm = _norm(delta, weight, sum_out, eps)
    _lib.call("citlali_hip_matvec_norm", _GGUF_TYPE[kind], _vp(w), _vp(x), ctypes.byref(nrm), _vp(y),
              1 if f32_out else 0, int(in_features), int(out_features))

