"""The C ABI without a GPU: the libraries load, export every symbol the
headers declare, and reject bad arguments before touching the device (the
failure cases of the reference's own checks: null buffers, in_features not
a multiple of 256, head_count % head_count_kv, position >= max_context)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_c_symbols():
    names = set()
    for fn in os.listdir(INCLUDE):
        if fn.endswith(".h"):
            text = open(os.path.join(INCLUDE, fn)).read()
            names.update(re.findall(r"\b(citlali_hip_\w+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    import pycitlali
    lib = pycitlali.load()
    names = declared_c_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", pycitlali._lib.HIP_LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (citlali_hip_\w+)", out))
    assert set(names) <= exported
    # the binding declares exactly the header's functions
    assert sorted(n for n, _, _ in pycitlali._lib.SIGNATURES) == names


def test_abi_version():
    import pycitlali
    assert pycitlali.load().citlali_hip_abi_version() == 1


def _status(fn, *args):
    import pycitlali
    lib = pycitlali.load()
    st = getattr(lib, fn)(*args)
    return st, pycitlali.last_error()


P = ctypes.c_void_p


@pytest.mark.parametrize("fn", ["citlali_hip_matvec_q4k", "citlali_hip_matvec_q6k", "citlali_hip_matvec_q4k_to_float",
                                "citlali_hip_matvec_q6k_to_float"])
def test_matvec_validation(fn):
    fake = P(0x10000)
    st, msg = _status(fn, P(0), fake, fake, 256, 4)
    assert st == 1 and "null buffer" in msg
    st, msg = _status(fn, fake, fake, fake, 1000, 4)
    assert st == 1 and "multiple of the 256-value super-block" in msg
    st, msg = _status(fn, fake, fake, fake, 0, 4)
    assert st == 1 and "positive" in msg
    st, msg = _status(fn, fake, fake, fake, 256, 0)
    assert st == 1
    st, msg = _status(fn, fake, fake, fake, 28672 + 256, 4)
    assert st == 1 and "exceeds" in msg
    st, msg = _status(fn, P(0x10001), fake, fake, 256, 4)
    assert st == 1 and "aligned" in msg


def test_matvec_group_validation():
    fake = P(0x10000)
    ints = lambda *v: (ctypes.c_int * len(v))(*v)
    ptrs = lambda *v: (ctypes.c_void_p * len(v))(*v)
    g = lambda n, types, ws, ys, rows, k: _status("citlali_hip_matvec_group", n, types, ws, fake, ys, rows, k)
    st, msg = g(0, ints(12), ptrs(0x10000), ptrs(0x10000), ints(4), 4096)
    assert st == 1 and "count" in msg
    st, msg = g(4, ints(12, 12, 12, 12), ptrs(*[0x10000] * 4), ptrs(*[0x10000] * 4), ints(4, 4, 4, 4), 4096)
    assert st == 1 and "count" in msg
    st, msg = g(2, ints(12, 10), ptrs(0x10000, 0x10000), ptrs(0x10000, 0x10000), ints(4, 4), 4096)
    assert st == 1 and "not Q4_K, Q6_K or F16" in msg
    st, msg = g(2, ints(12, 14), ptrs(0x10000, 0), ptrs(0x10000, 0x10000), ints(4, 4), 4096)
    assert st == 1 and "null buffer" in msg
    st, msg = g(1, ints(12), ptrs(0x10004), ptrs(0x10000), ints(4), 4096)
    assert st == 1 and "aligned" in msg
    st, msg = g(3, ints(14, 14, 14), ptrs(*[0x10000] * 3), ptrs(*[0x10000] * 3), ints(2 ** 30, 2 ** 30, 2 ** 30),
                4096)
    assert st == 1 and "INT_MAX" in msg
    st, msg = g(1, ints(14), ptrs(0x10000), ptrs(0x10000), ints(4), 1536)
    assert st == 2 and "no grouped kernel" in msg
    # fp16 weights (GGUF type 1): 16-byte aligned, never mixed with quantized ones
    st, msg = g(2, ints(1, 14), ptrs(0x10000, 0x10000), ptrs(0x10000, 0x10000), ints(4, 4), 4096)
    assert st == 2 and "F16 and quantized" in msg
    st, msg = g(1, ints(1), ptrs(0x10004), ptrs(0x10000), ints(4), 4096)
    assert st == 1 and "16-byte aligned" in msg
    st, msg = _status("citlali_hip_matvec_group", 1, None, ptrs(0x10000), fake, ptrs(0x10000), ints(4), 4096)
    assert st == 1 and "null array" in msg


def test_norm_prologue_validation():
    import pycitlali
    fake = P(0x10000)
    ints = lambda *v: (ctypes.c_int * len(v))(*v)
    ptrs = lambda *v: (ctypes.c_void_p * len(v))(*v)
    Norm = pycitlali._lib.Norm
    ok = Norm(0x20000, 0x30000, 0x40000, 1e-6)
    st, msg = _status("citlali_hip_matvec_norm", 12, fake, fake, None, fake, 0, 4096, 8)
    assert st == 1 and "null norm" in msg
    st, msg = _status("citlali_hip_matvec_norm", 12, fake, fake, ctypes.byref(Norm(0x20000, 0, 0, 1e-6)), fake, 0,
                      4096, 8)
    assert st == 1 and "norm weight" in msg
    st, msg = _status("citlali_hip_matvec_norm", 12, fake, fake, ctypes.byref(Norm(0x20004, 0x30000, 0, 1e-6)), fake,
                      0, 4096, 8)
    assert st == 1 and "delta must be 16-byte aligned" in msg
    st, msg = _status("citlali_hip_matvec_norm", 12, fake, fake, ctypes.byref(Norm(0x20000, 0x30000, 0x10000, 1e-6)),
                      fake, 0, 4096, 8)
    assert st == 1 and "sum_out must not be the input" in msg
    st, msg = _status("citlali_hip_matvec_norm", 10, fake, fake, ctypes.byref(ok), fake, 0, 4096, 8)
    assert st == 1 and "not Q4_K, Q6_K or F16" in msg
    st, msg = _status("citlali_hip_matvec_norm", 14, fake, fake, ctypes.byref(ok), fake, 1, 1536, 8)
    assert st == 2 and "no prologue kernel" in msg
    st, msg = _status("citlali_hip_matvec_group_norm", 1, ints(12), ptrs(0x10000), fake, ctypes.byref(ok),
                      ptrs(0x50000), ints(8), 20480)
    assert st == 2 and "no grouped kernel" in msg
    st, msg = _status("citlali_hip_matvec_group_norm", 0, ints(12), ptrs(0x10000), fake, ctypes.byref(ok),
                      ptrs(0x50000), ints(8), 4096)
    assert st == 1 and "count" in msg
    st, msg = _status("citlali_hip_matvec_gate_up_swiglu_norm", 12, fake, fake, fake, ctypes.byref(ok), P(0x50000),
                      12288, 8)
    assert st == 2 and "no fused kernel" in msg


def test_attention_validation():
    fake = P(0x10000)
    st, msg = _status("citlali_hip_attention", fake, fake, fake, fake, fake, 5, 5, 16, 8, 128)
    assert st == 1 and "position exceeds max_context" in msg
    st, msg = _status("citlali_hip_attention", fake, fake, fake, fake, fake, 0, 5, 12, 8, 128)
    assert st == 1 and "divisible" in msg
    st, msg = _status("citlali_hip_attention", fake, fake, fake, fake, fake, 0, 5, 16, 8, 96)
    assert st == 2 and "not built" in msg
    st, msg = _status("citlali_hip_attention", fake, fake, fake, fake, fake, 0, 5, 128, 8, 128)
    assert st == 2
    st, msg = _status("citlali_hip_attention", P(0), fake, fake, fake, fake, 0, 5, 16, 8, 128)
    assert st == 1 and "null" in msg


def test_embed_and_dequant_validation():
    fake = P(0x10000)
    st, msg = _status("citlali_hip_embed_q6k", fake, -1, fake, 1024)
    assert st == 1 and "vocab" in msg
    st, msg = _status("citlali_hip_embed_q6k", fake, 3, fake, 1000)
    assert st == 1
    st, msg = _status("citlali_hip_dequant_q4k_f16", P(0), ctypes.c_uint64(256), fake)
    assert st == 1


def test_workspace_query_is_host_only():
    import pycitlali
    lib = pycitlali.load()
    n = lib.citlali_hip_attention_workspace_bytes(32768, 16, 32, 8, 128)
    assert n > 0 and n % 4 == 0
    assert lib.citlali_hip_attention_workspace_bytes(64, 1, 32, 8, 128) == 0
    assert lib.citlali_hip_attention_workspace_bytes(100, 1, 12, 8, 128) == 0


def _plan_need(dev, bound, nseq, heads, kv, hd):
    _, n = dev.attention_plan_info(bound, nseq, heads, kv, hd)
    return 0 if n <= 1 else nseq * heads * n * (hd + 4) * 4


def test_workspace_covers_every_bucket_and_length():
    """The workspace query bounds the partials of the plan at every length up
    to its bound -- every power-of-two bucket a decode step plans for, and
    any max_positions_bound of the batched entry -- although the chunk count
    is not monotone in the length."""
    from pycitlali import device as dev
    # the counterexample of a bound sized by the plan at max_context alone:
    # 32/8/128 at max_context 3000 plans 24 chunks of 128, its 2048 bucket 32
    # chunks of 64
    assert dev.attention_plan_info(3000, 1, 32, 8, 128) == (128, 24)
    assert dev.attention_plan_info(2048, 1, 32, 8, 128) == (64, 32)
    assert dev.attention_workspace_bytes(3000, 1, 32, 8, 128) >= 32 * 32 * 132 * 4
    shapes = [(32, 8, 128), (16, 8, 128), (32, 4, 128), (40, 8, 128), (8, 8, 64), (16, 2, 64), (12, 12, 128)]
    for heads, kv, hd in shapes:
        for nseq in (1, 3, 16):
            prev = 0
            for m in list(range(1, 5000, 7)) + [8192, 8193, 12000, 32768, 40960, 131072]:
                ws = dev.attention_workspace_bytes(m, nseq, heads, kv, hd)
                assert ws >= prev, (heads, kv, hd, nseq, m)   # monotone in the bound
                prev = ws
                buckets = {dev.attention_plan_length(L, m) for L in (1, m)}
                b = 256
                while b < m:
                    buckets.add(b)
                    b *= 2
                for b in buckets:
                    assert _plan_need(dev, b, nseq, heads, kv, hd) <= ws, (heads, kv, hd, nseq, m, b)
                if m <= 4096 and m % 97 == 1:
                    for L in range(1, m + 1):
                        assert _plan_need(dev, L, nseq, heads, kv, hd) <= ws, (heads, kv, hd, nseq, m, L)


def test_device_array_fails_loudly_without_library(tmp_path, monkeypatch):
    import pycitlali._lib as L
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "HIP_LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(ImportError, match="not built"):
        L.load()


def test_synth_is_deterministic_and_shaped():
    from pycitlali import synth
    a = synth.quant_matrix("q4k", synth.Rng(0), 4, 512)
    b = synth.quant_matrix("q4k", synth.Rng(0), 4, 512)
    assert a.size == 4 * 2 * 144 and np.array_equal(a, b)
    d = a.reshape(-1, 144)[:, 0:2].copy().view(np.float16).astype(np.float64)
    assert np.all((d >= 1e-3 * 0.999) & (d <= 1e-2 * 1.001))
    z = synth.Rng(1).normal(200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_dispatch_timing_arguments():
    """Per-dispatch timing checks its arguments on the host and excludes the
    call-span timing (no HIP call: the events here are never used)."""
    import ctypes
    import pycitlali
    lib = pycitlali.load()
    arr = ctypes.c_void_p * 2
    fake = arr(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000))
    for n in (-1, 65):
        assert lib.citlali_hip_set_dispatch_timing(fake, fake, n) == pycitlali._lib.ERR_INVALID
        assert "outside [0, 64]" in pycitlali.last_error()
    assert lib.citlali_hip_set_dispatch_timing(None, fake, 1) == pycitlali._lib.ERR_INVALID
    assert "null event array" in pycitlali.last_error()
    assert lib.citlali_hip_set_dispatch_timing(fake, arr(ctypes.c_void_p(0x1000), None), 2) == pycitlali._lib.ERR_INVALID
    assert "null event in pair 1" in pycitlali.last_error()
    assert lib.citlali_hip_set_kernel_timing(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000)) == 0
    assert lib.citlali_hip_set_dispatch_timing(fake, fake, 2) == pycitlali._lib.ERR_INVALID
    assert "call-span timing is armed" in pycitlali.last_error()
    assert lib.citlali_hip_set_kernel_timing(None, None) == 0
    assert lib.citlali_hip_set_dispatch_timing(fake, fake, 2) == 0
    assert lib.citlali_hip_set_kernel_timing(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x2000)) == pycitlali._lib.ERR_INVALID
    assert "per-dispatch timing is armed" in pycitlali.last_error()
    cnt = ctypes.c_int(-1)
    assert lib.citlali_hip_dispatch_timing_count(ctypes.byref(cnt)) == 0 and cnt.value == 0
    assert lib.citlali_hip_set_dispatch_timing(None, None, 0) == 0
    assert lib.citlali_hip_dispatch_timing_count(None) == pycitlali._lib.ERR_INVALID


def test_kernel_timing_needs_both_events():
    import ctypes
    import pycitlali
    lib = pycitlali.load()
    st = lib.citlali_hip_set_kernel_timing(ctypes.c_void_p(0x1000), ctypes.c_void_p(0))
    assert st == pycitlali._lib.ERR_INVALID
    assert "both events" in pycitlali.last_error()
    assert lib.citlali_hip_set_kernel_timing(ctypes.c_void_p(0), ctypes.c_void_p(0)) == 0
