"""citlali_hip_attention_noalloc: decode attention that allocates nothing
(its split partials live in the library's static per-GPU scratch), through
the C ABI.

Bar: the same results as citlali_hip_attention bit for bit (same plan and
kernels), on calls in a row whose second input is smaller (the scratch keeps
the first call's partials; nothing of them may leak into the second), and
within |gpu - ref| <= 2e-3 + 1e-2*|ref| of the oracle.  A plan whose partials
exceed the scratch is rejected on the host, before any launch.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import tol_ok


def _inputs(hip, seed, L, heads, kv, hd):
    rng = hip.synth.Rng(seed)
    q = hip.synth.normal_f16(rng, heads * hd)
    k = hip.synth.normal_f16(rng, L * kv * hd)
    v = hip.synth.normal_f16(rng, L * kv * hd)
    return q, k, v


def _both(hip, q, k, v, L, heads, kv, hd):
    """(noalloc output, citlali_hip_attention output) as fp16 bit patterns"""
    dq, dk, dv = (hip.DeviceArray.from_numpy(a) for a in (q, k, v))
    out_n, out_a = hip.DeviceArray(heads * hd * 2), hip.DeviceArray(heads * hd * 2)
    scores = hip.DeviceArray(heads * L * 4)
    hip.device.attention_noalloc(dq, dk, dv, out_n, L - 1, L, heads, kv, hd)
    hip.device.attention(dq, dk, dv, scores, out_a, L - 1, L, heads, kv, hd)
    got = out_n.download(np.uint16, heads * hd), out_a.download(np.uint16, heads * hd)
    for a in (dq, dk, dv, out_n, out_a, scores):
        a.close()
    return got


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [
    ((32, 8, 128, 8192), (16, 8, 128, 1000)),    # config 3, then config 2's shape at a shorter length
    ((32, 4, 128, 16384), (32, 8, 128, 300)),    # 64 chunks, then a plan that fits one chunk
    ((16, 2, 64, 40000), (16, 8, 64, 700)),      # head_dim 64 (the VALU kernel)
])
def test_noalloc_equals_attention_on_calls_in_a_row(hip, orc, first, second):
    for i, (heads, kv, hd, L) in enumerate((first, second)):
        print(f"[attention_noalloc] call {i}: heads={heads} kv={kv} hd={hd} L={L}", flush=True)
        q, k, v = _inputs(hip, 1000 + 17 * i + L, L, heads, kv, hd)
        noalloc, plain = _both(hip, q, k, v, L, heads, kv, hd)
        assert np.array_equal(noalloc, plain), f"call {i}: differs from citlali_hip_attention"
        ref = orc.attention(q, k, v, L - 1, heads, kv, hd)
        assert np.all(tol_ok(noalloc.view(np.float16), ref)), f"call {i}: out of tolerance"


def test_noalloc_rejects_plans_beyond_the_scratch():
    """64 query heads at 524288 positions plan 512 chunks: 64 * 512 * 132 * 4
    bytes of partials, more than the 16 MiB scratch.  Checked on the host:
    fake device pointers, nothing launched, no GPU needed."""
    import pycitlali
    from pycitlali import device as dev
    lib = pycitlali.load()
    fake = ctypes.c_void_p(0x10000)
    L = 524288
    assert dev.attention_plan_info(dev.attention_plan_length(L, L), 1, 64, 8, 128) == (1024, 512)
    st = lib.citlali_hip_attention_noalloc(fake, fake, fake, fake, L - 1, L, 64, 8, 128)
    assert st == pycitlali._lib.ERR_INVALID
    msg = pycitlali.last_error()
    assert "scratch" in msg and str(64 * 512 * 132 * 4) in msg
    # every plan of up to 32 query heads fits: the library's own bound over
    # every plan length up to the largest position it accepts
    for bound in (L, 1 << 30, (1 << 31) - 1):
        for hd in (128, 64):
            assert dev.attention_workspace_bytes(bound, 1, 32, 8, hd) <= 16 << 20, (bound, hd)
    assert dev.attention_workspace_bytes(L, 1, 64, 8, 128) > 16 << 20
