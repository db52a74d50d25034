"""Pins the oracle's GEMV and attention (kernels.cu:195-338, 545-649) against
brute-force numpy on small shapes and against closed forms."""
from __future__ import annotations

import numpy as np
import pytest


def _synth():
    from pycitlali import synth
    return synth


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_matvec_equals_numpy_dot_of_dequantised_rows(orc, kind):
    s = _synth()
    rng = s.Rng(3)
    n, k = 48, 768
    w = s.quant_matrix(kind, rng, n, k)
    x = s.normal_f16(rng, k)
    wf = orc.dequant_f32(kind, w, n * k).reshape(n, k).astype(np.float64)
    xf = x.view(np.float16).astype(np.float64)
    np.testing.assert_allclose(orc.matvec(kind, w, x, k, n), wf @ xf, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
def test_matvec_closed_forms(orc, kind):
    s = _synth()
    rng = s.Rng(4)
    n, k = 16, 512
    w = s.quant_matrix(kind, rng, n, k)
    wf = orc.dequant_f32(kind, w, n * k).reshape(n, k).astype(np.float64)
    ones = np.full(k, 0x3C00, np.uint16)
    np.testing.assert_allclose(orc.matvec(kind, w, ones, k, n), wf.sum(axis=1), rtol=1e-12)
    for col in (0, 255, 256, 511):
        e = np.zeros(k, np.uint16)
        e[col] = 0x3C00
        np.testing.assert_array_equal(orc.matvec(kind, w, e, k, n), wf[:, col])
    x = s.normal_f16(rng, k)
    x2 = (x.view(np.float16) * np.float16(2)).view(np.uint16)
    np.testing.assert_array_equal(orc.matvec(kind, w, x2, k, n), 2 * orc.matvec(kind, w, x, k, n))


def test_f16dot_baseline_uses_fp16_weights(orc):
    s = _synth()
    rng = s.Rng(5)
    n, k = 8, 512
    w = s.quant_matrix("q4k", rng, n, k)
    x = s.normal_f16(rng, k)
    w16 = orc.dequant_f16("q4k", w, n * k).view(np.float16).astype(np.float64).reshape(n, k)
    ref = w16 @ x.view(np.float16).astype(np.float64)
    np.testing.assert_allclose(orc.matvec_f16dot("q4k", w, x, k, n), ref, rtol=1e-4, atol=1e-3)


def numpy_attention(q, kc, vc, L, heads, kv_heads, hd):
    qf = q.view(np.float16).astype(np.float64).reshape(heads, hd)
    k = kc.view(np.float16).astype(np.float64)[: L * kv_heads * hd].reshape(L, kv_heads, hd)
    v = vc.view(np.float16).astype(np.float64)[: L * kv_heads * hd].reshape(L, kv_heads, hd)
    out = np.empty((heads, hd))
    g = heads // kv_heads
    for h in range(heads):
        s = k[:, h // g, :] @ qf[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = p @ v[:, h // g, :] / p.sum()
    return out.reshape(-1)


@pytest.mark.parametrize("heads,kv,hd,L", [(4, 2, 64, 37), (8, 8, 128, 5), (12, 4, 128, 200)])
def test_attention_equals_numpy_softmax(orc, heads, kv, hd, L):
    s = _synth()
    rng = s.Rng(L)
    kc = s.normal_f16(rng, L * kv * hd)
    vc = s.normal_f16(rng, L * kv * hd)
    q = s.normal_f16(rng, heads * hd)
    np.testing.assert_allclose(orc.attention(q, kc, vc, L - 1, heads, kv, hd),
                               numpy_attention(q, kc, vc, L, heads, kv, hd), rtol=1e-12, atol=1e-12)
    f32 = orc.attention_f32(q, kc, vc, L - 1, heads, kv, hd, 2)
    np.testing.assert_allclose(f32, numpy_attention(q, kc, vc, L, heads, kv, hd), rtol=1e-4, atol=1e-5)


def test_attention_closed_forms(orc):
    s = _synth()
    rng = s.Rng(9)
    heads, kv, hd, L = 8, 2, 64, 50
    kc = s.normal_f16(rng, L * kv * hd)
    vc = s.normal_f16(rng, L * kv * hd)
    q = s.normal_f16(rng, heads * hd)
    v = vc.view(np.float16).astype(np.float64).reshape(L, kv, hd)
    # one position -> V[0]
    np.testing.assert_array_equal(orc.attention(q, kc, vc, 0, heads, kv, hd).reshape(heads, hd),
                                  np.repeat(v[0], heads // kv, axis=0))
    # zero query -> mean of V
    z = np.zeros(heads * hd, np.uint16)
    np.testing.assert_allclose(orc.attention(z, kc, vc, L - 1, heads, kv, hd).reshape(heads, hd),
                               np.repeat(v.mean(axis=0), heads // kv, axis=0), rtol=1e-12, atol=1e-13)
