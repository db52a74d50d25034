"""Pins of the oracle's forward_token helpers (kernels.cu:53-124, 474-533;
qwen_model.cpp:455-463) by closed forms, invariants and numpy's own
float -> fp16 casts.  Each check is chosen so a plausible slip (a missing
square root, sum instead of mean, the wrong rotation pair, the wrong weight
index, a last-instead-of-first tie rule) fails it."""
import math

import numpy as np
import pytest

H = np.float16


def bits(a):
    return np.asarray(a, H).view(np.uint16)


def vals(b):
    return np.asarray(b, np.uint16).view(H).astype(np.float64)


# ---- rms_norm (kernels.cu:67-93) -------------------------------------------
def test_rms_norm_known_answer(orc):
    # x = [3, 4]: rms = sqrt(12.5); out = x / rms exactly, then RNE to fp16
    out = orc.rms_norm(bits([3, 4]), bits([1, 1]), 0.0)
    exact = [3 / math.sqrt(12.5), 4 / math.sqrt(12.5)]
    assert np.array_equal(out, bits(np.array(exact, np.float64)))


def test_rms_norm_constant_vector_is_unit(orc):
    n = 4096
    for c in (0.5, -3.0, 1e-2):
        out = orc.rms_norm(bits(np.full(n, c)), bits(np.ones(n)), 1e-6)
        ref = c / math.sqrt(c * c + 1e-6)   # a sum instead of a mean would give ~1/64
        assert np.all(out == bits(np.float64(ref)))


def test_rms_norm_weight_is_elementwise_and_scale_invariant(orc, synth):
    rng = synth.Rng(3)
    n = 1024
    x = synth.normal_f16(rng, n)
    w = synth.normal_f16(rng, n)
    base = vals(orc.rms_norm(x, w, 0.0))
    # doubling the weights doubles every output exactly (outside the fp16
    # subnormal range, where the rounding step does not scale); scaling x by
    # 4 changes nothing (eps = 0)
    doubled = vals(orc.rms_norm(x, bits(2 * vals(w)), 0.0))
    normal = np.abs(base) >= 2.0 ** -14
    assert normal.sum() > 1000 * 0.99
    assert np.array_equal(doubled[normal], 2 * base[normal])
    assert np.all(np.abs(doubled - 2 * base) <= 2.0 ** -24)
    assert np.array_equal(orc.rms_norm(bits(4 * vals(x)), w, 0.0), bits(base))
    # permuting x and w together permutes the output (weight index = element index)
    p = np.random.default_rng(0).permutation(n)
    assert np.array_equal(orc.rms_norm(x[p], w[p], 0.0), bits(base)[p])


def test_rms_norm_zero_input_is_zero(orc):
    out = orc.rms_norm(np.zeros(64, np.uint16), bits(np.ones(64)), 1e-6)
    assert np.all(out == 0)


def test_rms_norm_heads_is_per_head_with_shared_weight(orc, synth):
    rng = synth.Rng(4)
    heads, hd = 8, 128
    x = synth.normal_f16(rng, heads * hd)
    x[hd:2 * hd] = bits(10 * vals(x[hd:2 * hd]))   # one head with a different scale
    w = synth.normal_f16(rng, hd)
    out = orc.rms_norm_heads(x, w, heads, hd, 1e-6)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        assert np.array_equal(out[sl], orc.rms_norm(x[sl], w, 1e-6))


# ---- rope (kernels.cu:485-521) ----------------------------------------------
def test_rope_position_zero_is_identity(orc, synth):
    x = synth.normal_f16(synth.Rng(5), 4 * 128)
    assert np.array_equal(orc.rope(x, 4, 128, 0, 1e6), x)


@pytest.mark.parametrize("i", [0, 1, 17, 63])
def test_rope_one_hot_rotates_pair_i_and_i_plus_half(orc, i):
    hd, pos, theta = 128, 37, 1e6
    x = np.zeros(hd, np.uint16)
    x[i] = bits(1.0)
    out = vals(orc.rope(x, 1, hd, pos, theta))
    ang = pos * theta ** (-2 * i / hd)
    expect = np.zeros(hd)
    expect[i], expect[i + hd // 2] = math.cos(ang), math.sin(ang)
    assert np.all(np.abs(out - expect) <= 2 ** -11 * np.abs(expect) + 2 ** -24 + 1e-6)


def test_rope_preserves_pair_norms(orc, synth):
    heads, hd = 4, 128
    x = synth.normal_f16(synth.Rng(6), heads * hd)
    out = vals(orc.rope(x, heads, hd, 1234, 1e6)).reshape(heads, 2, hd // 2)
    xin = vals(x).reshape(heads, 2, hd // 2)
    n0 = np.hypot(xin[:, 0], xin[:, 1])
    n1 = np.hypot(out[:, 0], out[:, 1])
    assert np.all(np.abs(n1 - n0) <= 2 ** -10 * n0 + 1e-4)


# ---- swiglu (kernels.cu:474-482) ---------------------------------------------
def test_swiglu_closed_forms(orc):
    g = bits([0.0, 1.0, 20.0, -20.0, 2.0])
    u = bits([5.0, 1.0, 1.0, 1.0, 0.0])
    out = vals(orc.swiglu(g, u))
    silu1 = 1 / (1 + math.exp(-1))
    assert out[0] == 0 and out[4] == 0
    assert out[1] == float(H(silu1))
    assert out[2] == float(H(20 / (1 + math.exp(-20))))
    assert abs(out[3]) < 1e-6


# ---- add (kernels.cu:53-65) --------------------------------------------------
def test_add_is_fp32_sum_rounded_nearest_even(orc, synth):
    rng = synth.Rng(7)
    a = synth.normal_f16(rng, 1 << 16)
    b = synth.normal_f16(rng, 1 << 16)
    ref = (a.view(H).astype(np.float32) + b.view(H).astype(np.float32)).astype(H).view(np.uint16)
    assert np.array_equal(orc.add(a, b), ref)
    assert np.array_equal(orc.add(a, np.zeros_like(a)), a)


# ---- store_kv (kernels.cu:524-533) -------------------------------------------
def test_store_kv_writes_one_row(orc, synth):
    rng = synth.Rng(8)
    kv, ctx, pos = 1024, 16, 9
    kc, vc = synth.normal_f16(rng, ctx * kv), synth.normal_f16(rng, ctx * kv)
    k, v = synth.normal_f16(rng, kv), synth.normal_f16(rng, kv)
    kc2, vc2 = orc.store_kv(k, v, kc, vc, pos)
    for new, old, row in ((kc2, kc, k), (vc2, vc, v)):
        new, old = new.reshape(ctx, kv), old.reshape(ctx, kv)
        assert np.array_equal(new[pos], row)
        assert np.array_equal(np.delete(new, pos, 0), np.delete(old, pos, 0))


# ---- greedy argmax (qwen_model.cpp:455-463) ----------------------------------
def test_argmax_rule(orc):
    assert orc.argmax(np.array([1, 5, 5, 2], np.float32)) == 1            # first of equal maxima
    assert orc.argmax(np.array([np.nan, np.inf, 3, -np.inf], np.float32)) == 2
    assert orc.argmax(np.array([np.nan, np.inf, -np.inf], np.float32)) == 0
    assert orc.argmax(np.array([-3e38, -np.inf], np.float32)) == 0
    r = np.random.default_rng(1)
    for _ in range(50):
        x = r.integers(-20, 20, 1000).astype(np.float32)
        x[r.integers(0, 1000, 30)] = np.nan
        x[r.integers(0, 1000, 5)] = np.inf
        masked = np.where(np.isfinite(x), x, -np.inf)
        assert orc.argmax(x) == int(np.argmax(masked))
