"""GPU parity of the fused-dequant GEMVs (kernels.cu:195-338) against the
oracle, through the C ABI.

Bar (north star): |gpu - ref| <= 2e-3 + 1e-2*|ref| with ref the exact fp32
weights accumulated in double; fp16 outputs additionally within one fp16
rounding of ref.  One-hot inputs pin the layout bit-exactly: with x = e_k and
fp32 output every kernel must return the fp32 weight column W[:, k] exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import tol_ok

pytestmark = pytest.mark.gpu

# (kind, out_features, in_features): BASELINE configs 1 and 3 plus edges
SHAPES = [
    ("q4k", 3072, 1024),     # cfg1: Qwen3-0.6B ffn_gate (nb = 4)
    ("q4k", 1024, 3072),     # same bytes, nb = 12 (ffn_down orientation)
    ("q4k", 4096, 4096),     # cfg3 attn_q / attn_o
    ("q4k", 1024, 4096),     # cfg3 attn_k
    ("q4k", 12288, 4096),    # cfg3 ffn_gate / ffn_up
    ("q6k", 1024, 4096),     # cfg3 attn_v
    ("q6k", 4096, 12288),    # cfg3 ffn_down (nb = 48)
    ("q6k", 1024, 1024),     # Qwen3-0.6B attn_v (nb = 4, 840-byte rows)
    ("q6k", 1024, 3072),     # Qwen3-0.6B ffn_down (nb = 12)
    ("q4k", 1, 256),         # one row, one block
    ("q6k", 1, 256),
    ("q4k", 37, 768),        # ragged rows, nb = 3
    ("q6k", 37, 768),
    # K = 4096 launch shapes: one pass with one / two rows per wave (<= 1024,
    # <= 4096 rows), streaming with one / two rows in flight (more rows)
    ("q4k", 7, 4096),
    ("q6k", 2500, 4096),
    ("q6k", 5000, 4096),
    ("q4k", 8192, 4096),
    ("q4k", 1030, 8192),     # nb = 32
    # rows shorter than one wave step (Qwen3-0.6B attn_o; more rows than one
    # pass covers: streamed)
    ("q4k", 1024, 2048),
    ("q6k", 6000, 1024),
    # rows of 4 and 8 blocks pack 4 / 2 rows per wave step: row counts that
    # leave a partial last unit, one pass and streamed
    ("q4k", 3, 1024),
    ("q6k", 4099, 1024),
    ("q4k", 16387, 1024),
    ("q4k", 5, 2048),
    ("q6k", 2049, 2048),
    ("q4k", 9001, 2048),
    # the other Qwen3 sizes: rows ending in a partial wave step
    ("q4k", 300, 2560),      # 4B hidden (nb = 10)
    ("q4k", 257, 5120),      # 14B / 32B hidden (nb = 20)
    ("q6k", 300, 6144),      # 1.7B FFN (nb = 24)
    ("q6k", 500, 9728),      # 4B FFN (nb = 38)
    ("q6k", 64, 17408),      # 14B FFN (nb = 68)
    ("q4k", 40, 25600),      # 32B FFN (nb = 100)
    ("q6k", 40, 25600),
    ("q6k", 3, 28672),       # the largest in_features the ABI takes
    ("q4k", 5, 28672),
]


def _inputs(hip, kind, n, k, seed):
    rng = hip.synth.Rng(seed)
    w = hip.synth.quant_matrix(kind, rng, n, k)
    x = hip.synth.normal_f16(rng, k)
    return w, x


@pytest.mark.parametrize("kind,n,k", SHAPES)
@pytest.mark.parametrize("f32_out", [False, True])
def test_matvec_matches_oracle(hip, orc, kind, n, k, f32_out):
    print(f"[matvec] kind={kind} n={n} k={k} f32={f32_out}", flush=True)
    w, x = _inputs(hip, kind, n, k, seed=1000 + n + k)
    dw = hip.DeviceArray.from_numpy(w)
    dx = hip.DeviceArray.from_numpy(x)
    dy = hip.DeviceArray(n * (4 if f32_out else 2))
    hip.device.matvec(kind, dw, dx, dy, k, n, f32_out=f32_out)
    got = dy.download(np.float32 if f32_out else np.uint16, n)
    if not f32_out:
        got = got.view(np.float16).astype(np.float64)
    ref = orc.matvec(kind, w, x, k, n)
    bad = ~tol_ok(got, ref)
    assert not bad.any(), f"{bad.sum()} rows out of tolerance, e.g. got {got[bad][:4]} ref {ref[bad][:4]}"
    # fp32 accumulation error (grows like sqrt(K)) plus, for fp16 outputs,
    # one nearest-even rounding: far inside the bar above
    err = np.abs(got - ref)
    acc = 1e-3 * np.sqrt(k / 4096.0) + 1e-5 * np.abs(ref)
    rnd = 0.0 if f32_out else 2.0 ** -11 * np.abs(ref)
    print(f"[matvec] max abs err {err.max():.3g}, max |y| {np.abs(ref).max():.3g}", flush=True)
    assert np.all(err <= acc + rnd)


@pytest.mark.parametrize("kind,n,k", [("q4k", 64, 1024), ("q6k", 64, 1024), ("q4k", 19, 3072), ("q6k", 19, 3072)])
def test_one_hot_input_returns_exact_weight_column(hip, orc, kind, n, k):
    w, _ = _inputs(hip, kind, n, k, seed=7)
    wf = orc.dequant_f32(kind, w, n * k).reshape(n, k)
    dw = hip.DeviceArray.from_numpy(w)
    dy = hip.DeviceArray(n * 4)
    rng = np.random.default_rng(3)
    for col in sorted(set([0, 1, 2, 3, 31, 32, 63, 64, 127, 128, 255, 256, k - 1] + list(rng.integers(0, k, 12)))):
        x = np.zeros(k, np.uint16)
        x[col] = 0x3C00  # 1.0
        dx = hip.DeviceArray.from_numpy(x)
        hip.device.matvec(kind, dw, dx, dy, k, n, f32_out=True)
        got = dy.download(np.float32, n)
        # equal values (a -0.0 weight sums with +0.0 lanes to +0.0, as in the
        # reference's tree reduction)
        np.testing.assert_array_equal(got, wf[:, col], err_msg=f"column {col}")


def test_linearity_and_row_sums(hip, orc):
    n, k = 256, 2048
    rng = hip.synth.Rng(11)
    w = hip.synth.quant_matrix("q4k", rng, n, k)
    x = hip.synth.normal_f16(rng, k)
    dw = hip.DeviceArray.from_numpy(w)
    dy = hip.DeviceArray(n * 4)
    # x = 1 gives the row sums of the fp32 weights
    ones = np.full(k, 0x3C00, np.uint16)
    hip.device.matvec("q4k", dw, hip.DeviceArray.from_numpy(ones), dy, k, n, f32_out=True)
    rs = orc.dequant_f32("q4k", w, n * k).reshape(n, k).astype(np.float64).sum(axis=1)
    assert np.all(tol_ok(dy.download(np.float32, n), rs, atol=1e-3, rtol=1e-5))
    # y(2x) == 2 y(x) exactly (power-of-two scaling commutes with rounding)
    x2 = (x.view(np.float16) * np.float16(2)).view(np.uint16)
    hip.device.matvec("q4k", dw, hip.DeviceArray.from_numpy(x), dy, k, n, f32_out=True)
    y1 = dy.download(np.float32, n)
    hip.device.matvec("q4k", dw, hip.DeviceArray.from_numpy(x2), dy, k, n, f32_out=True)
    np.testing.assert_array_equal(dy.download(np.float32, n), 2 * y1)


# BASELINE's full shapes: config 3's largest GEMVs and config 5's output
# GEMV (fp32 logits, 510 MB), through size-independent exact properties
FULL = [("q4k", 12288, 4096, False), ("q6k", 4096, 12288, False), ("q6k", 151936, 4096, True)]


@pytest.mark.parametrize("kind,n,k,f32", FULL)
def test_full_size_scaling_and_row_order(hip, kind, n, k, f32):
    """y(2x) = 2 y(x) bit for bit (power-of-two scaling commutes with every
    product, sum and rounding while nothing overflows and, for fp16 y, the
    value is a normal number: below 2^-14 the fp16 spacing is a fixed 2^-24,
    so there y(2x) is within one such step of 2 y(x)), and a matrix with its
    rows reversed gives the reversed y bit for bit (a row's result does not
    depend on which wave or workgroup computes it)."""
    rng = hip.synth.Rng(23)
    w = hip.synth.quant_matrix(kind, rng, n, k)
    x = hip.synth.normal_f16(rng, k)
    x2 = (x.view(np.float16) * np.float16(2)).view(np.uint16)
    dw = hip.DeviceArray.from_numpy(w)
    dy = hip.DeviceArray(n * 4)
    out = np.float32 if f32 else np.float16

    def run(wd, xv):
        hip.device.matvec(kind, wd, hip.DeviceArray.from_numpy(xv), dy, k, n, f32_out=f32)
        return dy.download(np.float32 if f32 else np.uint16, n).view(out).copy()

    y1 = run(dw, x)
    assert np.all(np.isfinite(y1))
    y2 = run(dw, x2)
    exact = np.ones(n, bool) if f32 else np.abs(y1.astype(np.float64)) >= 2.0 ** -14
    np.testing.assert_array_equal(y2[exact], y1[exact] * out(2))
    assert np.all(np.abs(y2[~exact].astype(np.float64) - 2 * y1[~exact].astype(np.float64)) <= 2.0 ** -24)
    dw.close()
    wr = np.ascontiguousarray(w.reshape(n, -1)[::-1])
    del w
    drev = hip.DeviceArray.from_numpy(wr)
    del wr
    np.testing.assert_array_equal(run(drev, x), y1[::-1])
    drev.close()
    dy.close()


def test_rows_permute_with_weights(hip):
    n, k = 96, 1024
    rng = hip.synth.Rng(5)
    w = hip.synth.quant_matrix("q6k", rng, n, k).reshape(n, -1)
    x = hip.synth.normal_f16(rng, k)
    perm = np.random.default_rng(0).permutation(n)
    dx = hip.DeviceArray.from_numpy(x)
    dy = hip.DeviceArray(n * 4)
    hip.device.matvec("q6k", hip.DeviceArray.from_numpy(w), dx, dy, k, n, f32_out=True)
    y = dy.download(np.float32, n)
    hip.device.matvec("q6k", hip.DeviceArray.from_numpy(np.ascontiguousarray(w[perm])), dx, dy, k, n, f32_out=True)
    np.testing.assert_array_equal(dy.download(np.float32, n), y[perm])
