"""GPU parity of the GEMVs whose input is a residual add + RMSNorm formed in
the launch itself (the reference's add_inplace + rms_norm before attn_q/k/v,
ffn_gate/up and the output, qwen_model.cpp:306, 340-341, 372, 385).  Each
must equal citlali_hip_add_rms_norm (or citlali_hip_rms_norm without a
delta) followed by the plain launch, bit for bit, and its sum_out must equal
the residual add_rms_norm leaves in x."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def up(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def inputs(hip, k, seed):
    rng = hip.synth.Rng(seed)
    x, d, w = (hip.synth.normal_f16(rng, k) for _ in range(3))
    return rng, x, d, w


def reference_norm(hip, x, d, w, k, eps=1e-6):
    """(normed input, residual) from the standalone launches."""
    dx, out = up(hip, x), hip.DeviceArray(k * 2)
    if d is None:
        hip.device.rms_norm(dx, up(hip, w), out, k, eps)
    else:
        hip.device.add_rms_norm(dx, up(hip, d), up(hip, w), out, k, eps)
    return out, dx.download(np.uint16, k)


@pytest.mark.parametrize("with_delta", [True, False])
@pytest.mark.parametrize("kinds,rows,k", [
    (("q4k", "q4k", "q6k"), (4096, 1024, 1024), 4096),   # Qwen3-8B attn_q/k/v
    (("q6k", "q4k"), (700, 9), 8192),
    (("q4k", "q4k", "q4k"), (300, 300, 300), 12288),
    (("q6k",), (64,), 16384),
    (("fp16", "fp16", "fp16"), (4096, 1024, 1024), 4096),
    (("fp16", "fp16"), (500, 20), 12288),
    (("q4k", "q4k", "q6k"), (2048, 1024, 1024), 1024),   # Qwen3-0.6B attn_q/k/v
    (("q6k",), (300,), 3072),
    (("fp16", "fp16", "fp16"), (2048, 1024, 1024), 1024),
    (("q4k", "q4k", "q6k"), (4096, 1024, 1024), 2560),   # Qwen3-4B
    (("q4k", "q6k"), (5120, 1024), 5120),                # Qwen3-14B
])
def test_group_norm_equals_add_rms_norm_then_group(hip, kinds, rows, k, with_delta):
    rng, x, d, w = inputs(hip, k, sum(rows) + k)
    d = d if with_delta else None
    ws = [up(hip, hip.synth.quant_matrix(kd, rng, n, k)) for kd, n in zip(kinds, rows)]
    normed, resid = reference_norm(hip, x, d, w, k)
    ref = [hip.DeviceArray(n * 2) for n in rows]
    hip.device.matvec_group(kinds, ws, normed, ref, rows, k)
    got = [hip.DeviceArray(n * 2) for n in rows]
    sum_out = up(hip, np.full(k, 0x7bff, np.uint16))
    hip.device.matvec_group_norm(kinds, ws, up(hip, x), up(hip, d) if d is not None else None, up(hip, w),
                                 sum_out if d is not None else None, 1e-6, got, rows, k)
    for g, r, n in zip(got, ref, rows):
        assert np.array_equal(g.download(np.uint16, n), r.download(np.uint16, n))
    if d is not None:
        assert np.array_equal(sum_out.download(np.uint16, k), resid)
    else:
        assert (sum_out.download(np.uint16, k) == 0x7bff).all()   # untouched


@pytest.mark.parametrize("kind,n,k", [("q4k", 12288, 4096), ("q6k", 1000, 8192), ("fp16", 12288, 4096),
                                      ("fp16", 900, 8192), ("q4k", 3072, 1024), ("q6k", 500, 2048),
                                      ("fp16", 3072, 1024), ("q4k", 9728, 2560), ("q4k", 2000, 5120),
                                      ("fp16", 1000, 5120)])
def test_gate_up_norm_equals_add_rms_norm_then_gate_up(hip, kind, n, k):
    rng, x, d, w = inputs(hip, k, n + k)
    wg, wu = (up(hip, hip.synth.quant_matrix(kind, rng, n, k)) for _ in range(2))
    normed, resid = reference_norm(hip, x, d, w, k)
    ref = hip.DeviceArray(n * 2)
    hip.device.matvec_gate_up_swiglu(kind, wg, wu, normed, ref, k, n)
    got, sum_out = hip.DeviceArray(n * 2), hip.DeviceArray(k * 2)
    hip.device.matvec_gate_up_swiglu_norm(kind, wg, wu, up(hip, x), up(hip, d), up(hip, w), sum_out, 1e-6, got, k, n)
    assert np.array_equal(got.download(np.uint16, n), ref.download(np.uint16, n))
    assert np.array_equal(sum_out.download(np.uint16, k), resid)


@pytest.mark.parametrize("f32_out", [True, False])
@pytest.mark.parametrize("kind,n,k", [("q6k", 30000, 4096), ("q4k", 5000, 4096), ("q6k", 777, 12288),
                                      ("q4k", 100, 16384), ("fp16", 30000, 4096), ("fp16", 333, 12288),
                                      ("q6k", 30000, 1024), ("q4k", 1000, 3072), ("fp16", 5000, 2048),
                                      ("q6k", 20000, 2560), ("q4k", 300, 5120)])
def test_matvec_norm_equals_add_rms_norm_then_matvec(hip, kind, n, k, f32_out):
    rng, x, d, w = inputs(hip, k, 3 * n + k)
    dw = up(hip, hip.synth.quant_matrix(kind, rng, n, k))
    normed, resid = reference_norm(hip, x, d, w, k)
    es = 4 if f32_out else 2
    ref, got = hip.DeviceArray(n * es), hip.DeviceArray(n * es)
    hip.device.matvec(kind, dw, normed, ref, k, n, f32_out=f32_out)
    sum_out = hip.DeviceArray(k * 2)
    hip.device.matvec_norm(kind, dw, up(hip, x), up(hip, d), up(hip, w), sum_out, 1e-6, got, k, n, f32_out=f32_out)
    dt = np.float32 if f32_out else np.uint16
    assert np.array_equal(got.download(dt, n).view(np.uint32 if f32_out else np.uint16),
                          ref.download(dt, n).view(np.uint32 if f32_out else np.uint16))
    assert np.array_equal(sum_out.download(np.uint16, k), resid)


def test_add_rms_norm_equals_add_then_rms_norm_at_every_length(hip):
    for n in (8, 100, 1024, 2048, 4096, 5000):
        rng = hip.synth.Rng(n)
        x, d, w = (hip.synth.normal_f16(rng, n) for _ in range(3))
        dx1, o1 = up(hip, x), hip.DeviceArray(n * 2)
        hip.device.add_inplace(dx1, up(hip, d), n)
        hip.device.rms_norm(dx1, up(hip, w), o1, n, 1e-6)
        dx2, o2 = up(hip, x), hip.DeviceArray(n * 2)
        hip.device.add_rms_norm(dx2, up(hip, d), up(hip, w), o2, n, 1e-6)
        assert np.array_equal(dx1.download(np.uint16, n), dx2.download(np.uint16, n)), n
        assert np.array_equal(o1.download(np.uint16, n), o2.download(np.uint16, n)), n


def test_norm_prologue_declines_other_lengths(hip):
    k, n = 1536, 64
    rng, x, d, w = inputs(hip, k, 1)
    dw = up(hip, hip.synth.quant_matrix("q4k", rng, n, k))
    y = up(hip, np.full(n, 0x3c00, np.uint16))
    with pytest.raises(hip.CitlaliError, match="no prologue kernel"):
        hip.device.matvec_norm("q4k", dw, up(hip, x), up(hip, d), up(hip, w), None, 1e-6, y, k, n)
    with pytest.raises(hip.CitlaliError, match="no grouped kernel"):
        hip.device.matvec_group_norm(["q4k"], [dw], up(hip, x), up(hip, d), up(hip, w), None, 1e-6, [y], [n], k)
    with pytest.raises(hip.CitlaliError, match="no fused kernel"):
        hip.device.matvec_gate_up_swiglu_norm("q4k", dw, dw, up(hip, x), up(hip, d), up(hip, w), None, 1e-6, y, k, n)
    assert (y.download(np.uint16, n) == 0x3c00).all()
