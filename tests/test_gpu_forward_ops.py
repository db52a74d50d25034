"""GPU parity of the forward_token helpers (kernels.cu:27-124, 474-533 and
the host argmax of qwen_model.cpp:455-463) through the C ABI, against the
oracle.  Bit-exact where the arithmetic is one fp32 operation and a
nearest-even store (add, copy, embed, store_kv, argmax); within the
north-star bar, and mostly within one fp16 step, elsewhere."""
import math

import numpy as np
import pytest

from conftest import tol_ok

pytestmark = pytest.mark.gpu
H = np.float16


def vals(b):
    return np.asarray(b, np.uint16).view(H).astype(np.float64)


def up(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def ulps(got_bits, ref_bits):
    """Distance in fp16 steps (same-sign values)."""
    g = np.asarray(got_bits, np.int64)
    r = np.asarray(ref_bits, np.int64)
    g = np.where(g & 0x8000, -(g & 0x7fff), g)
    r = np.where(r & 0x8000, -(r & 0x7fff), r)
    return np.abs(g - r)


@pytest.mark.parametrize("n", [1024, 4096, 5120])
def test_rms_norm(hip, orc, n):
    rng = hip.synth.Rng(100 + n)
    x, w = hip.synth.normal_f16(rng, n), hip.synth.normal_f16(rng, n)
    dx, dw, do = up(hip, x), up(hip, w), hip.DeviceArray(n * 2)
    hip.device.rms_norm(dx, dw, do, n, 1e-6)
    got = do.download(np.uint16, n)
    ref = orc.rms_norm(x, w, 1e-6)
    assert np.all(tol_ok(vals(got), vals(ref)))
    assert ulps(got, ref).max() <= 1


@pytest.mark.parametrize("heads,hd", [(32, 128), (8, 128), (16, 64)])
def test_rms_norm_heads(hip, orc, heads, hd):
    rng = hip.synth.Rng(7 * heads + hd)
    x, w = hip.synth.normal_f16(rng, heads * hd), hip.synth.normal_f16(rng, hd)
    dx, dw, do = up(hip, x), up(hip, w), hip.DeviceArray(heads * hd * 2)
    hip.device.rms_norm_heads(dx, dw, do, heads, hd, 1e-6)
    got = do.download(np.uint16, heads * hd)
    ref = orc.rms_norm_heads(x, w, heads, hd, 1e-6)
    assert ulps(got, ref).max() <= 1


@pytest.mark.parametrize("position", [0, 1, 37, 1000, 8191])
@pytest.mark.parametrize("heads,hd", [(32, 128), (8, 128), (16, 64)])
def test_rope(hip, orc, heads, hd, position):
    theta = 1e6
    rng = hip.synth.Rng(position * 31 + heads)
    x = hip.synth.normal_f16(rng, heads * hd)
    d = up(hip, x)
    hip.device.rope(d, heads, hd, position, theta)
    got = vals(d.download(np.uint16, heads * hd))
    ref = vals(orc.rope(x, heads, hd, position, theta))
    if position == 0:
        assert np.array_equal(got, vals(x))
        return
    # The fp32 inverse frequency theta^(-2i/hd) is within ~2 ulp of exact in
    # any powf, so the angle is known to ~angle * 2^-22; the pair norm bounds
    # what that moves.
    half = hd // 2
    xs = vals(x).reshape(heads, 2, half)
    norm = np.hypot(xs[:, 0], xs[:, 1])
    ang = position * theta ** (-2 * np.arange(half) / hd)
    slack = (norm * ang * 2.0 ** -22)[:, None, :].repeat(2, 1).reshape(-1)
    assert np.all(np.abs(got - ref) <= 2e-3 + 1e-2 * np.abs(ref) + slack)


def test_swiglu(hip, orc):
    n = 12288
    rng = hip.synth.Rng(9)
    g, u = hip.synth.normal_f16(rng, n), hip.synth.normal_f16(rng, n)
    g[:4] = np.array([0.0, 20.0, -20.0, 11.0], H).view(np.uint16)
    dg, du, do = up(hip, g), up(hip, u), hip.DeviceArray(n * 2)
    hip.device.swiglu(dg, du, do, n)
    got = do.download(np.uint16, n)
    ref = orc.swiglu(g, u)
    assert np.all(tol_ok(vals(got), vals(ref)))
    assert ulps(got, ref).max() <= 1


@pytest.mark.parametrize("fn", ["add_inplace", "add_bias_inplace"])
def test_add_is_bit_exact(hip, orc, fn):
    n = 4096 + 5
    rng = hip.synth.Rng(11)
    t, dlt = hip.synth.normal_f16(rng, n), hip.synth.normal_f16(rng, n)
    dt, dd = up(hip, t), up(hip, dlt)
    getattr(hip.device, fn)(dt, dd, n)
    assert np.array_equal(dt.download(np.uint16, n), orc.add(t, dlt))


def test_store_kv_copy_and_embed_are_exact(hip, orc):
    rng = hip.synth.Rng(12)
    kv, ctx, pos = 1024, 32, 17
    kc, vc = hip.synth.normal_f16(rng, ctx * kv), hip.synth.normal_f16(rng, ctx * kv)
    k, v = hip.synth.normal_f16(rng, kv), hip.synth.normal_f16(rng, kv)
    dkc, dvc = up(hip, kc), up(hip, vc)
    hip.device.store_kv(up(hip, k), up(hip, v), dkc, dvc, pos, kv)
    rk, rv = orc.store_kv(k, v, kc, vc, pos)
    assert np.array_equal(dkc.download(np.uint16, ctx * kv), rk)
    assert np.array_equal(dvc.download(np.uint16, ctx * kv), rv)
    # fp16 embedding row and plain copy
    hidden, vocab = 1024, 40
    table = hip.synth.normal_f16(rng, vocab * hidden)
    out = hip.DeviceArray(hidden * 2)
    hip.device.embed(up(hip, table), 33, out, hidden)
    assert np.array_equal(out.download(np.uint16, hidden), table[33 * hidden:34 * hidden])
    src = up(hip, table)
    dst = hip.DeviceArray(table.nbytes)
    hip.device.copy(src, dst, table.size)
    assert np.array_equal(dst.download(np.uint16, table.size), table)


def _argmax(hip, logits):
    d = up(hip, logits.astype(np.float32))
    o = hip.DeviceArray(4)
    hip.device.argmax(d, logits.size, o)
    return int(o.download(np.int32, 1)[0])


def test_argmax_matches_host_rule(hip, orc):
    r = np.random.default_rng(5)
    for n in (1, 7, 1000, 151936):
        x = r.standard_normal(n).astype(np.float32)
        if n > 10:
            top = np.float32(x.max() + 1)
            idx = np.sort(r.choice(n, 3, replace=False))
            x[idx] = top                                     # ties: the first wins
            x[r.choice(n, 5)] = np.nan
            x[r.choice(n, 2)] = np.inf
        assert _argmax(hip, x) == orc.argmax(x), n
    assert _argmax(hip, np.array([np.nan, np.inf, -np.inf], np.float32)) == 0
    assert _argmax(hip, np.full(5000, np.float32(-3e38))) == 0


@pytest.mark.parametrize("f32", [False, True])
@pytest.mark.parametrize("k,n", [
    (1024, 3072), (2560, 100), (28672, 64),       # whole 256-value blocks, any count: the flat walk
    (4096, 1024), (4096, 4096), (4096, 12288),    # Qwen3-8B shapes: one pass / streamed
    (8192, 1000), (12288, 4096), (16384, 300),    # longer rows (x from LDS beyond two steps)
    (2560, 300), (5120, 257),                     # rows ending in a partial wave step
    (17408, 30), (25600, 20),                     # beyond four steps: the flat walk
    (1000, 64),                                   # K not a multiple of 256: one wave per row
])
def test_matvec_fp16(hip, orc, k, n, f32):
    rng = hip.synth.Rng(k + n)
    w = hip.synth.normal_f16(rng, n * k)
    x = hip.synth.normal_f16(rng, k)
    ref = vals(w).reshape(n, k) @ vals(x) / 1.0
    dw, dx = up(hip, w), up(hip, x)
    dy = hip.DeviceArray(n * (4 if f32 else 2))
    hip.device.matvec("fp16", dw, dx, dy, k, n, f32_out=f32)
    got = dy.download(np.float32, n).astype(np.float64) if f32 else vals(dy.download(np.uint16, n))
    bound = 1e-3 * math.sqrt(k / 4096) * np.sqrt((vals(w).reshape(n, k) ** 2) @ (vals(x) ** 2)) + 1e-5
    if not f32:
        bound = bound + 2.0 ** -11 * np.abs(ref)
    assert np.all(tol_ok(got, ref))
    assert np.all(np.abs(got - ref) <= bound)


def test_kernel_timer_brackets_the_calls_kernels(hip):
    """KernelTimer spans the first kernel's start to the last kernel's end of
    the calls made while armed, and disarms afterwards.  Each span is the
    least of five trials (a single kernel's time varies with the clocks)."""
    n, k = 12288, 4096
    w = hip.synth.quant_matrix("q4k", hip.synth.Rng(1), n, k)
    dw, dx, dy = up(hip, w), up(hip, hip.synth.normal_f16(hip.synth.Rng(2), k)), hip.DeviceArray(n * 2)
    hip.device.matvec("q4k", dw, dx, dy, k, n)

    def span(calls):
        best = float("inf")
        for _ in range(5):
            t = hip.device.KernelTimer()
            with t:
                for _ in range(calls):
                    hip.device.matvec("q4k", dw, dx, dy, k, n)
            hip.device.matvec("q4k", dw, dx, dy, k, n)   # not timed
            hip.synchronize()
            best = min(best, t.ms())
        return best

    t1, t3 = span(1), span(3)
    assert 0 < t1 < 5 and t3 > 2.0 * t1, (t1, t3)


def test_dispatch_timer_stamps_each_kernel(hip):
    """DispatchTimer gives each kernel of the armed calls its own duration:
    one for a GEMV, two for a split attention (split + merge, 16 chunks at
    L = 1024), each positive and their sum of the order of the call-span
    KernelTimer's (each stamped dispatch carries its own event overhead, so
    the sum is only bounded loosely); more kernels than event pairs raise,
    and the library is disarmed afterwards."""
    n, k = 4096, 4096
    w = hip.synth.quant_matrix("q4k", hip.synth.Rng(1), n, k)
    dw, dx, dy = up(hip, w), up(hip, hip.synth.normal_f16(hip.synth.Rng(2), k)), hip.DeviceArray(n * 2)
    t = hip.device.DispatchTimer()
    with t:
        hip.device.matvec("q4k", dw, dx, dy, k, n)
    hip.synchronize()
    assert t.count == 1 and 0 < t.ms() < 1.0

    heads, kv, hd, L = 16, 8, 128, 1024
    rng = hip.synth.Rng(3)
    q = up(hip, hip.synth.normal_f16(rng, heads * hd))
    kc, vc = up(hip, hip.synth.normal_f16(rng, L * kv * hd)), up(hip, hip.synth.normal_f16(rng, L * kv * hd))
    ws, out = hip.DeviceArray(heads * L * 4), hip.DeviceArray(heads * hd * 2)
    attn = lambda: hip.device.attention(q, kc, vc, ws, out, L - 1, L, heads, kv, hd)
    attn()
    best_sum, best_span = float("inf"), float("inf")
    for _ in range(5):
        # each timed call with the queue drained around it (a stamped
        # dispatch's events otherwise also count the launches queued behind)
        t, span = hip.device.DispatchTimer(), hip.device.KernelTimer()
        hip.synchronize()
        with t:
            attn()
        hip.synchronize()
        with span:
            attn()
        hip.synchronize()
        each = t.each_ms()
        assert t.count == 2 and all(0 < e < 1.0 for e in each), each
        best_sum, best_span = min(best_sum, sum(each)), min(best_span, span.ms())
    assert 0.25 * best_span <= best_sum <= 1.5 * best_span, (best_sum, best_span)

    with pytest.raises(RuntimeError, match="2 kernels launched, 1 event pairs"):
        with hip.device.DispatchTimer(1):
            attn()
    hip.synchronize()
    cnt = __import__("ctypes").c_int()
    assert hip.load().citlali_hip_dispatch_timing_count(__import__("ctypes").byref(cnt)) == 0 and cnt.value == 2
    attn()   # disarmed: launches unstamped
    hip.synchronize()


def test_argmax_signed_zero_and_block_edges(hip, orc):
    """-0.0 and +0.0 are equal for the host's `>`: the first one wins.  The
    device reduces ranges of about 1024 values per block: maxima placed at
    range edges and in the last partial range are found."""
    x = np.full(5000, -1.0, np.float32)
    x[7], x[9] = -0.0, 0.0
    assert _argmax(hip, x) == orc.argmax(x) == 7
    n = 151936
    for pos in (0, 1023, 1024, 2047, n - 1):
        y = np.zeros(n, np.float32)
        y[pos] = 1.0
        y[min(n - 1, pos + 5)] = 1.0   # a later equal value
        assert _argmax(hip, y) == orc.argmax(y) == pos


# ---- fused forward_token steps: the separate launches' results, bit for bit ----
@pytest.mark.parametrize("n", [1024, 4096])
def test_add_rms_norm_equals_add_then_norm(hip, n):
    rng = hip.synth.Rng(500 + n)
    x, d, w = (hip.synth.normal_f16(rng, n) for _ in range(3))
    dx1, dd, dw = up(hip, x), up(hip, d), up(hip, w)
    o1 = hip.DeviceArray(n * 2)
    hip.device.add_inplace(dx1, dd, n)
    hip.device.rms_norm(dx1, dw, o1, n, 1e-6)
    dx2, o2 = up(hip, x), hip.DeviceArray(n * 2)
    hip.device.add_rms_norm(dx2, dd, dw, o2, n, 1e-6)
    assert np.array_equal(dx1.download(np.uint16, n), dx2.download(np.uint16, n))
    assert np.array_equal(o1.download(np.uint16, n), o2.download(np.uint16, n))


@pytest.mark.parametrize("with_norm", [True, False])
@pytest.mark.parametrize("heads,kv,hd,pos", [(32, 8, 128, 700), (16, 8, 128, 0), (16, 4, 64, 37)])
def test_qk_norm_rope_store_equals_separate_launches(hip, heads, kv, hd, pos, with_norm):
    rng = hip.synth.Rng(heads * 1000 + pos)
    ctx = 1024
    q, k, v = hip.synth.normal_f16(rng, heads * hd), hip.synth.normal_f16(rng, kv * hd), hip.synth.normal_f16(rng, kv * hd)
    qw, kw = hip.synth.normal_f16(rng, hd), hip.synth.normal_f16(rng, hd)
    cache0 = hip.synth.normal_f16(rng, ctx * kv * hd)
    # separate launches (qwen_model.cpp:326-336)
    dq, dk, dv = up(hip, q), up(hip, k), up(hip, v)
    kc1, vc1 = up(hip, cache0), up(hip, cache0)
    if with_norm:
        hip.device.rms_norm_heads(dq, up(hip, qw), dq, heads, hd, 1e-6)
        hip.device.rms_norm_heads(dk, up(hip, kw), dk, kv, hd, 1e-6)
    hip.device.rope(dq, heads, hd, pos, 1e6)
    hip.device.rope(dk, kv, hd, pos, 1e6)
    hip.device.store_kv(dk, dv, kc1, vc1, pos, kv * hd)
    # fused
    fq = up(hip, q)
    kc2, vc2 = up(hip, cache0), up(hip, cache0)
    hip.device.qk_norm_rope_store(fq, up(hip, k), up(hip, v), up(hip, qw) if with_norm else None,
                                  up(hip, kw) if with_norm else None, heads, kv, hd, pos, 1e6, 1e-6, kc2, vc2)
    assert np.array_equal(dq.download(np.uint16, heads * hd), fq.download(np.uint16, heads * hd))
    assert np.array_equal(kc1.download(np.uint16), kc2.download(np.uint16))
    assert np.array_equal(vc1.download(np.uint16), vc2.download(np.uint16))


@pytest.mark.parametrize("kind,n,k", [("q4k", 12288, 4096), ("q4k", 3000, 8192), ("q6k", 2048, 4096),
                                      ("fp16", 12288, 4096), ("fp16", 3000, 8192), ("q4k", 3072, 1024),
                                      ("q6k", 700, 3072), ("fp16", 5000, 2048), ("q4k", 1000, 2560),
                                      ("q6k", 500, 5120), ("fp16", 700, 5120), ("q4k", 5, 4096), ("q6k", 1, 2048),
                                      ("q4k", 2049, 4096), ("q4k", 3, 1024), ("q4k", 3073, 1024),
                                      ("q6k", 7, 2048), ("fp16", 2051, 1024)])
def test_gate_up_swiglu_equals_two_gemvs_and_swiglu(hip, kind, n, k):
    """Also fewer rows than one workgroup's eight waves (waves without a row),
    a row count that leaves the last workgroup a short range, and rows of 4
    or 8 blocks (four / two rows per wave step) whose count leaves the last
    step part-filled."""
    rng = hip.synth.Rng(n + k)
    wg, wu = hip.synth.quant_matrix(kind, rng, n, k), hip.synth.quant_matrix(kind, rng, n, k)
    x = hip.synth.normal_f16(rng, k)
    dg, du, dx = up(hip, wg), up(hip, wu), up(hip, x)
    g, u, a1 = hip.DeviceArray(n * 2), hip.DeviceArray(n * 2), hip.DeviceArray(n * 2)
    hip.device.matvec(kind, dg, dx, g, k, n)
    hip.device.matvec(kind, du, dx, u, k, n)
    hip.device.swiglu(g, u, a1, n)
    a2 = hip.DeviceArray(n * 2)
    hip.device.matvec_gate_up_swiglu(kind, dg, du, dx, a2, k, n)
    assert np.array_equal(a1.download(np.uint16, n), a2.download(np.uint16, n))


def test_gate_up_swiglu_declines_other_lengths(hip):
    d = hip.DeviceArray(1 << 20)
    with pytest.raises(hip.CitlaliError, match="no fused kernel"):
        hip.device.matvec_gate_up_swiglu("q4k", d, d, d, d, 1536, 64)


@pytest.mark.parametrize("nbytes,offset", [(16 << 20, 0), ((100 << 20) + 12345, 4096), ((64 << 20) - 2, 6)])
def test_large_host_to_device_copies_are_exact(hip, nbytes, offset):
    """citlali_hip_memcpy_h2d from 16 MB up (the pinned double-buffered
    staging path): every byte arrives, across piece boundaries, at an offset
    into the destination, with the bytes around it untouched."""
    rng = np.random.default_rng(nbytes)
    src = rng.integers(0, 256, nbytes, dtype=np.uint8)
    dev = up(hip, np.full(offset + nbytes + 4096, 0xA5, np.uint8))
    dev.upload(src, offset)
    got = dev.download(np.uint8, offset + nbytes + 4096)
    assert np.array_equal(got[offset:offset + nbytes], src)
    assert (got[:offset] == 0xA5).all() and (got[offset + nbytes:] == 0xA5).all()
