"""GPU parity of citlali_hip_qk_norm_rope_store_attention: the step's q/k
head RMSNorm + RoPE, the KV store and decode attention in one launch (no
reference counterpart; qwen_model.cpp:315-338 makes them separate launches).
It must equal citlali_hip_qk_norm_rope_store followed by
citlali_hip_attention (scalar position), or the _at form followed by
citlali_hip_attention_batched (device position, planned for the bucket), bit
for bit: the output and both caches.  Cache rows at and beyond the position
hold NaN patterns, so a row read before it is written would show."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NAN16 = 0x7E00


def up(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def make(hip, heads, kv_heads, ctx, pos, seed, norms=True):
    hd = 128
    rng = hip.synth.Rng(seed)
    q = hip.synth.normal_f16(rng, heads * hd)
    k = hip.synth.normal_f16(rng, kv_heads * hd)
    v = hip.synth.normal_f16(rng, kv_heads * hd)
    qn = hip.synth.normal_f16(rng, hd) if norms else None
    kn = hip.synth.normal_f16(rng, hd) if norms else None
    kc = hip.synth.normal_f16(rng, ctx * kv_heads * hd).reshape(ctx, -1)
    vc = hip.synth.normal_f16(rng, ctx * kv_heads * hd).reshape(ctx, -1)
    kc[pos:] = NAN16
    vc[pos:] = NAN16
    return q, k, v, qn, kn, kc.reshape(-1), vc.reshape(-1)


def run_pair(hip, heads, kv_heads, ctx, pos, seed, device_position, norms=True):
    hd, theta, eps = 128, 1e6, 1e-6
    q, k, v, qn, kn, kc, vc = make(hip, heads, kv_heads, ctx, pos, seed, norms)
    dqn = up(hip, qn) if norms else None
    dkn = up(hip, kn) if norms else None
    ws_bytes = max(heads * ctx * 4, hip.device.attention_workspace_bytes(ctx, 1, heads, kv_heads, hd))
    plan = hip.device.attention_plan_length(pos + 1, ctx)
    outs = []
    for fused in (False, True):
        dq, dk, dv = up(hip, q), up(hip, k), up(hip, v)
        dkc, dvc = up(hip, kc), up(hip, vc)
        ws, out = hip.DeviceArray(ws_bytes), hip.DeviceArray(heads * hd * 2)
        st = up(hip, np.array([pos], np.int32))
        if fused:
            hip.device.qk_norm_rope_store_attention(dq, dk, dv, dqn, dkn, heads, kv_heads, hd,
                                                    st if device_position else pos, plan, ctx, theta, eps, dkc, dvc,
                                                    ws, ws_bytes, out)
            assert np.array_equal(dq.download(np.uint16), q)   # q is only read
        elif device_position:
            hip.device.qk_norm_rope_store_at(dq, dk, dv, dqn, dkn, heads, kv_heads, hd, st, ctx, theta, eps, dkc,
                                             dvc)
            hip.device.attention_batched(dq, dkc, dvc, 0, st, plan, 1, heads, kv_heads, hd, ws, ws_bytes, out)
        else:
            hip.device.qk_norm_rope_store(dq, dk, dv, dqn, dkn, heads, kv_heads, hd, pos, theta, eps, dkc, dvc)
            hip.device.attention(dq, dkc, dvc, ws, out, pos, ctx, heads, kv_heads, hd)
        outs.append([out.download(np.uint16), dkc.download(np.uint16), dvc.download(np.uint16)])
    return outs


@pytest.mark.parametrize("device_position", [False, True])
@pytest.mark.parametrize("heads,kv_heads", [(32, 8), (16, 8), (64, 8), (24, 8), (40, 8)])
def test_fused_equals_separate_launches(hip, heads, kv_heads, device_position):
    ctx = 1200
    for pos in (0, 1, 15, 16, 63, 64, 200, 255, 256, 300, 511, 512, 700, 1023, ctx - 1):
        ref, got = run_pair(hip, heads, kv_heads, ctx, pos, heads * 1000 + pos, device_position)
        for name, a, b in zip(("out", "k_cache", "v_cache"), ref, got):
            assert np.array_equal(a, b), (name, pos)
        assert not np.isnan(ref[0].view(np.float16)).any(), pos


@pytest.mark.parametrize("device_position", [False, True])
def test_fused_without_norm_weights(hip, device_position):
    for pos in (0, 37, 511, 4095):
        ref, got = run_pair(hip, 32, 8, 4096, pos, 7 + pos, device_position, norms=False)
        for name, a, b in zip(("out", "k_cache", "v_cache"), ref, got):
            assert np.array_equal(a, b), (name, pos)


@pytest.mark.parametrize("device_position", [False, True])
def test_fused_long_context(hip, device_position):
    """L = 8192 (32 chunks of 256, the merge kernel) and 8000 (a partial
    last chunk)."""
    for pos in (8191, 7999):
        ref, got = run_pair(hip, 32, 8, 8192, pos, 99 + pos, device_position)
        for name, a, b in zip(("out", "k_cache", "v_cache"), ref, got):
            assert np.array_equal(a, b), (name, pos)


@pytest.mark.parametrize("device_position", [False, True])
def test_fused_row_loads(hip, device_position):
    """Past 64K positions one sequence of 8 KV heads plans more than 512
    (KV head, chunk) units, and the split kernel switches to its row-load form
    (rows staged through LDS instead of direct loads), where the prologue
    substitutes the step's k/v row into the staged K/V rows.  ctx 70000: the
    plan is 69 chunks of 1024 (72 units of 8 KV heads would be 576)."""
    ctx = 70000
    for pos in (66000, 69999):
        plan = hip.device.attention_plan_length(pos + 1, ctx)
        chunk, splits = hip.device.attention_plan_info(plan, 1, 32, 8, 128)
        assert 8 * splits > 512, (plan, chunk, splits)
        ref, got = run_pair(hip, 32, 8, ctx, pos, 5 + pos, device_position)
        for name, a, b in zip(("out", "k_cache", "v_cache"), ref, got):
            assert np.array_equal(a, b), (name, pos)
        assert not np.isnan(ref[0].view(np.float16)).any(), pos


def test_fused_declines_other_shapes(hip):
    heads, kv_heads, hd, ctx = 8, 8, 128, 64
    z = hip.DeviceArray(heads * ctx * hd * 2)
    with pytest.raises(hip.CitlaliError, match="no fused kernel"):
        hip.device.qk_norm_rope_store_attention(z, z, z, None, None, heads, kv_heads, hd, 3, 0, ctx, 1e6, 1e-6, z, z,
                                                z, heads * ctx * 4, z)
    with pytest.raises(hip.CitlaliError, match="no fused kernel"):
        hip.device.qk_norm_rope_store_attention(z, z, z, None, None, 16, 8, 64, 3, 0, ctx, 1e6, 1e-6, z, z, z,
                                                heads * ctx * 4, z)


def test_fused_position_outside_the_plan_writes_nothing(hip):
    """A device position of -1 (or at the bucket's bound) leaves the caches
    alone, as the separate _at launches do for a position outside the
    cache."""
    heads, kv_heads, ctx = 32, 8, 600
    q, k, v, qn, kn, kc, vc = make(hip, heads, kv_heads, ctx, ctx, 3)
    dkc, dvc = up(hip, kc), up(hip, vc)
    ws_bytes = max(heads * ctx * 4, hip.device.attention_workspace_bytes(ctx, 1, heads, kv_heads, 128))
    ws, out = hip.DeviceArray(ws_bytes), hip.DeviceArray(heads * 128 * 2)
    for p in (-1, 256):
        st = up(hip, np.array([p], np.int32))
        hip.device.qk_norm_rope_store_attention(up(hip, q), up(hip, k), up(hip, v), up(hip, qn), up(hip, kn), heads,
                                                kv_heads, 128, st, 256, ctx, 1e6, 1e-6, dkc, dvc, ws, ws_bytes, out)
        assert np.array_equal(dkc.download(np.uint16), kc) and np.array_equal(dvc.download(np.uint16), vc), p
