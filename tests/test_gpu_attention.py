"""GPU parity of decode attention (kernels.cu:545-649) against the oracle,
through the C ABI.

Bar (north star): |gpu - ref| <= 2e-3 + 1e-2*|ref| against the double
precision oracle.  Closed forms: one position gives V[0]; q = 0 gives the
mean of V; query heads sharing a kv head with equal q give equal outputs;
the result does not depend on how the positions are split into chunks.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import tol_ok

pytestmark = pytest.mark.gpu


def _cache(hip, seed, L, kv_heads, hd, max_ctx=None, scale=1.0):
    rng = hip.synth.Rng(seed)
    max_ctx = max_ctx or L
    k = hip.synth.normal_f16(rng, max_ctx * kv_heads * hd, scale)
    v = hip.synth.normal_f16(rng, max_ctx * kv_heads * hd)
    return k, v


def _run(hip, q, k, v, position, max_ctx, heads, kv_heads, hd, scores=True):
    dq = hip.DeviceArray.from_numpy(q)
    dk = hip.DeviceArray.from_numpy(k)
    dv = hip.DeviceArray.from_numpy(v)
    ds = hip.DeviceArray(heads * max_ctx * 4) if scores else None
    do = hip.DeviceArray(heads * hd * 2)
    hip.device.attention(dq, dk, dv, ds, do, position, max_ctx, heads, kv_heads, hd)
    return do.download(np.uint16, heads * hd).view(np.float16).astype(np.float64)


CASES = [
    # (heads, kv_heads, head_dim, L, max_ctx)
    (16, 8, 128, 1024, 1024),    # cfg2: Qwen3-0.6B
    (32, 8, 128, 8192, 8192),    # cfg3: Qwen3-8B at L = 8192
    (32, 8, 128, 1, 64),
    (32, 8, 128, 17, 64),
    (32, 8, 128, 65, 2048),
    (32, 8, 128, 1000, 1024),
    (16, 8, 128, 3000, 4096),
    (40, 8, 128, 777, 1024),     # group 5 (Qwen3-14B shape)
    (64, 8, 128, 513, 600),      # group 8
    (8, 8, 128, 300, 300),       # group 1
    (16, 8, 64, 700, 700),       # head_dim 64
    (32, 4, 64, 129, 200),
]


@pytest.mark.parametrize("heads,kv_heads,hd,L,max_ctx", CASES)
def test_attention_matches_oracle(hip, orc, heads, kv_heads, hd, L, max_ctx):
    print(f"[attention] heads={heads} kv={kv_heads} hd={hd} L={L} max_ctx={max_ctx}", flush=True)
    k, v = _cache(hip, 100 + L + heads, L, kv_heads, hd, max_ctx)
    q = hip.synth.normal_f16(hip.synth.Rng(L * 7 + hd), heads * hd)
    got = _run(hip, q, k, v, L - 1, max_ctx, heads, kv_heads, hd)
    ref = orc.attention(q, k, v, L - 1, heads, kv_heads, hd)
    bad = ~tol_ok(got, ref)
    assert not bad.any(), f"{bad.sum()} values out of tolerance; max err {np.abs(got - ref).max()}"
    # within one fp16 rounding plus fp32 noise
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2 ** -10 + 1e-4)


# Plans of many chunks.  The merge kernel folds up to 64 chunks per pass at
# head_dim 128 and 128 at head_dim 64 (8 per thread), and each wave lane
# reads the maxima of chunks lane, lane + 64, ...: these run one to five
# fold passes and one to five maxima reads per lane.
# (heads, kv_heads, head_dim, L, chunks the plan must make)
MANY_SPLITS = [
    (32, 4, 128, 16384, 64),
    (16, 2, 128, 32768, 128),
    (8, 1, 128, 300000, 293),
    (16, 2, 64, 40000, 125),
    (16, 2, 64, 80000, 157),
]


@pytest.mark.parametrize("heads,kv_heads,hd,L,splits", MANY_SPLITS)
def test_attention_many_splits(hip, orc, heads, kv_heads, hd, L, splits):
    print(f"[attention many splits] heads={heads} kv={kv_heads} hd={hd} L={L}", flush=True)
    bound = hip.device.attention_plan_length(L, L)
    assert hip.device.attention_plan_info(bound, 1, heads, kv_heads, hd)[1] == splits
    k, v = _cache(hip, 300 + heads, L, kv_heads, hd)
    q = hip.synth.normal_f16(hip.synth.Rng(L + hd), heads * hd)
    got = _run(hip, q, k, v, L - 1, L, heads, kv_heads, hd)
    ref = orc.attention(q, k, v, L - 1, heads, kv_heads, hd)
    assert np.all(tol_ok(got, ref)), f"max err {np.abs(got - ref).max()}"
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2 ** -10 + 1e-4)


def test_config4_batched_at_its_lengths(hip, orc):
    """BASELINE config 4 at its workload: 16 sequences at 32/8/128 with KV
    lengths uniform in [4096, 32768] drawn as bench.py draws them
    (numpy default_rng(4)), one batched launch planned for 32768 positions
    (64 chunks per sequence: the merge's largest batch, 8 chunks per
    thread), every sequence against the oracle."""
    nseq, heads, kv, hd, max_len = 16, 32, 8, 128, 32768
    lens = np.random.default_rng(4).integers(4096, max_len + 1, nseq)
    print(f"[attention cfg4] lengths {lens.tolist()}", flush=True)
    assert hip.device.attention_plan_info(max_len, nseq, heads, kv, hd) == (512, 64)
    stride = max_len * kv * hd
    gen = np.random.default_rng(40)
    k = np.zeros(nseq * stride, np.uint16)
    v = np.zeros(nseq * stride, np.uint16)
    for s, L in enumerate(lens):   # positions past a sequence's length stay zero and are never read
        n = int(L) * kv * hd
        k[s * stride:s * stride + n] = gen.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16)
        v[s * stride:s * stride + n] = gen.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16)
    q = gen.standard_normal(nseq * heads * hd, dtype=np.float32).astype(np.float16).view(np.uint16)
    pos = (lens - 1).astype(np.int32)
    ws_bytes = hip.device.attention_workspace_bytes(max_len, nseq, heads, kv, hd)
    dws = hip.DeviceArray(ws_bytes)
    dq, dk, dv = (hip.DeviceArray.from_numpy(a) for a in (q, k, v))
    dpos = hip.DeviceArray.from_numpy(pos)
    do = hip.DeviceArray(nseq * heads * hd * 2)
    hip.device.attention_batched(dq, dk, dv, stride, dpos, max_len, nseq, heads, kv, hd, dws, ws_bytes, do)
    got = do.download(np.uint16).view(np.float16).astype(np.float64).reshape(nseq, heads * hd)
    for a in (dq, dk, dv, dpos, do, dws):
        a.close()
    for s in range(nseq):
        sl = slice(s * stride, (s + 1) * stride)
        ref = orc.attention(q[s * heads * hd:(s + 1) * heads * hd], k[sl], v[sl], int(pos[s]), heads, kv, hd)
        assert np.all(tol_ok(got[s], ref)), f"sequence {s} (L={lens[s]}): max err {np.abs(got[s] - ref).max()}"
        assert np.all(np.abs(got[s] - ref) <= np.abs(ref) * 2 ** -10 + 1e-4), f"sequence {s} (L={lens[s]})"


def test_attention_without_scores_buffer(hip, orc):
    heads, kv, hd, L = 32, 8, 128, 4096
    k, v = _cache(hip, 5, L, kv, hd)
    q = hip.synth.normal_f16(hip.synth.Rng(6), heads * hd)
    got = _run(hip, q, k, v, L - 1, L, heads, kv, hd, scores=False)
    assert np.all(tol_ok(got, orc.attention(q, k, v, L - 1, heads, kv, hd)))


@pytest.mark.parametrize("heads,kv_heads,L", [(32, 8, 8192), (16, 8, 1024), (32, 8, 32768)])
def test_full_size_value_scaling(hip, heads, kv_heads, L):
    """At the benchmark lengths (configs 3 and 2, and config 4's longest
    sequence): doubling every V value doubles the output bit for bit
    wherever it is a normal fp16 number (the softmax weights do not change;
    the products, sums, the normalisation and the rounding commute with a
    power-of-two factor).  Below 2^-14 the fp16 spacing is a fixed 2^-24, so
    there the doubled output is the rounding of twice the exact value, within
    one such step of twice the first output."""
    hd = 128
    k, v = _cache(hip, 31, L, kv_heads, hd)
    q = hip.synth.normal_f16(hip.synth.Rng(32), heads * hd)
    v2 = (v.view(np.float16) * np.float16(2)).view(np.uint16)
    a = _run(hip, q, k, v, L - 1, L, heads, kv_heads, hd)
    b = _run(hip, q, k, v2, L - 1, L, heads, kv_heads, hd)
    assert np.all(np.isfinite(a))
    normal = np.abs(a) >= 2.0 ** -14
    assert normal.mean() > 0.9
    np.testing.assert_array_equal(b[normal], 2 * a[normal])
    assert np.all(np.abs(b[~normal] - 2 * a[~normal]) <= 2.0 ** -24)


def test_single_position_returns_v0(hip):
    heads, kv, hd = 32, 8, 128
    k, v = _cache(hip, 9, 16, kv, hd)
    q = hip.synth.normal_f16(hip.synth.Rng(10), heads * hd)
    got = _run(hip, q, k, v, 0, 16, heads, kv, hd)
    v0 = v[: kv * hd].view(np.float16).astype(np.float64).reshape(kv, hd)
    np.testing.assert_array_equal(got.reshape(heads, hd), np.repeat(v0, heads // kv, axis=0))


def test_zero_query_gives_mean_of_values(hip):
    heads, kv, hd, L = 16, 8, 128, 2500
    k, v = _cache(hip, 12, L, kv, hd)
    q = np.zeros(heads * hd, np.uint16)
    got = _run(hip, q, k, v, L - 1, L, heads, kv, hd).reshape(heads, hd)
    mean = v.view(np.float16).astype(np.float64).reshape(L, kv, hd).mean(axis=0)
    ref = np.repeat(mean, heads // kv, axis=0)
    assert np.all(np.abs(got - ref) <= 2e-3 + 1e-2 * np.abs(ref))


def test_gqa_heads_with_equal_queries_agree(hip):
    heads, kv, hd, L = 32, 8, 128, 1500
    k, v = _cache(hip, 13, L, kv, hd)
    qh = hip.synth.normal_f16(hip.synth.Rng(14), kv * hd).reshape(kv, 1, hd)
    q = np.ascontiguousarray(np.repeat(qh, heads // kv, axis=1).reshape(-1))
    got = _run(hip, q, k, v, L - 1, L, heads, kv, hd).reshape(kv, heads // kv, hd)
    for g in range(1, heads // kv):
        np.testing.assert_array_equal(got[:, g], got[:, 0])


def test_batched_matches_single_sequence_calls(hip, orc):
    """16 sequences in one launch == 16 single-sequence launches (cfg4 shape,
    shortened so the oracle stays fast)."""
    nseq, heads, kv, hd, max_ctx = 16, 32, 8, 128, 3000
    rng = hip.synth.Rng(2024)
    lens = (rng.u64(nseq) % np.uint64(max_ctx)).astype(np.int64) + 1
    lens[0], lens[1] = 1, max_ctx
    stride = max_ctx * kv * hd
    k = hip.synth.normal_f16(rng, nseq * stride)
    v = hip.synth.normal_f16(rng, nseq * stride)
    q = hip.synth.normal_f16(rng, nseq * heads * hd)
    pos = (lens - 1).astype(np.int32)
    ws_bytes = hip.device.attention_workspace_bytes(max_ctx, nseq, heads, kv, hd)
    dws = hip.DeviceArray(max(ws_bytes, 16))
    dq, dk, dv = (hip.DeviceArray.from_numpy(a) for a in (q, k, v))
    dpos = hip.DeviceArray.from_numpy(pos)
    do = hip.DeviceArray(nseq * heads * hd * 2)
    hip.device.attention_batched(dq, dk, dv, stride, dpos, max_ctx, nseq, heads, kv, hd, dws, ws_bytes, do)
    got = do.download(np.uint16).view(np.float16).astype(np.float64).reshape(nseq, heads * hd)
    for s in range(nseq):
        sl = slice(s * stride, (s + 1) * stride)
        qs = q[s * heads * hd:(s + 1) * heads * hd]
        ref = orc.attention(qs, k[sl], v[sl], int(pos[s]), heads, kv, hd)
        assert np.all(tol_ok(got[s], ref)), f"sequence {s} (L={lens[s]})"
        single = _run(hip, qs, k[sl], v[sl], int(pos[s]), max_ctx, heads, kv, hd)
        assert np.all(np.abs(single - got[s]) <= np.abs(ref) * 2 ** -10 + 1e-4)


@pytest.mark.parametrize("heads,kv,nseq", [(16, 8, 16), (64, 8, 16), (32, 4, 32)])
def test_batched_row_loads_each_group(hip, orc, heads, kv, nseq):
    """Launches of more than 512 workgroups read K and V as whole rows
    through LDS (the planned load form for saturating launches); GQA groups
    2, 8 and 8-of-4 through that form against the oracle, lengths up to
    3000 with the extremes 1 and 3000."""
    hd, max_ctx = 128, 3000
    chunk, splits = hip.device.attention_plan_info(max_ctx, nseq, heads, kv, hd)
    assert nseq * kv * splits > 512, "the case must plan the row-load form"
    rng = hip.synth.Rng(77 + heads + nseq)
    lens = (rng.u64(nseq) % np.uint64(max_ctx)).astype(np.int64) + 1
    lens[0], lens[1] = 1, max_ctx
    stride = max_ctx * kv * hd
    k = hip.synth.normal_f16(rng, nseq * stride)
    v = hip.synth.normal_f16(rng, nseq * stride)
    q = hip.synth.normal_f16(rng, nseq * heads * hd)
    pos = (lens - 1).astype(np.int32)
    ws_bytes = hip.device.attention_workspace_bytes(max_ctx, nseq, heads, kv, hd)
    dws = hip.DeviceArray(max(ws_bytes, 16))
    dq, dk, dv = (hip.DeviceArray.from_numpy(a) for a in (q, k, v))
    dpos = hip.DeviceArray.from_numpy(pos)
    do = hip.DeviceArray(nseq * heads * hd * 2)
    hip.device.attention_batched(dq, dk, dv, stride, dpos, max_ctx, nseq, heads, kv, hd, dws, ws_bytes, do)
    got = do.download(np.uint16).view(np.float16).astype(np.float64).reshape(nseq, heads * hd)
    for a in (dq, dk, dv, dpos, do, dws):
        a.close()
    for s in range(nseq):
        sl = slice(s * stride, (s + 1) * stride)
        ref = orc.attention(q[s * heads * hd:(s + 1) * heads * hd], k[sl], v[sl], int(pos[s]), heads, kv, hd)
        assert np.all(tol_ok(got[s], ref)), f"sequence {s} (L={lens[s]}): max err {np.abs(got[s] - ref).max()}"


def test_batched_rejects_small_workspace(hip):
    heads, kv, hd, nseq, max_ctx = 32, 8, 128, 4, 4096
    need = hip.device.attention_workspace_bytes(max_ctx, nseq, heads, kv, hd)
    assert need > 0
    d = hip.DeviceArray(1 << 20)
    pos = hip.DeviceArray.from_numpy(np.full(nseq, max_ctx - 1, np.int32))
    with pytest.raises(hip.CitlaliError, match="workspace"):
        hip.device.attention_batched(d, d, d, 0, pos, max_ctx, nseq, heads, kv, hd, d, need - 16, d)


def test_batched_position_past_bound_is_cut_at_bound(hip):
    """A device position >= max_positions_bound attends over positions
    0..bound-1 (the caches end there), exactly like position = bound - 1."""
    nseq, heads, kv, hd, bound = 3, 32, 8, 128, 1000
    rng = hip.synth.Rng(77)
    stride = bound * kv * hd
    k = hip.synth.normal_f16(rng, nseq * stride)
    v = hip.synth.normal_f16(rng, nseq * stride)
    q = hip.synth.normal_f16(rng, nseq * heads * hd)
    ws_bytes = hip.device.attention_workspace_bytes(bound, nseq, heads, kv, hd)
    dws = hip.DeviceArray(max(ws_bytes, 16))
    dq, dk, dv = (hip.DeviceArray.from_numpy(a) for a in (q, k, v))
    outs = []
    for last in (bound - 1, bound + 500):
        dpos = hip.DeviceArray.from_numpy(np.array([10, last, 999], np.int32))
        do = hip.DeviceArray(nseq * heads * hd * 2)
        hip.device.attention_batched(dq, dk, dv, stride, dpos, bound, nseq, heads, kv, hd, dws, ws_bytes, do)
        outs.append(do.download(np.uint16))
    assert np.array_equal(outs[0], outs[1])
