"""GPU parity of the replayable decode-step entry points (no reference
counterpart; they read the token and position from device memory so one
forward_token step of qwen_model.cpp:239-465 can be captured in a HIP graph).
Each must equal its scalar form bit for bit at the values it reads; the
attention planned for a length's bucket must equal citlali_hip_attention at
every position of the bucket; a captured graph replayed several times, with
eager work and synchronisations in between, must match the eager result on
every replay."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
H = np.float16


def up(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def state_array(hip, token, position, step=0):
    return up(hip, np.array([token, position, step, 0], np.int32))


@pytest.mark.parametrize("token", [0, 5, 511])
def test_embed_q6k_at_equals_scalar(hip, token):
    vocab, hidden = 512, 1024
    rng = hip.synth.Rng(3)
    table = up(hip, hip.synth.quant_matrix("q6k", rng, vocab, hidden))
    a, b = hip.DeviceArray(hidden * 2), hip.DeviceArray(hidden * 2)
    hip.device.embed_q6k(table, token, a, hidden)
    hip.device.embed_q6k_at(table, state_array(hip, token, 0), vocab, b, hidden)
    assert np.array_equal(a.download(np.uint16, hidden), b.download(np.uint16, hidden))


@pytest.mark.parametrize("token", [-1, 512, 1 << 30])
def test_embed_at_out_of_range_token_gives_zeros(hip, token):
    vocab, hidden = 512, 1024
    rng = hip.synth.Rng(4)
    q6 = up(hip, hip.synth.quant_matrix("q6k", rng, vocab, hidden))
    f16 = up(hip, hip.synth.normal_f16(rng, vocab * hidden))
    for fn, table in ((hip.device.embed_q6k_at, q6), (hip.device.embed_at, f16)):
        out = up(hip, np.full(hidden, 0x3c00, np.uint16))
        fn(table, state_array(hip, token, 0), vocab, out, hidden)
        assert (out.download(np.uint16, hidden) == 0).all()


def test_embed_f16_at_equals_scalar(hip):
    vocab, hidden = 300, 768
    table = up(hip, hip.synth.normal_f16(hip.synth.Rng(5), vocab * hidden))
    a, b = hip.DeviceArray(hidden * 2), hip.DeviceArray(hidden * 2)
    hip.device.embed(table, 299, a, hidden)
    hip.device.embed_at(table, state_array(hip, 299, 0), vocab, b, hidden)
    assert np.array_equal(a.download(np.uint16, hidden), b.download(np.uint16, hidden))


def qk_inputs(hip, heads, kv_heads, hd, ctx, seed):
    rng = hip.synth.Rng(seed)
    q = hip.synth.normal_f16(rng, heads * hd)
    k = hip.synth.normal_f16(rng, kv_heads * hd)
    v = hip.synth.normal_f16(rng, kv_heads * hd)
    qn = hip.synth.normal_f16(rng, hd)
    kn = hip.synth.normal_f16(rng, hd)
    cache = hip.synth.normal_f16(rng, ctx * kv_heads * hd)
    return q, k, v, qn, kn, cache


@pytest.mark.parametrize("position", [0, 17, 299])
def test_qk_norm_rope_store_at_equals_scalar(hip, position):
    heads, kv_heads, hd, ctx = 16, 8, 128, 300
    q, k, v, qn, kn, cache = qk_inputs(hip, heads, kv_heads, hd, ctx, position + 1)
    outs = []
    for use_state in (False, True):
        dq, dk, dv, dqn, dkn = up(hip, q), up(hip, k), up(hip, v), up(hip, qn), up(hip, kn)
        kc, vc = up(hip, cache), up(hip, cache[::-1].copy())
        if use_state:
            st = state_array(hip, 0, position)   # the position is state[1]
            hip.device.qk_norm_rope_store_at(dq, dk, dv, dqn, dkn, heads, kv_heads, hd, st.at(4), ctx, 1e6, 1e-6,
                                             kc, vc)
        else:
            hip.device.qk_norm_rope_store(dq, dk, dv, dqn, dkn, heads, kv_heads, hd, position, 1e6, 1e-6, kc, vc)
        outs.append([a.download(np.uint16) for a in (dq, kc, vc)])
    for x, y in zip(*outs):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("position", [-1, 300, 1 << 20])
def test_qk_norm_rope_store_at_out_of_range_writes_no_cache(hip, position):
    heads, kv_heads, hd, ctx = 16, 8, 128, 300
    q, k, v, qn, kn, cache = qk_inputs(hip, heads, kv_heads, hd, ctx, 9)
    kc, vc = up(hip, cache), up(hip, cache)
    st = state_array(hip, 0, position)
    hip.device.qk_norm_rope_store_at(up(hip, q), up(hip, k), up(hip, v), up(hip, qn), up(hip, kn), heads, kv_heads,
                                     hd, st.at(4), ctx, 1e6, 1e-6, kc, vc)
    assert np.array_equal(kc.download(np.uint16), cache)
    assert np.array_equal(vc.download(np.uint16), cache)


def test_argmax_advance_updates_state_and_tokens(hip):
    n = 151936
    rng = np.random.default_rng(1)
    logits = rng.standard_normal(n).astype(np.float32)
    logits[12345] = 50.0
    logits[99999] = 50.0                      # tie: the first index wins
    dl = up(hip, logits)
    st = state_array(hip, 7, 40, 2)
    toks = up(hip, np.full(4, -5, np.int32))
    hip.device.argmax_advance(dl, n, st, toks, 4)
    assert list(st.download(np.int32, 4)) == [12345, 41, 3, 0]
    assert list(toks.download(np.int32, 4)) == [-5, -5, 12345, -5]
    idx = hip.DeviceArray(4)
    hip.device.argmax(dl, n, idx)
    assert idx.download(np.int32, 1)[0] == 12345
    # past the capacity: the state advances, the token array is left alone
    st2 = state_array(hip, 0, 0, 4)
    hip.device.argmax_advance(dl, n, st2, toks, 4)
    assert list(st2.download(np.int32, 4)) == [12345, 1, 5, 0]
    assert list(toks.download(np.int32, 4)) == [-5, -5, 12345, -5]


def test_plan_length_buckets(hip):
    pl = hip.device.attention_plan_length
    assert [pl(n, 4096) for n in (1, 255, 256, 257, 512, 513, 4096)] == [256, 256, 256, 512, 512, 1024, 4096]
    assert [pl(n, 600) for n in (1, 300, 512, 513, 600)] == [256, 512, 512, 600, 600]
    assert [pl(n, 100) for n in (1, 100)] == [100, 100]
    assert pl(0, 100) == 0 and pl(101, 100) == 0


@pytest.mark.parametrize("max_context", [1000, 8192])
def test_attention_at_device_position_equals_scalar_attention(hip, max_context):
    heads, kv_heads, hd = 32, 8, 128
    rng = hip.synth.Rng(max_context)
    kc = up(hip, hip.synth.normal_f16(rng, max_context * kv_heads * hd))
    vc = up(hip, hip.synth.normal_f16(rng, max_context * kv_heads * hd))
    q = up(hip, hip.synth.normal_f16(rng, heads * hd))
    # the partials of the longest plan (more than the reference's
    # heads x max_context floats when chunks are short)
    ws_bytes = max(heads * max_context * 4,
                   hip.device.attention_workspace_bytes(max_context, 1, heads, kv_heads, hd))
    scores = hip.DeviceArray(ws_bytes)
    for pos in (0, 100, 255, 256, 300, 511, 700, max_context - 1):
        if pos >= max_context:
            continue
        a, b = hip.DeviceArray(heads * hd * 2), hip.DeviceArray(heads * hd * 2)
        hip.device.attention(q, kc, vc, scores, a, pos, max_context, heads, kv_heads, hd)
        plan = hip.device.attention_plan_length(pos + 1, max_context)
        hip.device.attention_batched(q, kc, vc, 0, up(hip, np.array([pos], np.int32)), plan, 1, heads, kv_heads, hd,
                                     scores, ws_bytes, b)
        assert np.array_equal(a.download(np.uint16), b.download(np.uint16)), pos


def test_graph_replays_match_eager_every_time(hip):
    """A captured step (embed at the state's token, q/k norm + RoPE + KV store
    at its position, attention, argmax advance) replayed 4 times with eager
    work between; every replay equals the same launches run eagerly."""
    vocab, hidden, heads, kv_heads, hd, ctx = 512, 4096, 32, 8, 128, 600
    rng = hip.synth.Rng(21)
    table = up(hip, hip.synth.quant_matrix("q6k", rng, vocab, hidden))
    qn, kn = up(hip, hip.synth.normal_f16(rng, hd)), up(hip, hip.synth.normal_f16(rng, hd))
    cache0 = hip.synth.normal_f16(rng, ctx * kv_heads * hd)
    logits = up(hip, np.random.default_rng(2).standard_normal(vocab).astype(np.float32))

    k_in = up(hip, hip.synth.normal_f16(rng, kv_heads * hd))
    v_in = up(hip, hip.synth.normal_f16(rng, kv_heads * hd))

    def make_bufs():
        return dict(x=hip.DeviceArray(hidden * 2), out=hip.DeviceArray(heads * hd * 2),
                    kc=up(hip, cache0), vc=up(hip, cache0), ws=hip.DeviceArray(heads * ctx * 4),
                    state=state_array(hip, 3, 250), toks=up(hip, np.full(8, -1, np.int32)))

    def step(b):
        # the embedded row is the query (hidden == heads * head_dim)
        x = b["x"]
        hip.device.embed_q6k_at(table, b["state"], vocab, x, hidden)
        hip.device.qk_norm_rope_store_at(x, k_in, v_in, qn, kn, heads, kv_heads, hd, b["state"].at(4), ctx, 1e6, 1e-6,
                                         b["kc"], b["vc"])
        hip.device.attention_batched(x, b["kc"], b["vc"], 0, b["state"].at(4), 256, 1, heads, kv_heads, hd,
                                     b["ws"], heads * ctx * 4, b["out"])
        hip.device.argmax_advance(logits, vocab, b["state"], b["toks"], 8)

    eager = make_bufs()
    results = []
    for _ in range(4):
        step(eager)
        hip.synchronize()
        results.append([eager[k].download(np.uint16 if k != "state" and k != "toks" else np.int32)
                        for k in ("out", "kc", "state", "toks")])

    s = hip.device.Stream()
    hip.device.set_stream(s)
    try:
        g_bufs = make_bufs()
        hip.synchronize()
        graph = hip.device.Graph.capture(lambda: step(g_bufs))
        try:
            for r in range(4):
                graph.launch()
                hip.synchronize()
                got = [g_bufs[k].download(np.uint16 if k != "state" and k != "toks" else np.int32)
                       for k in ("out", "kc", "state", "toks")]
                for a, b in zip(got, results[r]):
                    assert np.array_equal(a, b), f"replay {r}"
                # eager work between replays on the same stream
                scratch = hip.DeviceArray(hidden * 2)
                hip.device.embed_q6k(table, r, scratch, hidden)
                hip.synchronize()
        finally:
            graph.close()
    finally:
        hip.device.set_stream(None)
        s.close()
