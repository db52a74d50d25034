"""GPU parity of citlali_hip_matvec_group: attn_q, attn_k and attn_v of one
layer (qwen_model.cpp:315-321, each a LinearBackend::forward of
linear_backend.cpp:17-61) in one launch.  Every output must equal the
separate matvec_q4k / matvec_q6k launch bit for bit (same lane mapping and
summation order), and one case is also held to the north-star bar against
the oracle's fp32 restatement."""
import numpy as np
import pytest

from conftest import tol_ok

pytestmark = pytest.mark.gpu
H = np.float16


def up(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def run_group(hip, kinds, rows, k, seed):
    rng = hip.synth.Rng(seed)
    ws = [hip.synth.quant_matrix(kd, rng, n, k) for kd, n in zip(kinds, rows)]
    x = hip.synth.normal_f16(rng, k)
    dws, dx = [up(hip, w) for w in ws], up(hip, x)
    sep = [hip.DeviceArray(n * 2) for n in rows]
    for kd, dw, y, n in zip(kinds, dws, sep, rows):
        hip.device.matvec(kd, dw, dx, y, k, n)
    grp = [hip.DeviceArray(n * 2) for n in rows]
    hip.device.matvec_group(kinds, dws, dx, grp, rows, k)
    got = [g.download(np.uint16, n) for g, n in zip(grp, rows)]
    ref = [s.download(np.uint16, n) for s, n in zip(sep, rows)]
    return ws, x, got, ref


CASES = [
    # Qwen3-8B attn_q / attn_k Q4_K, attn_v Q6_K
    (("q4k", "q4k", "q6k"), (4096, 1024, 1024), 4096),
    # one type only, three matrices (one row set)
    (("q4k", "q4k", "q4k"), (2048, 512, 512), 4096),
    (("q6k", "q6k", "q6k"), (1024, 256, 256), 8192),
    # Q6_K first, ragged row counts, every streamed length
    (("q6k", "q4k", "q4k"), (1000, 7, 3), 4096),
    (("q4k", "q6k", "q4k"), (513, 1, 130), 8192),
    (("q4k", "q6k", "q6k"), (96, 64, 33), 12288),
    (("q6k", "q4k", "q6k"), (200, 100, 5), 16384),
    (("q6k", "q6k"), (300, 2), 16384),
    # more rows than one pass covers: the streaming split of the workgroups
    (("q4k", "q4k", "q6k"), (8192, 1024, 1024), 4096),
    (("q6k", "q6k", "q4k"), (4000, 4000, 4000), 4096),
    # fewer than three matrices
    (("q4k",), (4096,), 4096),
    (("q6k", "q4k"), (1024, 4096), 4096),
    (("q4k", "q6k"), (1, 1), 4096),
    # fp16 weights (DequantizeToFp16): the plain launch is matvec_fp16
    (("fp16", "fp16", "fp16"), (4096, 1024, 1024), 4096),
    (("fp16", "fp16", "fp16"), (8192, 1024, 1024), 4096),
    (("fp16", "fp16"), (513, 7), 8192),
    (("fp16", "fp16", "fp16"), (300, 100, 3), 12288),
    (("fp16",), (200,), 16384),
    # rows shorter than one wave step (Qwen3-0.6B: hidden 1024, attn_o 2048,
    # ffn_down 3072): one pass of one / two rows per wave, streamed beyond
    (("q4k", "q4k", "q6k"), (2048, 1024, 1024), 1024),
    (("q6k", "q4k"), (700, 300), 2048),
    (("q4k", "q6k", "q4k"), (5000, 33, 1), 3072),
    (("q6k", "q6k", "q6k"), (1024, 1024, 3000), 1024),
    (("fp16", "fp16", "fp16"), (2048, 1024, 1024), 1024),
    (("fp16",), (6000,), 3072),
    # rows of 4 / 8 blocks pack four / two rows per wave step: units that
    # straddle two matrices and a part-filled last unit
    (("q4k", "q4k", "q6k"), (2047, 1025, 1023), 1024),
    (("q6k", "q4k"), (701, 301), 2048),
    (("fp16", "fp16", "fp16"), (1023, 1, 2), 1024),
    (("q4k", "q4k", "q4k"), (9001, 4093, 3), 1024),
    # the other Qwen3 sizes (4B hidden 2560, 14B / 32B hidden 5120, 1.7B /
    # 4B FFN 6144 / 9728): partial last wave step
    (("q4k", "q4k", "q6k"), (4096, 1024, 1024), 2560),
    (("q4k", "q4k", "q6k"), (5120, 1024, 1024), 5120),
    (("q6k", "q4k"), (100, 200), 6144),
    (("q4k",), (300,), 9728),
    (("fp16", "fp16", "fp16"), (512, 128, 128), 5120),
]


@pytest.mark.parametrize("kinds,rows,k", CASES)
def test_group_equals_separate_launches(hip, kinds, rows, k):
    _, _, got, ref = run_group(hip, kinds, rows, k, seed=sum(rows) + k)
    for g, r in zip(got, ref):
        assert np.array_equal(g, r)


def test_group_qwen3_8b_against_oracle(hip, orc):
    kinds, rows, k = ("q4k", "q4k", "q6k"), (4096, 1024, 1024), 4096
    ws, x, got, _ = run_group(hip, kinds, rows, k, seed=77)
    for kd, w, g, n in zip(kinds, ws, got, rows):
        ref = orc.matvec(kd, w, x, k, n)
        assert tol_ok(g.view(H).astype(np.float64), ref).all()


@pytest.mark.parametrize("k", [1536, 20480])
def test_group_declines_other_lengths_without_writing(hip, k):
    n = 64
    rng = hip.synth.Rng(5)
    w = up(hip, hip.synth.quant_matrix("q4k", rng, n, k))
    x = up(hip, hip.synth.normal_f16(rng, k))
    y = up(hip, np.full(n, 0x3c00, np.uint16))
    with pytest.raises(hip.CitlaliError, match="no grouped kernel"):
        hip.device.matvec_group(["q4k"], [w], x, [y], [n], k)
    assert (y.download(np.uint16, n) == 0x3c00).all()


def test_group_declines_fp16_mixed_with_quantized(hip):
    n, k = 64, 4096
    rng = hip.synth.Rng(6)
    wq = up(hip, hip.synth.quant_matrix("q4k", rng, n, k))
    wf = up(hip, hip.synth.quant_matrix("fp16", rng, n, k))
    x = up(hip, hip.synth.normal_f16(rng, k))
    y = [up(hip, np.full(n, 0x3c00, np.uint16)) for _ in range(2)]
    with pytest.raises(hip.CitlaliError, match="F16 and quantized"):
        hip.device.matvec_group(["q4k", "fp16"], [wq, wf], x, y, [n, n], k)
    assert all((t.download(np.uint16, n) == 0x3c00).all() for t in y)


def test_group_rejects_bad_arguments(hip):
    d = hip.DeviceArray(1 << 20)
    with pytest.raises(hip.CitlaliError, match="count"):
        hip.device.matvec_group([], [], d, [], [], 4096)
    with pytest.raises(hip.CitlaliError, match="count"):
        hip.device.matvec_group(["q4k"] * 4, [d] * 4, d, [d] * 4, [1] * 4, 4096)
    with pytest.raises(hip.CitlaliError, match="multiple of the 256"):
        hip.device.matvec_group(["q4k"], [d], d, [d], [8], 4000)
    with pytest.raises(hip.CitlaliError, match="must be positive"):
        hip.device.matvec_group(["q4k", "q6k"], [d, d], d, [d, d], [8, 0], 4096)
