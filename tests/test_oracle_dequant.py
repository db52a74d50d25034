"""Pins the oracle's Q4_K / Q6_K dequantisation (weight_loader.cpp:28-38,
147-323; kernels.cu:134-186): golden vectors written by the compiled
reference, the compiled reference itself on fresh random blocks, and closed
forms that expose the index permutation and the scale/min packing."""
from __future__ import annotations

import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("kind", ["q4k", "q6k"])
@pytest.mark.parametrize("fixture", ["random", "realistic"])
def test_dequant_matches_reference_golden(orc, kind, fixture):
    g = np.load(os.path.join(GOLDEN, f"dequant_{kind}_{fixture}.npz"), allow_pickle=False)
    np.testing.assert_array_equal(orc.dequant_f16(kind, g["blocks"], g["fp16"].size), g["fp16"])


@pytest.mark.parametrize("kind,nbytes", [("q4k", 144), ("q6k", 210)])
@pytest.mark.parametrize("count", [256 * 2000, 256 * 3 + 17, 1])
def test_dequant_matches_compiled_reference(orc, ref, kind, nbytes, count):
    nb = (count + 255) // 256
    blocks = np.random.default_rng(count).integers(0, 256, nb * nbytes, dtype=np.uint8)
    np.testing.assert_array_equal(orc.dequant_f16(kind, blocks, count), ref.dequant(kind, blocks, count))


@pytest.mark.parametrize("kind,nbytes", [("q4k", 144), ("q6k", 210)])
def test_f16_routine_is_rounded_f32_routine(orc, kind, nbytes):
    blocks = np.random.default_rng(1).integers(0, 256, 500 * nbytes, dtype=np.uint8)
    f32 = orc.dequant_f32(kind, blocks, 500 * 256)
    np.testing.assert_array_equal(orc.dequant_f16(kind, blocks, 500 * 256), orc.f2h(f32))


def q4k_block(d=1.0, dmin=0.0, sc=None, mn=None, qs=None):
    """Builds one Q4_K block from explicit 6-bit codes (packing of
    weight_loader.cpp:28-38, written out independently here)."""
    sc = [0] * 8 if sc is None else sc
    mn = [0] * 8 if mn is None else mn
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[4:16] = s
    b[16:] = 0 if qs is None else qs
    return b


def test_q4k_scale_min_unpacking_closed_form(orc):
    sc = [1, 2, 3, 63, 17, 40, 5, 62]
    mn = [9, 0, 33, 7, 61, 2, 48, 1]
    blk = q4k_block(d=1.0, dmin=0.5, sc=sc, mn=mn, qs=np.full(128, 0xFF, np.uint8))
    v = orc.dequant_f32("q4k", blk, 256)
    for g in range(8):
        np.testing.assert_array_equal(v[32 * g:32 * (g + 1)], np.float32(15 * sc[g] - 0.5 * mn[g]))


def test_q4k_index_permutation_one_hot(orc):
    # a single non-zero nibble at qs byte i reveals which output it feeds
    for i in [0, 1, 31, 32, 63, 64, 100, 127]:
        for hi in (0, 1):
            qs = np.zeros(128, np.uint8)
            qs[i] = 0x10 if hi else 0x01
            v = orc.dequant_f32("q4k", q4k_block(1.0, 0.0, [1] * 8, [0] * 8, qs), 256)
            j, r = divmod(i, 32)
            expect = np.zeros(256, np.float32)
            expect[64 * j + 32 * hi + r] = 1.0
            np.testing.assert_array_equal(v, expect)


def test_q4k_zero_scales_give_zero(orc):
    blk = q4k_block(0.0, 0.0, [63] * 8, [63] * 8, np.full(128, 0xFF, np.uint8))
    assert not orc.dequant_f32("q4k", blk, 256).view(np.uint32).any()


def test_q6k_closed_forms(orc):
    blk = np.zeros(210, np.uint8)
    blk[192:208] = 1
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    # all-zero codes -> q = -32 everywhere
    np.testing.assert_array_equal(orc.dequant_f32("q6k", blk, 256), np.full(256, -32, np.float32))
    # one-hot over ql nibbles and qh bit pairs
    for h in (0, 1):
        for part in range(4):
            for i in (0, 15, 16, 31):
                b = blk.copy()
                b[64 * h + 32 * (part & 1) + i] = 0x0F if part < 2 else 0xF0
                b[128 + 32 * h + i] = 3 << (2 * part)
                v = orc.dequant_f32("q6k", b, 256)
                e = 128 * h + 32 * part + i
                assert v[e] == 63 - 32, (h, part, i)
                others = np.delete(v, e)
                assert np.all((others == -32) | (others == 15 - 32) | (others == 48 - 32))
    # signed scales: scale index 8h + i/16 + 2*part
    b = blk.copy()
    b[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    v = orc.dequant_f32("q6k", b, 256)
    for e in range(256):
        h, part, i = e // 128, (e % 128) // 32, e % 32
        assert v[e] == -32.0 * (8 * h + i // 16 + 2 * part - 8)


def test_embed_is_nearest_even_of_f32_dequant(orc, synth):
    """orc_embed_q6k = numpy's IEEE (nearest-even) cast of the fp32 dequant
    row (pinned above) -- the reference kernel's __float2half store."""
    hidden, vocab = 1024, 7
    table = synth.q6k_blocks(synth.Rng(9), vocab * hidden // 256)
    for tok in (0, 3, vocab - 1):
        row = table[tok * (hidden // 256) * 210:(tok + 1) * (hidden // 256) * 210]
        f32 = orc.dequant_f32("q6k", row, hidden)
        np.testing.assert_array_equal(orc.embed_q6k(table, tok, hidden), f32.astype(np.float16).view(np.uint16))
