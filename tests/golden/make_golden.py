"""Writes the golden vectors under tests/golden/ from the reference's own host
routines, compiled from /root/reference into oracle/_ref by oracle/Makefile.

    make -C oracle && python tests/golden/make_golden.py

Fixtures (inputs and the reference's outputs only):
  dequant_{q4k,q6k}_random.npz     64 super-blocks of uniform random bytes
                                   (d/dmin include NaN, Inf, subnormals)
  dequant_{q4k,q6k}_realistic.npz  64 super-blocks with d, dmin in [1e-3, 1e-2]
                                   (the BASELINE input recipe)
  f2h.npz                          fp32 inputs around every rounding boundary,
                                   exact ties, subnormals, overflow, NaN/Inf,
                                   and random bit patterns -> float_to_half_bits
  h2f.npz                          all 65536 fp16 patterns -> half_bits_to_float
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "citlali-llm-engine_amd"))

from oracle_binding import RefLib  # noqa: E402
from pycitlali import synth  # noqa: E402


def f2h_inputs() -> np.ndarray:
    vals = []
    # every fp16 value, its midpoints to both neighbours, and one fp32 ulp either side
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    nxt = np.append(f[1:], np.float32(65520.0))
    mid = ((f.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    for m in (mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf))):
        vals.append(m[::7])
        vals.append(-m[3::11])
    vals.append(np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 65504.0, 65519.99, 65520.0, 1e9,
                          2 ** -24, 2 ** -25, 2 ** -25 * 1.0001, 2 ** -26, 1e-30, 1.0 + 2 ** -11,
                          1.0 + 3 * 2 ** -11, 3.0 + 9 * 2 ** -10], np.float32))
    rng = np.random.default_rng(1234)
    vals.append(rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32))
    return np.concatenate(vals).astype(np.float32)


def main() -> None:
    ref = RefLib.try_load()
    if ref is None:
        raise SystemExit("oracle/_ref/libcitlali_ref.so is not built (make -C oracle)")
    for kind, nbytes in (("q4k", 144), ("q6k", 210)):
        r = synth.Rng(0x5EED + nbytes)
        blocks = r.bytes(64 * nbytes)
        np.savez_compressed(os.path.join(HERE, f"dequant_{kind}_random.npz"), blocks=blocks,
                            fp16=ref.dequant(kind, blocks, 64 * 256))
        blocks = synth.q4k_blocks(r, 64) if kind == "q4k" else synth.q6k_blocks(r, 64)
        np.savez_compressed(os.path.join(HERE, f"dequant_{kind}_realistic.npz"), blocks=blocks,
                            fp16=ref.dequant(kind, blocks, 64 * 256))
    x = f2h_inputs()
    np.savez_compressed(os.path.join(HERE, "f2h.npz"), f32_bits=x.view(np.uint32), fp16=ref.f2h(x))
    h = np.arange(65536, dtype=np.uint16)
    np.savez_compressed(os.path.join(HERE, "h2f.npz"), f32_bits=ref.h2f(h).view(np.uint32))
    for n in sorted(os.listdir(HERE)):
        if n.endswith(".npz"):
            print(n, os.path.getsize(os.path.join(HERE, n)))


if __name__ == "__main__":
    main()
