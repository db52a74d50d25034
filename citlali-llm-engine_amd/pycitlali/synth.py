"""Seeded synthetic inputs for the decode hot path (shared by bench and tests).

A counter-based splitmix64 stream gives the same values on any machine and is
fully vectorised.  Normals come from the stream's own Box-Muller transform;
fp16 values are produced once on the host with the reference's host rounding
rule and handed to both the GPU and the CPU checker as identical bits.

Random K-quant super-blocks follow the layouts of weight_loader.cpp:147-323:
Q4_K (144 B): bytes 4..143 uniform, d and dmin = fp16(U[d_lo, d_hi]);
Q6_K (210 B): bytes 0..207 uniform (int8 scales), d = fp16(U[d_lo, d_hi]).
"""
from __future__ import annotations

import numpy as np

from .dtype import float_to_half_bits

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

Q4K_BYTES = 144
Q6K_BYTES = 210
QK = 256


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


class Rng:
    """splitmix64 over a counter: draw i of seed s is mix(s + (i+1)*golden)."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        self.counter = 0

    def u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            idx = np.arange(self.counter + 1, self.counter + n + 1, dtype=np.uint64)
            self.counter += n
            return _mix(self.state + idx * _GOLDEN)

    def uniform(self, n: int) -> np.ndarray:
        """float64 in [0, 1)."""
        return (self.u64(n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)

    def normal(self, n: int) -> np.ndarray:
        raw = self.u64(2 * n)
        u1 = ((raw[0::2] >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)
        u2 = (raw[1::2] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)

    def bytes(self, n: int) -> np.ndarray:
        return self.u64((n + 7) // 8).view(np.uint8)[:n].copy()


def normal_f16(rng: Rng, n: int, scale: float = 1.0) -> np.ndarray:
    """fp16 bits of N(0, scale^2) samples."""
    return float_to_half_bits((rng.normal(n) * scale).astype(np.float32))


def _half_scales(rng: Rng, n: int, lo: float, hi: float) -> np.ndarray:
    u = rng.uniform(n)
    return float_to_half_bits((lo + (hi - lo) * u).astype(np.float32))


def q4k_blocks(rng: Rng, n_blocks: int, d_lo: float = 1e-3, d_hi: float = 1e-2,
               dmin_lo: float | None = None, dmin_hi: float | None = None) -> np.ndarray:
    """n_blocks random Q4_K super-blocks as a flat uint8 array."""
    b = rng.bytes(n_blocks * Q4K_BYTES).reshape(n_blocks, Q4K_BYTES)
    d = _half_scales(rng, n_blocks, d_lo, d_hi)
    dm = _half_scales(rng, n_blocks, d_lo if dmin_lo is None else dmin_lo, d_hi if dmin_hi is None else dmin_hi)
    b[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    b[:, 2:4] = dm.view(np.uint8).reshape(n_blocks, 2)
    return b.reshape(-1)


def q6k_blocks(rng: Rng, n_blocks: int, d_lo: float = 1e-3, d_hi: float = 1e-2) -> np.ndarray:
    """n_blocks random Q6_K super-blocks as a flat uint8 array."""
    b = rng.bytes(n_blocks * Q6K_BYTES).reshape(n_blocks, Q6K_BYTES)
    d = _half_scales(rng, n_blocks, d_lo, d_hi)
    b[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return b.reshape(-1)


def quant_matrix(kind: str, rng: Rng, rows: int, cols: int, **kw) -> np.ndarray:
    """Row-major [rows][cols/256] super-blocks of the given kind ("q4k"/"q6k"),
    or for "fp16" a [rows*cols] matrix of N(0, 1) fp16 bits."""
    if kind == "fp16":
        return normal_f16(rng, rows * cols)
    nb = rows * (cols // QK)
    return q4k_blocks(rng, nb, **kw) if kind == "q4k" else q6k_blocks(rng, nb, **kw)
