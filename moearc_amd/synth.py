"""Seeded synthetic inputs for the attention path (vectorised SplitMix64).

Two generators over the same SplitMix64 stream (the reference tests' RNG,
crates/moearc-kernels/tests/common/mod.rs:11-37):

* ``unit(seed, n, skip)`` -- the reference tests' ``Rng::unit`` values, uniform in [-1, 1)
  evaluated in f32, as the ``skip``-th .. ``skip+n-1``-th draws of ``Rng::new(seed)``. Draw k of
  SplitMix64 is ``mix(seed + (k+1) * 0x9E3779B97F4A7C15)``, so the stream vectorises exactly.
* ``normal(seed, n)`` -- N(0, 1) values for the benchmark shapes: Box-Muller over pairs of draws,
  u1 = ((x >> 11) + 1) * 2^-53 in (0, 1], u2 = (y >> 11) * 2^-53, z = sqrt(-2 ln u1) cos(2 pi u2),
  computed in float64 and rounded once to float32.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, skip: int = 0) -> np.ndarray:
    """Draws skip .. skip+n-1 of SplitMix64 seeded with ``seed``."""
    k = np.arange(skip + 1, skip + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + k * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def unit(seed: int, n: int, skip: int = 0) -> np.ndarray:
    """``Rng::unit`` draws: (low32 as f32 / 2^32) * 2 - 1, all in f32."""
    lo = (splitmix64(seed, n, skip) & np.uint64(0xFFFFFFFF)).astype(np.float32)
    return (lo / np.float32(4294967296.0)) * np.float32(2.0) - np.float32(1.0)


def normal(seed: int, n: int, chunk: int = 1 << 22) -> np.ndarray:
    """n standard-normal float32 values (Box-Muller, one value per pair of draws)."""
    out = np.empty(n, np.float32)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        r = splitmix64(seed, 2 * m, 2 * s)
        x, y = r[0::2], r[1::2]
        u1 = ((x >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
        u2 = (y >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        out[s:s + m] = (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)
    return out


def f16_bits(x: np.ndarray) -> np.ndarray:
    """IEEE binary16 bits of x (round-to-nearest-even), the cache's storage format."""
    return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)


def random_block_table(seed: int, n_pages: int) -> np.ndarray:
    """A seeded permutation of 0..n_pages-1 (scattered pages, as a long-lived allocator hands out)."""
    keys = splitmix64(seed, n_pages)
    return np.argsort(keys, kind="stable").astype(np.uint32)
