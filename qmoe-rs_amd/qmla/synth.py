"""Seeded synthetic inputs for benchmarks (host side, numpy).

Same generator definition as the test fixtures: SplitMix64 output i of a
stream seeded with `seed` is mix(seed + (i + 1) * 0x9E3779B97F4A7C15);
uniform integers take the top 32 bits by multiply-shift.  Large device
tensors are filled on the GPU with qmla_fill_normal_f32 instead.
"""
from __future__ import annotations

import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)


def splitmix64_at(seed: int, idx: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.asarray(idx, np.uint64) + np.uint64(1)) * _GOLD
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform_int(n: int, seed: int, lo: int, hi: int) -> np.ndarray:
    """n integers uniform in [lo, hi] (inclusive)."""
    x = splitmix64_at(seed, np.arange(n, dtype=np.uint64)) >> np.uint64(32)
    rng = np.uint64(hi - lo + 1)
    with np.errstate(over="ignore"):
        return (lo + ((x * rng) >> np.uint64(32)).astype(np.int64)).astype(np.int32)


def v3_decode_lengths(batch: int = 64, seed: int = 4, lo: int = 1024, hi: int = 32768) -> np.ndarray:
    """Ragged context lengths of the 128-head decode workload: cached tokens
    U[lo, hi] plus the one new token."""
    return uniform_int(batch, seed, lo, hi) + 1
