"""Deterministic synthetic inputs shared by the benchmark and the parity tests.

Counter-based: element i of stream ``seed`` is a pure function of (seed, i)
(SplitMix64 finaliser over seed * 2^32 + i, Box-Muller for normals), so the
GPU run and the CPU check regenerate identical bytes from the seed alone and
any slice can be produced without the rest.  Workload seeds are
``0x7EE70000 + index`` with the index of the workload in the benchmark
table.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x7EE70000
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = z + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _u01(seed: int, start: int, n: int) -> np.ndarray:
    """Uniform doubles in (0, 1) for counters [start, start + n)."""
    ctr = np.arange(start, start + n, dtype=np.uint64) + np.uint64((seed & 0xFFFFFFFF) << 32)
    bits = _mix(ctr) >> np.uint64(11)
    return (bits.astype(np.float64) + 0.5) * (1.0 / (1 << 53))


def uniform(seed: int, shape, low: float = 0.0, high: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        m = min(_CHUNK, n - s)
        out[s:s + m] = (low + (high - low) * _u01(seed, s, m)).astype(np.float32)
    return out.reshape(shape)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        m = min(_CHUNK, n - s)
        # element i uses counters 2i and 2i+1 (Box-Muller, cosine branch)
        u = _u01(seed, 2 * s, 2 * m)
        u1, u2 = u[0::2], u[1::2]
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        out[s:s + m] = (mean + std * z).astype(np.float32)
    return out.reshape(shape)


def workload_seed(index: int, stream: int = 0) -> int:
    """Seed for tensor `stream` of workload `index` (distinct streams per tensor)."""
    return (SEED_BASE + index + (stream << 20)) & 0xFFFFFFFF
