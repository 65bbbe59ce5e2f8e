"""Deterministic synthetic inputs shared by the benchmark and the parity tests.

Tensors come from numpy's PCG64 generator seeded per (workload, tensor):
the same seed gives the same bytes on every host running the same numpy,
so a GPU run and its CPU check regenerate identical inputs from the seed
alone.  Workload seeds are ``0x7EE70000 + index`` with the index of the
workload in the benchmark table, plus a per-tensor stream number.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x7EE70000


def uniform(seed: int, shape, low: float = 0.0, high: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    u = rng.random(shape, dtype=np.float32)
    if low == 0.0 and high == 1.0:
        return u
    return (np.float32(low) + np.float32(high - low) * u).astype(np.float32)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    z = rng.standard_normal(shape, dtype=np.float32)
    if mean == 0.0 and std == 1.0:
        return z
    z *= np.float32(std)
    z += np.float32(mean)
    return z


def workload_seed(index: int, stream: int = 0) -> int:
    """Seed for tensor `stream` of workload `index` (distinct streams per tensor)."""
    return SEED_BASE + index + (stream << 20)
