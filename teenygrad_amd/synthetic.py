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


def resnet50_convs():
    """The 53 convolutions of ResNet-50 (torchvision v1.5: stride on the 3x3 of
    a bottleneck) at 224x224 input, as (name, C_IN, C_OUT, H_IN, K, stride,
    pad, relu).  BN is folded into a bias; ReLU follows the stem, c1 and c2,
    while c3 and the downsample conv end with the residual add (not a conv),
    so they carry no fused activation."""
    layers = [("stem", 3, 64, 224, 7, 2, 3, True)]
    stages = [(64, 256, 3, 56), (128, 512, 4, 56), (256, 1024, 6, 28), (512, 2048, 3, 14)]
    cin = 64
    for si, (width, out, blocks, hin) in enumerate(stages):
        s = 1 if si == 0 else 2
        for bi in range(blocks):
            h = hin if bi == 0 else hin // s
            stride = s if bi == 0 else 1
            layers.append((f"l{si + 1}b{bi}c1", cin, width, h, 1, 1, 0, True))
            layers.append((f"l{si + 1}b{bi}c2", width, width, h, 3, stride, 1, True))
            layers.append((f"l{si + 1}b{bi}c3", width, out, h // stride, 1, 1, 0, False))
            if bi == 0:
                layers.append((f"l{si + 1}b{bi}ds", cin, out, h, 1, stride, 0, False))
            cin = out
    return layers
