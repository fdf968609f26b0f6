"""Seeded synthetic inputs for benchmarks and examples.

Matrices, images and layer parameters are drawn from numpy's PCG64 generator
with a fixed seed per tensor, so every run (and any CPU check of a run's
results) regenerates exactly the same data.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def randn(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    """float32 N(0, scale^2) samples."""
    return (rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def uniform(shape, seed: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """float32 U[lo, hi) samples."""
    return rng(seed).uniform(lo, hi, size=shape).astype(np.float32)
