"""Seeded synthetic inputs for the Q8 matmul workloads.

Distributions (the measured configurations):
  activations  A ~ N(0, 1), drawn in float32 and rounded to fp16
  weights      q = discrete uniform integers in [-127, 127] (int8)
  scales       s = fp16(U[1e-3, 1e-2]), one per 32-element K block
PRNG: numpy's PCG64 via numpy.random.default_rng(seed); within one case the
draws happen in the order A, q, s (weights of several layers: q then s, layer
by layer).  No real checkpoints are available offline, so every input is
synthetic.
"""
from __future__ import annotations

import numpy as np


def activations(rng: np.random.Generator, m: int, k: int) -> np.ndarray:
    return rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)


def q8_weight(rng: np.random.Generator, n: int, k: int):
    qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sc = rng.uniform(1e-3, 1e-2, size=(n, k // 32)).astype(np.float16)
    return qs, sc


def gemm_case(seed: int, m: int, n: int, k: int):
    """(A f16 [M][K], qs int8 [N][K], scales f16 [N][K/32])"""
    rng = np.random.default_rng(seed)
    a = activations(rng, m, k)
    qs, sc = q8_weight(rng, n, k)
    return a, qs, sc


def gemv_case(seed: int, n: int, k: int):
    """(x f16 [K], qs, scales) for M = 1."""
    a, qs, sc = gemm_case(seed, 1, n, k)
    return a[0], qs, sc
