"""Synthetic benchmark workloads (seeded host inputs).

Five configurations of the hot path, each drawn from one NumPy
``default_rng(seed)`` generator in the order listed -- the same stream the
reference's ``cp.random.seed(seed)`` followed by ``randn`` / ``randint`` /
``uniform`` calls produces (src/macmetalpy/random.py:17-80):

C1 fused elementwise  y = sqrt(abs(x)) + exp(-x**2), x float32 N(0,1), 2^20
C2 binary 2^28        a + b, sin(a) on float32 N(0,1); int32 floor_divide /
                      mod with a ~ U[-2^30, 2^30), b ~ U[1, 1000] with a random
                      sign (p = 0.5)
C3 reductions / scan  sum, mean, argmax (axis=None, axis=1) of a (16384,
                      16384) float32 N(0,1); cumsum of 2^28 int32 U[-100, 100]
                      and float32 U[0, 1)
C4 matmul             float32 4096^2 @ 4096^2, float16 8192^2 @ 8192^2,
                      batched float32 (64,1024,1024) @ (64,1024,1024); entries
                      N(0,1)/sqrt(K)
C5 fusion chain       z = sum(tanh(x*r + 1.0) * exp(-abs(x)) - log1p(x*x),
                      axis=1), x (8192, 8192) N(0,1), r (1, 8192) U[0.5, 2)

``scale`` divides the element counts (tests use small scales; the benchmark
uses 1).
"""
from __future__ import annotations

import numpy as np

__all__ = ["c1_inputs", "c2_float_inputs", "c2_int_inputs", "c3_matrix", "c3_scan_inputs",
           "c4_inputs", "c5_inputs", "SEEDS"]

SEEDS = {"c1": 0, "c2": 2, "c3": 3, "c3_scan": 4, "c4": 1, "c5": 5}


def c1_inputs(n: int = 1 << 20):
    return np.random.default_rng(SEEDS["c1"]).standard_normal(n, dtype=np.float32)


def c2_float_inputs(n: int = 1 << 28):
    ab = np.random.default_rng(SEEDS["c2"]).standard_normal((2, n), dtype=np.float32)
    return ab[0], ab[1]


def c2_int_inputs(n: int = 1 << 28):
    g = np.random.default_rng(SEEDS["c2"])
    a = g.integers(-2 ** 30, 2 ** 30, n, dtype=np.int32)
    b = g.integers(1, 1000, n, endpoint=True, dtype=np.int32)
    sign = np.where(g.random(n) < 0.5, -1, 1).astype(np.int32)
    return a, b * sign


def c3_matrix(rows: int = 16384, cols: int = 16384):
    return np.random.default_rng(SEEDS["c3"]).standard_normal((rows, cols), dtype=np.float32)


def c3_scan_inputs(n: int = 1 << 28):
    g = np.random.default_rng(SEEDS["c3_scan"])
    ci = g.integers(-100, 100, n, endpoint=True, dtype=np.int32)
    cf = g.random(n, dtype=np.float32)
    return ci, cf


def c4_inputs(kind: str, n: int | None = None):
    """kind: 'f32' (4096^2), 'f16' (8192^2), 'batched' (64, 1024, 1024)."""
    g = np.random.default_rng(SEEDS["c4"])
    if kind == "f32":
        n = n or 4096
        a = g.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))
        b = g.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))
        return a, b
    if kind == "f16":
        n = n or 8192
        a = (g.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))).astype(np.float16)
        b = (g.standard_normal((n, n), dtype=np.float32) / np.float32(np.sqrt(n))).astype(np.float16)
        return a, b
    if kind == "batched":
        n = n or 1024
        a = g.standard_normal((64, n, n), dtype=np.float32) / np.float32(np.sqrt(n))
        b = g.standard_normal((64, n, n), dtype=np.float32) / np.float32(np.sqrt(n))
        return a, b
    raise ValueError(kind)


def c5_inputs(rows: int = 8192, cols: int = 8192):
    g = np.random.default_rng(SEEDS["c5"])
    x = g.standard_normal((rows, cols), dtype=np.float32)
    r = g.uniform(0.5, 2.0, (1, cols)).astype(np.float32)
    return x, r
