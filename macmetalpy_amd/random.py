"""Seeded host-side random inputs (reference: src/macmetalpy/random.py:8-80).

Same module state and draws as the reference, so ``seed(s)`` followed by
``randn``/``rand``/``randint``/``uniform`` produces bit-identical inputs:
a NumPy ``default_rng(s)`` PCG64 generator; ``randn``/``rand`` draw float32
directly, ``uniform``/``normal`` draw float64 and cast to float32,
``randint`` draws int32.  Results are host-resident arrays.
"""
from __future__ import annotations

import numpy as np

from .ndarray import ndarray

_rng_gen = np.random.default_rng()


def _fnd(x):
    return ndarray._from_np_direct(np.asarray(x))


def seed(s=None):
    global _rng_gen
    _rng_gen = np.random.default_rng(s)


def get_generator():
    return _rng_gen


def rand(*shape):
    return _fnd(_rng_gen.random(shape or None, dtype=np.float32))


def randn(*shape):
    return _fnd(_rng_gen.standard_normal(shape or None, dtype=np.float32))


def random(size=None):
    return _fnd(_rng_gen.random(size, dtype=np.float32))


def standard_normal(size=None):
    return _fnd(_rng_gen.standard_normal(size, dtype=np.float32))


def randint(low, high=None, size=None, dtype=int):
    return _fnd(np.asarray(_rng_gen.integers(low, high, size=size, dtype=np.int32), dtype=np.int32))


def normal(loc=0.0, scale=1.0, size=None):
    return _fnd(_rng_gen.normal(loc, scale, size).astype(np.float32))


def uniform(low=0.0, high=1.0, size=None):
    return _fnd(_rng_gen.uniform(low, high, size).astype(np.float32))
