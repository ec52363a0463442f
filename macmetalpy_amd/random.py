"""Seeded random inputs (reference: src/macmetalpy/random.py).

Same module state and draws as the reference, so ``seed(s)`` followed by
any of its functions produces bit-identical arrays: one NumPy
``default_rng(s)`` PCG64 generator for every draw; ``randn`` / ``rand`` /
``random`` / ``standard_normal`` / ``standard_exponential`` draw float32
directly, the other continuous distributions draw float64 and cast to
float32, the discrete ones return int32.  Results are host-resident arrays
(uploaded on first device use), as the reference's.

Permutations move data on the device: ``shuffle`` / ``permutation`` /
``permuted`` / ``choice`` draw their index permutation or sample indices
from the same generator (NumPy's Fisher-Yates consumes the same numbers
for an index range as for the data) and gather with the device kernels.
``Generator`` / ``default_rng`` mirror the reference's: methods act on the
module generator, and a seed reseeds it.
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


def _shape(shape):
    return shape or None


def rand(*shape):
    return _fnd(_rng_gen.random(_shape(shape), dtype=np.float32))


def randn(*shape):
    return _fnd(_rng_gen.standard_normal(_shape(shape), dtype=np.float32))


def random(size=None):
    return _fnd(_rng_gen.random(size, dtype=np.float32))


def standard_normal(size=None):
    return _fnd(_rng_gen.standard_normal(size, dtype=np.float32))


def standard_exponential(size=None):
    return _fnd(_rng_gen.standard_exponential(size, dtype=np.float32))


def randint(low, high=None, size=None, dtype=int):
    return _fnd(np.asarray(_rng_gen.integers(low, high, size=size, dtype=np.int32), dtype=np.int32))


def random_integers(low, high=None, size=None):
    if high is None:
        low, high = 1, low
    return randint(low, high + 1, size=size)


def random_sample(size=None):
    return random(size=size)


ranf = random
sample = random


# Continuous distributions: float64 draws of the generator's method with
# the same name, cast to float32.  Discrete ones: int32.
_FLOAT32_DRAWS = ("normal", "uniform", "beta", "exponential", "gamma", "standard_cauchy",
                  "standard_gamma", "standard_t", "chisquare", "laplace", "logistic", "lognormal",
                  "gumbel", "rayleigh", "triangular", "weibull", "vonmises", "wald", "pareto",
                  "dirichlet", "f", "power", "noncentral_chisquare", "noncentral_f")
_INT32_DRAWS = ("binomial", "poisson", "geometric", "zipf", "logseries", "multinomial",
                "hypergeometric", "negative_binomial")


def _float_draw(name):
    def draw(*args, **kwargs):
        return _fnd(getattr(_rng_gen, name)(*args, **kwargs).astype(np.float32))
    draw.__name__ = name
    draw.__doc__ = f"float32 cast of numpy.random.Generator.{name} on the module generator."
    return draw


def _int_draw(name):
    def draw(*args, **kwargs):
        return _fnd(np.asarray(getattr(_rng_gen, name)(*args, **kwargs), dtype=np.int32))
    draw.__name__ = name
    draw.__doc__ = f"int32 numpy.random.Generator.{name} on the module generator."
    return draw


for _n in _FLOAT32_DRAWS:
    globals()[_n] = _float_draw(_n)
for _n in _INT32_DRAWS:
    globals()[_n] = _int_draw(_n)
del _n


def _host_arg(x):
    return x.get() if isinstance(x, ndarray) else np.asarray(x)


def multivariate_normal(mean, cov, size=None):
    return _fnd(_rng_gen.multivariate_normal(_host_arg(mean), _host_arg(cov), size)
                .astype(np.float32))


# ------------------------------------------------------------ permutations
def _dev(x):
    from .creation import asarray
    return asarray(x)


def shuffle(a):
    """Shuffles the first axis in place: the generator's permutation of its
    length, applied by a device gather."""
    from .indexing import take
    if not isinstance(a, ndarray):
        raise TypeError("shuffle needs a macmetalpy array to modify in place")
    if a.ndim == 0:
        raise TypeError("shuffle of a 0-d array")
    perm = _rng_gen.permutation(a.shape[0])
    a[...] = take(a, _dev(perm.astype(np.int64)), axis=0)


def permutation(x):
    """A permuted range (int32) for an integer, otherwise the first axis of
    a copy permuted; as in the reference an array comes back as float32."""
    from .indexing import take
    if isinstance(x, (int, np.integer)):
        return _fnd(np.asarray(_rng_gen.permutation(int(x)), dtype=np.int32))
    a = _dev(x)
    if a.ndim == 0:
        raise np.exceptions.AxisError("x must be an integer or at least 1-dimensional")
    perm = _rng_gen.permutation(a.shape[0])
    return take(a, _dev(perm.astype(np.int64)), axis=0).astype(np.float32)


def permuted(x, axis=None, out=None):
    """Each 1-D slice along ``axis`` (the flattened array for None) shuffled
    independently, slices in C order as NumPy walks them."""
    from .indexing import take, take_along_axis
    from .manipulation import moveaxis
    a = _dev(x)
    if axis is None:
        perm = _rng_gen.permutation(a.size)
        r = take(a.ravel(), _dev(perm.astype(np.int64))).reshape(tuple(a.shape))
    else:
        from .ndarray import _normalize_axis
        ax = _normalize_axis(axis, a.ndim)
        m = moveaxis(a, ax, -1)
        outer = tuple(m.shape[:-1])
        n = m.shape[-1]
        idx = np.empty(outer + (n,), dtype=np.int64)
        for o in np.ndindex(*outer):
            idx[o] = _rng_gen.permutation(n)
        r = moveaxis(take_along_axis(m, _dev(idx), axis=-1), -1, ax).copy()
    if out is not None:
        out[...] = r
        return out
    return r


def choice(a, size=None, replace=True, p=None):
    """Sample indices from the generator (the draws NumPy makes for a
    population of that size), then the population gathered on the device."""
    from .indexing import take
    pv = _host_arg(p) if p is not None else None
    if isinstance(a, (int, np.integer)):
        return _fnd(np.asarray(_rng_gen.choice(int(a), size=size, replace=replace, p=pv)))
    pop = _dev(a)
    if pop.ndim != 1:
        raise ValueError("a must be 1-dimensional or an integer")
    idx = np.asarray(_rng_gen.choice(pop.shape[0], size=size, replace=replace, p=pv))
    r = take(pop, _dev(idx.astype(np.int64).ravel()))
    return r.reshape(idx.shape)


# ------------------------------------------------------------ state, misc
def bytes(length):
    return np.random.bytes(length)


def get_state():
    return _rng_gen.bit_generator.state


def set_state(state):
    _rng_gen.bit_generator.state = state


get_bit_generator = np.random.get_bit_generator
set_bit_generator = np.random.set_bit_generator
BitGenerator = np.random.BitGenerator
MT19937 = np.random.MT19937
PCG64 = np.random.PCG64
PCG64DXSM = np.random.PCG64DXSM
Philox = np.random.Philox
SFC64 = np.random.SFC64
SeedSequence = np.random.SeedSequence
RandomState = np.random.RandomState


class Generator:
    """The reference's Generator: a seed reseeds the module generator and
    every method draws from it."""

    def __init__(self, seed_val=None):
        if seed_val is not None:
            seed(seed_val)

    def integers(self, low, high=None, size=None, dtype=int, endpoint=False):
        if high is None:
            low, high = 0, low
        if endpoint:
            high = high + 1
        return randint(low, high, size=size, dtype=dtype)

    def random(self, size=None, dtype=np.float32, out=None):
        return random(size=size)

    def standard_normal(self, size=None, dtype=np.float32, out=None):
        return standard_normal(size)

    def standard_exponential(self, size=None, dtype=np.float32, method="zig", out=None):
        return standard_exponential(size)

    def shuffle(self, x, axis=0):
        return shuffle(x)

    def permutation(self, x, axis=0):
        return permutation(x)

    def permuted(self, x, axis=None, out=None):
        return permuted(x, axis=axis, out=out)

    def choice(self, a, size=None, replace=True, p=None, axis=0, shuffle=True):
        return choice(a, size=size, replace=replace, p=p)

    def multivariate_normal(self, mean, cov, size=None, check_valid="warn", tol=1e-8, *,
                            method="svd"):
        return multivariate_normal(mean, cov, size)

    def bytes(self, length):
        return _rng_gen.bytes(length)

    @property
    def bit_generator(self):
        return _rng_gen.bit_generator

    def __getattr__(self, name):
        if name in _FLOAT32_DRAWS or name in _INT32_DRAWS:
            return globals()[name]
        raise AttributeError(name)


def default_rng(seed_val=None):
    return Generator(seed_val)


__all__ = ["seed", "get_generator", "rand", "randn", "random", "standard_normal",
           "standard_exponential", "randint", "random_integers", "random_sample", "ranf",
           "sample", "multivariate_normal", "shuffle", "permutation", "permuted", "choice",
           "bytes", "get_state", "set_state", "get_bit_generator", "set_bit_generator",
           "BitGenerator", "MT19937", "PCG64", "PCG64DXSM", "Philox", "SFC64", "SeedSequence",
           "RandomState", "Generator", "default_rng"] + list(_FLOAT32_DRAWS) + list(_INT32_DRAWS)
