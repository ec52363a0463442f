"""Seeded draws match the reference's stream bit for bit (the reference
draws every distribution from one NumPy default_rng(seed), random.py:8-330,
float32 casts for continuous and int32 for discrete results), replayed here
with NumPy itself; permutations gather on the device from the same draws."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu
R = cp.random


def _h(a):
    return a.get() if hasattr(a, "get") else np.asarray(a)


def _same(got, want):
    got, want = _h(got), np.asarray(want)
    assert got.shape == want.shape and got.dtype == want.dtype, (got.shape, want.shape, got.dtype, want.dtype)
    assert np.array_equal(got, want, equal_nan=True)


CONT = [("normal", (1.0, 2.0)), ("uniform", (-1.0, 3.0)), ("beta", (2.0, 3.0)), ("exponential", (2.0,)),
        ("gamma", (2.0, 1.5)), ("standard_cauchy", ()), ("standard_gamma", (2.5,)), ("standard_t", (4.0,)),
        ("chisquare", (3.0,)), ("laplace", (0.5, 2.0)), ("logistic", (0.0, 1.0)), ("lognormal", (0.0, 0.5)),
        ("gumbel", (1.0, 2.0)), ("rayleigh", (2.0,)), ("triangular", (0.0, 1.0, 3.0)), ("weibull", (1.5,)),
        ("vonmises", (0.0, 2.0)), ("wald", (1.0, 2.0)), ("pareto", (3.0,)), ("f", (3.0, 5.0)),
        ("power", (2.0,)), ("noncentral_chisquare", (3.0, 1.0)), ("noncentral_f", (3.0, 5.0, 1.0))]
DISC = [("binomial", (10, 0.3)), ("poisson", (4.0,)), ("geometric", (0.3,)), ("zipf", (2.0,)),
        ("logseries", (0.7,)), ("hypergeometric", (10, 5, 6)), ("negative_binomial", (5, 0.4))]


def test_distributions_replay():
    R.seed(1234)
    g = np.random.default_rng(1234)
    _same(R.rand(3, 4), g.random((3, 4), dtype=np.float32))
    _same(R.randn(5), g.standard_normal(5, dtype=np.float32))
    _same(R.random(7), g.random(7, dtype=np.float32))
    _same(R.standard_exponential(6), g.standard_exponential(6, dtype=np.float32))
    _same(R.randint(0, 100, size=9), g.integers(0, 100, size=9, dtype=np.int32))
    _same(R.random_integers(5, size=4), g.integers(1, 6, size=4, dtype=np.int32))
    for name, args in CONT:
        _same(getattr(R, name)(*args, size=50), getattr(g, name)(*args, size=50).astype(np.float32))
    for name, args in DISC:
        _same(getattr(R, name)(*args, size=50), np.asarray(getattr(g, name)(*args, size=50), dtype=np.int32))
    _same(R.dirichlet([1.0, 2.0, 3.0], size=4), g.dirichlet([1.0, 2.0, 3.0], size=4).astype(np.float32))
    _same(R.multinomial(20, [0.2, 0.3, 0.5], size=3),
          np.asarray(g.multinomial(20, [0.2, 0.3, 0.5], size=3), dtype=np.int32))
    cov = np.array([[2.0, 0.3], [0.3, 1.0]])
    _same(R.multivariate_normal(cp.array(np.zeros(2)), cp.array(cov), size=5),
          g.multivariate_normal(np.zeros(2), cov, size=5).astype(np.float32))
    _same(R.randn(3), g.standard_normal(3, dtype=np.float32))


def test_permutations_replay():
    R.seed(7)
    g = np.random.default_rng(7)
    x = np.arange(40, dtype=np.float32).reshape(10, 4) * 1.5
    d = cp.array(x)
    R.shuffle(d)
    hx = x.copy()
    g.shuffle(hx)
    _same(d, hx)
    _same(R.permutation(12), np.asarray(g.permutation(12), dtype=np.int32))
    iv = np.arange(9, dtype=np.int32) * 3
    _same(R.permutation(cp.array(iv)), np.asarray(g.permutation(iv), dtype=np.float32))
    m = np.arange(24, dtype=np.int32).reshape(4, 6)
    t = m.copy()
    g.shuffle(t.ravel())
    _same(R.permuted(cp.array(m)), t)
    t = m.copy()
    np.apply_along_axis(lambda a: g.shuffle(a) or a, 1, t)
    _same(R.permuted(cp.array(m), axis=1), t)
    t = m.copy()
    np.apply_along_axis(lambda a: g.shuffle(a) or a, 0, t)
    _same(R.permuted(cp.array(m), axis=0), t)
    pop = np.linspace(0, 1, 11).astype(np.float32)
    _same(R.choice(cp.array(pop), size=6), g.choice(pop, size=6))
    _same(R.choice(cp.array(pop), size=(2, 3), replace=False), g.choice(pop, size=(2, 3), replace=False))
    p = np.full(11, 1 / 11)
    _same(R.choice(cp.array(pop), size=5, p=cp.array(p)), g.choice(pop, size=5, p=p))
    _same(R.choice(20, size=4), np.asarray(g.choice(20, size=4)))
    _same(R.rand(4), g.random(4, dtype=np.float32))


def test_generator_and_state():
    gen = R.default_rng(99)
    g = np.random.default_rng(99)
    _same(gen.random(5), g.random(5, dtype=np.float32))
    _same(gen.integers(10, size=3), g.integers(0, 10, size=3, dtype=np.int32))
    _same(gen.normal(0.0, 1.0, 4), g.normal(0.0, 1.0, 4).astype(np.float32))
    _same(gen.poisson(3.0, 4), np.asarray(g.poisson(3.0, 4), dtype=np.int32))
    st = R.get_state()
    a = R.rand(6)
    R.set_state(st)
    _same(R.rand(6), _h(a))
    assert isinstance(R.bytes(5), bytes) and len(R.bytes(5)) == 5
