"""cp.linalg on the device against NumPy / LAPACK: solve, inv, det,
slogdet, cholesky, qr, eigh, svd and what is built on them, the norms and
the product helpers; polyfit through lstsq.  Factorizations agree to
rounding (LAPACK blocks and orders its sums differently): float64 to
rtol 1e-9, float32 to rtol 2e-4 on well-conditioned inputs.  Eigen- and
singular vectors are unique only up to sign, so they are checked through
reconstruction and orthonormality; QR uses LAPACK's reflector signs and is
compared entry by entry."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu
LA = cp.linalg


def _h(a):
    return a.get() if hasattr(a, "get") else np.asarray(a)


def _close(got, want, rtol=1e-9, atol=1e-10, dtype=True):
    got, want = _h(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    if dtype:
        assert got.dtype == want.dtype, (got.dtype, want.dtype)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)


def _m(shape, dtype=np.float64, seed=0, spd=False, well=True):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(shape)
    if well and shape[-1] == shape[-2]:
        a = a + np.eye(shape[-1]) * shape[-1] * 0.5
    if spd:
        a = a @ np.swapaxes(a, -1, -2) + np.eye(shape[-1]) * shape[-1]
    return a.astype(dtype)


TOL = {np.float64: (1e-9, 1e-10), np.float32: (2e-4, 2e-5)}


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_solve_inv_det(dt):
    rt, at = TOL[dt]
    for n in (1, 2, 5, 33, 130):
        a = _m((n, n), dt, n)
        b = _m((n,), dt, n + 1, well=False)
        B = _m((n, 3), dt, n + 2, well=False)
        _close(LA.solve(cp.array(a), cp.array(b)), np.linalg.solve(a, b), rt, at)
        _close(LA.solve(cp.array(a), cp.array(B)), np.linalg.solve(a, B), rt, at)
        _close(LA.inv(cp.array(a)), np.linalg.inv(a), rt, at)
        _close(LA.det(cp.array(a)), np.linalg.det(a), rt * 10, 0)
        s, l = LA.slogdet(cp.array(a))
        ws, wl = np.linalg.slogdet(a)
        _close(s, ws, 0, 0)
        _close(l, wl, rt, at)
    A = _m((3, 6, 6), dt, 7)
    Bb = _m((3, 6, 2), dt, 8, well=False)
    _close(LA.solve(cp.array(A), cp.array(Bb)), np.linalg.solve(A, Bb), rt, at)
    _close(LA.solve(cp.array(A[0]), cp.array(Bb)), np.linalg.solve(A[0], Bb), rt, at)
    _close(LA.inv(cp.array(A)), np.linalg.inv(A), rt, at)
    _close(LA.det(cp.array(A)), np.linalg.det(A), rt * 10, 0)


def test_singular_and_dtypes():
    s = np.array([[1.0, 2.0], [2.0, 4.0]])
    with pytest.raises(LA.LinAlgError):
        LA.solve(cp.array(s), cp.array(np.ones(2)))
    with pytest.raises(LA.LinAlgError):
        LA.inv(cp.array(s))
    z = np.zeros((3, 3))
    _close(LA.det(cp.array(z)), np.linalg.det(z), 0, 0)
    sg, ld = LA.slogdet(cp.array(z))
    assert float(_h(sg)) == 0.0 and _h(ld) == -np.inf
    p = np.array([[0.0, 1.0, 0.0], [0.0, 0.0, 1.0], [1.0, 0.0, 0.0]])
    _close(LA.det(cp.array(p)), np.linalg.det(p), 1e-15, 0)
    q = np.array([[0.0, 1.0], [1.0, 0.0]])
    _close(LA.det(cp.array(q)), np.linalg.det(q), 1e-15, 0)
    i = np.array([[2, 1], [1, 3]], dtype=np.int32)
    _close(LA.inv(cp.array(i)), np.linalg.inv(i))
    with pytest.raises(TypeError):
        LA.inv(cp.array(np.eye(2, dtype=np.float16)))
    with pytest.raises(LA.LinAlgError):
        LA.inv(cp.array(np.ones((2, 3))))


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_cholesky_qr(dt):
    rt, at = TOL[dt]
    for n in (1, 4, 40):
        a = _m((n, n), dt, 20 + n, spd=True)
        _close(LA.cholesky(cp.array(a)), np.linalg.cholesky(a), rt, at * n)
        _close(LA.cholesky(cp.array(a), upper=True), np.linalg.cholesky(a, upper=True), rt, at * n)
    A = _m((2, 5, 5), dt, 30, spd=True)
    _close(LA.cholesky(cp.array(A)), np.linalg.cholesky(A), rt, at * 5)
    with pytest.raises(LA.LinAlgError):
        LA.cholesky(cp.array(-np.eye(3, dtype=dt)))
    for shape in ((6, 4), (4, 6), (5, 5), (50, 20), (3, 7, 5)):
        a = _m(shape, dt, 40, well=False)
        for mode in ("reduced", "complete"):
            gq, gr = LA.qr(cp.array(a), mode=mode)
            wq, wr = np.linalg.qr(a, mode=mode)
            _close(gq, wq, rt * 10, at * 10)
            _close(gr, wr, rt * 10, at * 10)
        _close(LA.qr(cp.array(a), mode="r"), np.linalg.qr(a, mode="r"), rt * 10, at * 10)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_eigh(dt):
    rt, at = TOL[dt]
    for n in (1, 2, 7, 64):
        g = _m((n, n), np.float64, 50 + n, well=False)
        a = ((g + g.T) / 2).astype(dt)
        w, v = LA.eigh(cp.array(a))
        ww = np.linalg.eigvalsh(a)
        _close(w, ww, rt, at * n)
        vh = _h(v).astype(np.float64)
        np.testing.assert_allclose(vh @ np.diag(_h(w)) @ vh.T, a, rtol=0, atol=at * 50 * n)
        np.testing.assert_allclose(vh.T @ vh, np.eye(n), rtol=0, atol=at * 50 * n)
        _close(LA.eigvalsh(cp.array(a)), ww, rt, at * n)
    g = _m((6, 6), dt, 60, well=False)
    _close(LA.eigvalsh(cp.array(g), UPLO="U"), np.linalg.eigvalsh(g, UPLO="U"), rt, at * 6)
    _close(LA.eigvalsh(cp.array(g)), np.linalg.eigvalsh(g), rt, at * 6)
    b = _m((3, 5, 5), np.float64, 61, well=False)
    b = ((b + np.swapaxes(b, 1, 2)) / 2).astype(dt)
    _close(LA.eigh(cp.array(b))[0], np.linalg.eigh(b)[0], rt, at * 5)
    e = np.diag([3.0, 1.0, 1.0, 2.0]).astype(dt)
    _close(LA.eigvalsh(cp.array(e)), np.linalg.eigvalsh(e), rt, at)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_svd_family(dt):
    rt, at = TOL[dt]
    for shape in ((7, 5), (5, 7), (6, 6), (1, 4), (40, 25), (2, 6, 3)):
        a = _m(shape, dt, 70, well=False)
        u, s, vh = LA.svd(cp.array(a), full_matrices=False)
        ws = np.linalg.svd(a, compute_uv=False)
        _close(s, ws, rt, at * 10)
        uh, sh, vhh = (_h(x).astype(np.float64) for x in (u, s, vh))
        np.testing.assert_allclose(uh @ (sh[..., :, None] * vhh), a, rtol=0, atol=at * 100)
        k = min(shape[-2:])
        np.testing.assert_allclose(np.swapaxes(uh, -1, -2) @ uh, np.broadcast_to(np.eye(k), uh.shape[:-2] + (k, k)),
                                   rtol=0, atol=at * 100)
        U, S, Vh = LA.svd(cp.array(a))
        Uh, Vhh = _h(U).astype(np.float64), _h(Vh).astype(np.float64)
        m, n = shape[-2:]
        assert Uh.shape[-2:] == (m, m) and Vhh.shape[-2:] == (n, n)
        np.testing.assert_allclose(np.swapaxes(Uh, -1, -2) @ Uh, np.broadcast_to(np.eye(m), Uh.shape), rtol=0, atol=at * 100)
        np.testing.assert_allclose(Vhh @ np.swapaxes(Vhh, -1, -2), np.broadcast_to(np.eye(n), Vhh.shape), rtol=0, atol=at * 100)
        _close(LA.svdvals(cp.array(a)), ws, rt, at * 10)
        _close(LA.svd(cp.array(a), compute_uv=False), ws, rt, at * 10)
    a = _m((8, 6), dt, 71, well=False)
    _close(LA.pinv(cp.array(a)), np.linalg.pinv(a), rt * 10, at * 10)
    r = (_m((9, 3), np.float64, 72, well=False) @ _m((3, 7), np.float64, 73, well=False)).astype(dt)
    assert LA.matrix_rank(cp.array(r)) == np.linalg.matrix_rank(r) == 3
    assert LA.matrix_rank(cp.array(np.zeros(4))) == 0
    sq = _m((5, 5), dt, 74)
    _close(LA.cond(cp.array(sq)), np.linalg.cond(sq), rt * 10, 0)
    for p in (1, -1, np.inf, "fro", -2):
        _close(LA.cond(cp.array(sq), p), np.linalg.cond(sq, p), rt * 10, 0)


def test_lstsq_polyfit():
    a = _m((30, 4), np.float64, 80, well=False)
    b = _m((30,), np.float64, 81, well=False)
    B = _m((30, 2), np.float64, 82, well=False)
    for rhs in (b, B):
        gx, gr, grank, gs = LA.lstsq(cp.array(a), cp.array(rhs))
        wx, wr, wrank, ws = np.linalg.lstsq(a, rhs)
        _close(gx, wx)
        _close(gr, wr, 1e-9, 1e-9)
        assert grank == wrank
        _close(gs, ws)
    r = a[:, :2] @ _m((2, 4), np.float64, 83, well=False)
    gx, gr, grank, _ = LA.lstsq(cp.array(r), cp.array(b))
    wx, wr, wrank, _ = np.linalg.lstsq(r, b)
    assert grank == wrank == 2 and _h(gr).shape == wr.shape == (0,)
    _close(gx, wx, 1e-8, 1e-9)
    w = _m((5, 3), np.float64, 84, well=False)
    _close(LA.lstsq(cp.array(w.T), cp.array(b[:3]))[0], np.linalg.lstsq(w.T, b[:3])[0], 1e-8, 1e-9)
    x = np.linspace(-2, 3, 40)
    y = 0.5 * x ** 3 - x + 2 + np.sin(7 * x) * 0.1
    for deg in (1, 3, 5):
        _close(cp.polyfit(cp.array(x), cp.array(y), deg), np.polyfit(x, y, deg), 1e-8, 1e-9)
    Y = np.stack([y, 2 * y + 1], axis=1)
    _close(cp.polyfit(cp.array(x), cp.array(Y), 2), np.polyfit(x, Y, 2), 1e-8, 1e-9)


def test_norms():
    a = _m((5, 7), np.float64, 90, well=False)
    v = a[0]
    for ord_ in (None, 0, 1, 2, np.inf, -np.inf, 3, -1.5):
        _close(LA.norm(cp.array(v), ord_), np.linalg.norm(v, ord_), 1e-12, 1e-12)
    for ord_ in (None, "fro", "nuc", 1, -1, 2, -2, np.inf, -np.inf):
        _close(LA.norm(cp.array(a), ord_), np.linalg.norm(a, ord_), 1e-10, 1e-12)
    t = _m((3, 4, 5), np.float64, 91, well=False)
    for ax in (0, 1, -1, (0, 1), (2, 0), (1, 2)):
        for kd in (False, True):
            _close(LA.norm(cp.array(t), axis=ax, keepdims=kd), np.linalg.norm(t, axis=ax, keepdims=kd), 1e-12, 1e-12)
    _close(LA.norm(cp.array(t), 1, axis=(2, 0)), np.linalg.norm(t, 1, axis=(2, 0)), 1e-12, 1e-12)
    _close(LA.norm(cp.array(t), np.inf, axis=(1, 2)), np.linalg.norm(t, np.inf, axis=(1, 2)), 1e-12, 1e-12)
    _close(LA.norm(cp.array(t)), np.linalg.norm(t), 1e-12, 1e-12)
    _close(LA.norm(cp.array(t), keepdims=True), np.linalg.norm(t, keepdims=True), 1e-12, 1e-12)
    _close(LA.vector_norm(cp.array(t), ord=3, axis=1), np.linalg.vector_norm(t, ord=3, axis=1), 1e-12, 1e-12)
    _close(LA.matrix_norm(cp.array(t), ord=1), np.linalg.matrix_norm(t, ord=1), 1e-12, 1e-12)
    i = np.arange(12, dtype=np.int32).reshape(3, 4)
    _close(LA.norm(cp.array(i)), np.linalg.norm(i), 1e-12)
    f = a.astype(np.float32)
    _close(LA.norm(cp.array(f)), np.linalg.norm(f), 1e-6)


def test_products_and_helpers():
    ai = np.array([[1, 2], [3, 1]], dtype=np.int64)
    for n in (0, 1, 2, 3, 5, 8, 13):
        _close(LA.matrix_power(cp.array(ai), n), np.linalg.matrix_power(ai, n), 0, 0)
    af = _m((4, 4), np.float64, 100)
    _close(LA.matrix_power(cp.array(af), -3), np.linalg.matrix_power(af, -3), 1e-9, 1e-12)
    ms = [_m(s, np.float64, 101 + k, well=False) for k, s in enumerate([(10, 30), (30, 5), (5, 60), (60, 8)])]
    _close(LA.multi_dot([cp.array(m) for m in ms]), np.linalg.multi_dot(ms), 1e-10, 1e-10)
    _close(LA.multi_dot([cp.array(ms[0][0]), cp.array(ms[1]), cp.array(ms[2][:, 0])]),
           np.linalg.multi_dot([ms[0][0], ms[1], ms[2][:, 0]]), 1e-10, 1e-10)
    t = _m((2, 3, 6), np.float64, 105)
    tb = _m((2, 3), np.float64, 106, well=False)
    ta = np.einsum("ijk,kl->ijl", t, _m((6, 6), np.float64, 107)).reshape(2, 3, 2, 3) + \
        np.eye(6).reshape(2, 3, 2, 3) * 5
    _close(LA.tensorsolve(cp.array(ta), cp.array(tb)), np.linalg.tensorsolve(ta, tb), 1e-9, 1e-10)
    _close(LA.tensorinv(cp.array(ta), 2), np.linalg.tensorinv(ta, 2), 1e-9, 1e-10)
    x, y = _m((4, 3), np.float64, 108, well=False), _m((4, 3), np.float64, 109, well=False)
    _close(LA.cross(cp.array(x), cp.array(y)), np.linalg.cross(x, y), 1e-14, 1e-14)
    _close(LA.diagonal(cp.array(t), offset=1), np.linalg.diagonal(t, offset=1), 0, 0)
    _close(LA.matrix_transpose(cp.array(t)), np.linalg.matrix_transpose(t), 0, 0)
    _close(LA.outer(cp.array(x[0]), cp.array(y[1])), np.linalg.outer(x[0], y[1]), 0, 0)
    _close(LA.tensordot(cp.array(t), cp.array(t), axes=([1, 2], [1, 2])),
           np.linalg.tensordot(t, t, axes=([1, 2], [1, 2])), 1e-12, 1e-12)
    _close(LA.trace(cp.array(t)), np.linalg.trace(t), 1e-14, 1e-14)
    _close(LA.vecdot(cp.array(x), cp.array(y)), np.linalg.vecdot(x, y), 1e-14, 1e-14)
    _close(LA.matmul(cp.array(x), cp.array(y.T.copy())), np.linalg.matmul(x, y.T), 1e-12, 1e-12)


def test_larger_batched():
    a = _m((2, 200, 200), np.float64, 120)
    b = _m((2, 200, 5), np.float64, 121, well=False)
    _close(LA.solve(cp.array(a), cp.array(b)), np.linalg.solve(a, b), 1e-9, 1e-10)
    g = _m((96, 96), np.float64, 122, well=False)
    s = (g + g.T) / 2
    _close(LA.eigvalsh(cp.array(s)), np.linalg.eigvalsh(s), 1e-9, 1e-10)
    r = _m((160, 90), np.float64, 123, well=False)
    _close(LA.svdvals(cp.array(r)), np.linalg.svd(r, compute_uv=False), 1e-9, 1e-10)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_blocked_lu_sizes(dt):
    # orders >= 256 take the blocked LU (64-column panels, matmul updates)
    rt, at = TOL[dt]
    for n in (256, 300, 517):
        a = _m((n, n), dt, 200 + n)
        b = _m((n, 3), dt, 201 + n, well=False)
        _close(LA.solve(cp.array(a), cp.array(b)), np.linalg.solve(a, b), rt * 10, at * 10)
        sg, ld = LA.slogdet(cp.array(a))
        ws, wl = np.linalg.slogdet(a)
        _close(sg, ws, 0, 0)
        _close(ld, wl, rt * 10, at * 10)
    a = _m((260, 260), dt, 210)
    _close(LA.inv(cp.array(a)), np.linalg.inv(a), rt * 10, at * 10)
    p = np.eye(300, dtype=dt)[np.random.default_rng(3).permutation(300)] * 2
    _close(LA.det(cp.array(p)), np.linalg.det(p).astype(dt), rt * 10, 0)
    A = _m((3, 280, 280), dt, 211)
    B = _m((3, 280, 2), dt, 212, well=False)
    _close(LA.solve(cp.array(A), cp.array(B)), np.linalg.solve(A, B), rt * 10, at * 10)
    s = _m((320, 320), dt, 213)
    s[:, 100] = 0
    with pytest.raises(LA.LinAlgError):
        LA.solve(cp.array(s), cp.array(np.ones(320, dt)))
    _close(LA.det(cp.array(s)), np.zeros((), dt), 0, 0)


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_blocked_cholesky_sizes(dt):
    # orders >= 256 take the blocked Cholesky (only the lower triangle is read)
    rt, at = TOL[dt]
    for n in (256, 333):
        a = _m((n, n), np.float64, 300 + n, spd=True)
        lo = np.tril(a) + np.triu(np.full((n, n), 7.0), 1)   # garbage above the diagonal
        want = np.linalg.cholesky(a.astype(dt))
        _close(LA.cholesky(cp.array(lo.astype(dt))), want, rt * 10, at * n)
    bad = _m((300, 300), np.float64, 310, spd=True)
    bad[200, 200] = -1.0
    with pytest.raises(LA.LinAlgError):
        LA.cholesky(cp.array(bad.astype(dt)))


def test_split_k_matmul():
    # small outputs with long sums run as a batched matmul over K chunks
    rng = np.random.default_rng(400)
    for dt, rt in ((np.float64, 1e-12), (np.float32, 2e-5)):
        for (m, k, n) in ((64, 40000, 32), (1, 16384, 1), (100, 20001, 100), (3, 70000, 5)):
            a = rng.standard_normal((m, k)).astype(dt)
            b = rng.standard_normal((k, n)).astype(dt)
            want = a.astype(np.float64) @ b.astype(np.float64)
            got = _h(cp.matmul(cp.array(a), cp.array(b)))
            assert got.dtype == dt and got.shape == (m, n)
            np.testing.assert_allclose(got, want, rtol=rt, atol=rt * np.sqrt(k) * 5)
    x = rng.standard_normal((64, 1 << 18))
    np.testing.assert_allclose(_h(cp.cov(cp.array(x))), np.cov(x), rtol=1e-10, atol=1e-12)


def test_eig_symmetric():
    g = _m((6, 6), np.float64, 500, well=False)
    s = (g + g.T) / 2
    w, v = LA.eig(cp.array(s))
    ww = np.linalg.eig(s)[0]
    assert _h(w).dtype == ww.dtype == np.float64
    np.testing.assert_allclose(np.sort(_h(w)), np.sort(ww), rtol=1e-10, atol=1e-12)
    vh = _h(v)
    np.testing.assert_allclose(s @ vh, vh * _h(w)[None, :], rtol=0, atol=1e-10)
    np.testing.assert_allclose(np.sort(_h(LA.eigvals(cp.array(s)))), np.sort(np.linalg.eigvals(s)),
                               rtol=1e-10, atol=1e-12)
    with pytest.raises(NotImplementedError):
        LA.eig(cp.array(g))


def test_nan_input_and_convergence_errors():
    """NumPy's behaviour on non-finite input: svd (and what is built on it)
    raises LinAlgError('SVD did not converge'), eig / eigvals refuse NaN /
    inf, eigh returns without raising."""
    a = np.array([[np.nan, 0.0], [0.0, 1.0]])
    A = cp.array(a)
    for f in (cp.linalg.svd, cp.linalg.pinv, cp.linalg.matrix_rank, cp.linalg.cond):
        with pytest.raises(cp.linalg.LinAlgError, match="SVD did not converge"):
            f(A)
        with pytest.raises(np.linalg.LinAlgError):
            getattr(np.linalg, f.__name__)(a)
    for f in (cp.linalg.eig, cp.linalg.eigvals):
        with pytest.raises(cp.linalg.LinAlgError, match="infs or NaNs"):
            f(A)
    w, v = cp.linalg.eigh(A)  # no error, as NumPy
    assert w.shape == (2,)
