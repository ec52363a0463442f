"""Host-side logic of the composed routines, checked on the CPU (no device
calls): einsum subscript parsing, pad's periodic index maps, the
matrix-chain order of multi_dot, pad's value typing, the legacy error
object, and the seeded random stream (host-resident draws)."""
import numpy as np
import pytest

from macmetalpy_amd import routines, linalg, host_api
import macmetalpy_amd as cp


@pytest.mark.parametrize("sub,shapes,want_out", [
    ("ij,jk->ik", [(2, 3), (3, 4)], "ik"),
    ("ij,jk", [(2, 3), (3, 4)], "ik"),
    ("ii", [(3, 3)], ""),
    ("ba,ca", [(2, 3), (4, 3)], "bc"),
    ("i,i", [(3,), (3,)], ""),
])
def test_einsum_parse_plain(sub, shapes, want_out):
    specs, out = routines._parse_einsum(sub, shapes)
    assert out == want_out
    assert [len(s) for s in specs] == [len(s) for s in shapes]


def test_einsum_parse_ellipsis():
    specs, out = routines._parse_einsum("...ij,...jk->...ik", [(5, 2, 3, 4), (2, 4, 6)])
    assert len(specs[0]) == 4 and len(specs[1]) == 3
    assert specs[0][2:] == "ij" and specs[1][1:] == "jk"
    assert specs[0][1] == specs[1][0]          # rightmost ellipsis dims aligned
    assert out.endswith("ik") and len(out) == 4
    _, impl = routines._parse_einsum("...i,i", [(7, 3), (3,)])
    assert len(impl) == 1                       # ellipsis only; i summed
    with pytest.raises(ValueError):
        routines._parse_einsum("ij,jk->il", [(2, 3), (3, 4)])
    with pytest.raises(ValueError):
        routines._parse_einsum("ij", [(2, 3, 4)])


@pytest.mark.parametrize("mode", ["edge", "wrap", "reflect", "symmetric"])
def test_pad_index_maps_match_numpy(mode):
    for n in range(1, 7):
        x = np.arange(10, 10 + n)
        for b in range(0, 13):
            for e in range(0, 13):
                idx = routines._pad_index(n, b, e, mode)
                assert np.array_equal(x[idx], np.pad(x, (b, e), mode=mode)), (n, b, e)


def test_pad_scalar_pairs_typing():
    one = routines._scalar_pairs(3, 2)
    assert one == [(one[0][0],) * 2] * 2 and isinstance(one[0][0], np.integer)
    two = routines._scalar_pairs((1.5, 2), 3)
    assert len(two) == 3 and isinstance(two[0][0], np.floating)
    table = routines._scalar_pairs(((1, 2), (3, 4)), 2)
    assert table == [[1, 2], [3, 4]] and type(table[0][0]) is int   # weak Python scalars


def test_matrix_chain_order():
    shapes = [(10, 30), (30, 5), (5, 60), (60, 8)]
    s = linalg._chain_order(shapes)

    def cost(i, j):
        if i == j:
            return 0
        k = s[i][j]
        return cost(i, k) + cost(k + 1, j) + shapes[i][0] * shapes[k][1] * shapes[j][1]

    best = {}

    def brute(i, j):
        if i == j:
            return 0
        if (i, j) not in best:
            best[(i, j)] = min(brute(i, k) + brute(k + 1, j) + shapes[i][0] * shapes[k][1] * shapes[j][1]
                               for k in range(i, j))
        return best[(i, j)]

    assert cost(0, 3) == brute(0, 3)


def test_error_object_roundtrip():
    old = host_api.geterrobj()
    try:
        host_api.seterrobj([8192, (2 << 0) | (0 << 3) | (1 << 6) | (3 << 9), None])
        st = np.geterr()
        assert st == {"divide": "raise", "over": "ignore", "under": "warn", "invalid": "call"}
        assert host_api.geterrobj()[1] == (2 << 0) | (0 << 3) | (1 << 6) | (3 << 9)
    finally:
        host_api.seterrobj(old)
    assert host_api.common_type(np.zeros(2, np.int32), np.zeros(2, np.float32)) is np.float64
    assert host_api.common_type(np.zeros(2, np.float16)) is np.float16
    assert host_api.set_numeric_ops() == {}


def test_seeded_draws_are_the_reference_stream():
    cp.random.seed(5)
    g = np.random.default_rng(5)
    a = cp.random.randn(4, 3)
    b = cp.random.gamma(2.0, 1.0, size=6)
    c = cp.random.poisson(3.0, size=6)
    assert a._np_data is not None and b._np_data is not None      # host-resident draws
    assert np.array_equal(a._np_data, g.standard_normal((4, 3), dtype=np.float32))
    assert np.array_equal(b._np_data, g.gamma(2.0, 1.0, size=6).astype(np.float32))
    assert np.array_equal(c._np_data, np.asarray(g.poisson(3.0, size=6), dtype=np.int32))
    st = cp.random.get_state()
    x = cp.random.rand(5)._np_data
    cp.random.set_state(st)
    assert np.array_equal(cp.random.rand(5)._np_data, x)
