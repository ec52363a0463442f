"""Seeded random expression DAGs through the fusion engine.

The reference compiles each lazy DAG into one generated kernel
(_fusion.py:297-409) and checks chains of fused ops against NumPy
(tests/test_fusion.py:9-209).  Here random DAGs -- broadcast row, column
and 1-D leaves, strided and transposed views, Python scalars, shared
subexpressions, optional row or whole-array sums at the root -- are
evaluated three ways:

* unfused (one library kernel per op): every node is checked against
  NumPy applied to the device values of its own operands -- exact ops
  bit for bit, transcendentals within 2 ULP of the float64 evaluation;
* fused (one generated kernel per DAG): bit for bit equal to the unfused
  result, NaN == NaN;
* a fused sum at the root: within 1 ULP of the float64 sum of the
  unfused values (float results; int32 results sum to int64 exactly).

Mixed DAGs draw int32, float32 and float64 leaves, so NumPy's promotion
(int32 with float32 or a Python float gives float64) runs through fused
casts; every node's dtype must be NumPy's.

Integer DAGs (wrapping int32 arithmetic, floor_divide / mod by signed
divisors, bitwise ops, shifts) are compared with NumPy evaluating the
whole expression, bit for bit, fused and unfused."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 5), (17, 129), (64, 1000), (1, 4096), (257, 33), (8, 4096), (100, 64)]


class Node:
    """One expression node: a leaf (index into the leaf table), a unary,
    binary or where op.  Shared subexpressions are the same Node object."""

    __slots__ = ("kind", "op", "kids", "leaf", "bound")

    def __init__(self, kind, op=None, kids=(), leaf=None, bound=1.0):
        self.kind, self.op, self.kids, self.leaf, self.bound = kind, op, tuple(kids), leaf, bound


# float unary ops: name -> (apply on module m, float64 reference or None
# for exact ops, output bound from input bound)
F_UNARY = {
    "neg": (lambda m, a: -a, None, lambda b: b),
    "abs": (lambda m, a: m.abs(a), None, lambda b: b),
    "square": (lambda m, a: a * a, None, lambda b: b * b),
    "tanh": (lambda m, a: m.tanh(a), np.tanh, lambda b: 1.0),
    "sin": (lambda m, a: m.sin(a), np.sin, lambda b: 1.0),
    "cos": (lambda m, a: m.cos(a), np.cos, lambda b: 1.0),
    "exp": (lambda m, a: m.exp(a), np.exp, lambda b: float(np.exp(min(b, 80.0)))),
    "log1p": (lambda m, a: m.log1p(a), np.log1p, lambda b: float(np.log1p(b)) + 1.0),
    "sqrt": (lambda m, a: m.sqrt(a), None, lambda b: float(np.sqrt(b))),
}
# domain guards applied to the operand before the op (themselves nodes)
F_GUARD = {"log1p": "abs", "sqrt": "abs", "exp": "negabs"}
F_BINARY = {
    "add": (lambda m, a, b: a + b, lambda x, y: x + y),
    "sub": (lambda m, a, b: a - b, lambda x, y: x + y),
    "mul": (lambda m, a, b: a * b, lambda x, y: x * y),
    "max": (lambda m, a, b: m.maximum(a, b), max),
    "min": (lambda m, a, b: m.minimum(a, b), max),
    "div": (lambda m, a, b: a / (m.abs(b) + 1.0), lambda x, y: x),
}
I_BINARY = {
    "add": lambda m, a, b: a + b,
    "sub": lambda m, a, b: a - b,
    "mul": lambda m, a, b: a * b,
    "and": lambda m, a, b: a & b,
    "or": lambda m, a, b: a | b,
    "xor": lambda m, a, b: a ^ b,
    "max": lambda m, a, b: m.maximum(a, b),
    "min": lambda m, a, b: m.minimum(a, b),
}


def _make_leaves(rng, R, C, dtypes, n):
    """n leaves: (host array or Python scalar, device array or scalar); each
    leaf's dtype is drawn from ``dtypes`` (a dtype or a list of them)."""
    leaves = []
    choices = list(dtypes) if isinstance(dtypes, (list, tuple)) else [dtypes]
    for _ in range(n):
        kind = rng.choice(["full", "full", "row", "col", "vec", "strided", "transposed", "scalar"])
        dtype = choices[int(rng.integers(len(choices)))]
        if dtype in (np.float32, np.float64):
            draw = lambda shape: rng.standard_normal(shape).astype(dtype)  # noqa: E731
        else:
            draw = lambda shape: rng.integers(-2**20, 2**20, shape, dtype=np.int32)  # noqa: E731
        if kind == "scalar":
            v = float(np.round(rng.uniform(-3, 3), 3)) if dtype != np.int32 else int(rng.integers(-50, 50))
            leaves.append((v, v))
            continue
        if kind == "full":
            h = draw((R, C)); d = cp.array(h)
        elif kind == "row":
            h = draw((1, C)); d = cp.array(h)
        elif kind == "col":
            h = draw((R, 1)); d = cp.array(h)
        elif kind == "vec":
            h = draw((C,)); d = cp.array(h)
        elif kind == "strided":
            base = draw((2 * R, C)); h = base[::2]; d = cp.array(base)[::2]
        else:
            base = draw((C, R)); h = base.T; d = cp.array(base).T
        leaves.append((h, d))
    if all(np.ndim(h) == 0 for h, _ in leaves):            # at least one array leaf
        h = draw((R, C))
        leaves[0] = (h, cp.array(h))
    return leaves


def _leaf_bound(h):
    return float(np.max(np.abs(h))) if np.ndim(h) else abs(float(h))


def _float_tree(rng, leaves, depth, pool):
    if depth == 0 or rng.random() < 0.25:
        i = int(rng.integers(len(leaves)))
        return Node("leaf", leaf=i, bound=_leaf_bound(leaves[i][0]))
    if pool and rng.random() < 0.15:                       # shared subexpression
        return pool[int(rng.integers(len(pool)))]
    r = rng.random()
    if r < 0.4:
        op = str(rng.choice(list(F_UNARY)))
        kid = _float_tree(rng, leaves, depth - 1, pool)
        if kid.kind == "leaf" and np.ndim(leaves[kid.leaf][0]) == 0:
            return kid                                     # no op on a bare scalar
        guard = F_GUARD.get(op)
        if guard == "abs":
            kid = Node("un", "abs", [kid], bound=kid.bound)
        elif guard == "negabs":
            kid = Node("un", "neg", [Node("un", "abs", [kid], bound=kid.bound)], bound=kid.bound)
        if op in ("sin", "cos") and kid.bound > 1e4:
            op = "tanh"
        if op == "square" and kid.bound > 1e6:
            op = "tanh"
        node = Node("un", op, [kid], bound=F_UNARY[op][2](kid.bound))
    elif r < 0.9:
        op = str(rng.choice(list(F_BINARY)))
        a = _float_tree(rng, leaves, depth - 1, pool)
        b = _float_tree(rng, leaves, depth - 1, pool)
        if op == "mul" and a.bound * b.bound > 1e12:
            op = "add"
        if (a.kind == "leaf" and np.ndim(leaves[a.leaf][0]) == 0
                and b.kind == "leaf" and np.ndim(leaves[b.leaf][0]) == 0):
            return a
        node = Node("bin", op, [a, b], bound=F_BINARY[op][1](a.bound, b.bound))
    else:
        kids = [_float_tree(rng, leaves, depth - 1, pool) for _ in range(4)]
        if any(k.kind == "leaf" and np.ndim(leaves[k.leaf][0]) == 0 for k in kids):
            return kids[0]
        node = Node("where", kids=kids, bound=max(kids[2].bound, kids[3].bound))
    pool.append(node)
    return node


def _apply(m, node, vals):
    if node.kind == "un":
        return F_UNARY[node.op][0](m, vals[0])
    if node.kind == "bin":
        return F_BINARY[node.op][0](m, vals[0], vals[1])
    return m.where(vals[0] > vals[1], vals[2], vals[3])


def _eval(m, node, leaf_vals, memo):
    key = id(node)
    if key not in memo:
        if node.kind == "leaf":
            memo[key] = leaf_vals[node.leaf]
        else:
            memo[key] = _apply(m, node, [_eval(m, k, leaf_vals, memo) for k in node.kids])
    return memo[key]


def _same(a, b):
    """Bit for bit, NaN == NaN."""
    a = np.ascontiguousarray(a); b = np.ascontiguousarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    nan = np.isnan(a) & np.isnan(b) if a.dtype.kind == "f" else np.zeros(a.shape, bool)
    bad = (a.view(np.uint8).reshape(a.shape + (-1,)) != b.view(np.uint8).reshape(b.shape + (-1,))).any(-1)
    assert not np.any(bad & ~nan), f"{int(np.sum(bad & ~nan))} elements differ"


def _host(v):
    return v.get() if isinstance(v, cp.ndarray) else v


def _check_node_unfused(node, got, kid_vals):
    """NumPy applied to the device operands of this node (Python scalars
    stay Python scalars, so NumPy promotes exactly as the library does)."""
    got = np.asarray(got)
    with np.errstate(all="ignore"):
        want = np.asarray(_apply(np, node, kid_vals))
        assert got.dtype == want.dtype, (node.kind, node.op, got.dtype, want.dtype)
        if node.kind == "un" and F_UNARY[node.op][1] is not None:
            if got.dtype == np.float32:
                want = F_UNARY[node.op][1](np.asarray(kid_vals[0]).astype(np.float64))
                want = want.astype(np.float32)
            d = ref.ulp_distance(got, want)
            assert int(np.max(d, initial=0)) <= 2, f"{node.op} {got.dtype}: {int(np.max(d))} ULP"
            return
    _same(got, want)


@pytest.mark.parametrize("seed", range(40))
def test_random_float_dag(seed):
    _run_float_dag(seed, 1000, np.float32)


@pytest.mark.parametrize("seed", range(24))
def test_random_mixed_dtype_dag(seed):
    """int32, float32 and float64 leaves: NumPy's promotion (int32 with
    float32 or a Python float gives float64) through fused casts."""
    _run_float_dag(seed, 3000, [np.float32, np.int32, np.float32, np.float64])


def _run_float_dag(seed, base, dtypes):
    rng = np.random.default_rng(base + seed)
    R, C = SHAPES[seed % len(SHAPES)]
    leaves = _make_leaves(rng, R, C, dtypes, int(rng.integers(2, 6)))
    root = None
    while root is None or root.kind == "leaf":
        root = _float_tree(rng, leaves, int(rng.integers(2, 6)), [])
    host_leaves = [h for h, _ in leaves]
    dev_leaves = [d for _, d in leaves]

    # unfused: every node against NumPy on its own device operands
    cp.set_config(fusion=False)
    memo = {}
    _eval(cp, root, dev_leaves, memo)
    host = {k: _host(v) for k, v in memo.items()}

    def walk(node, seen):
        if id(node) in seen or node.kind == "leaf":
            return
        seen.add(id(node))
        for k in node.kids:
            walk(k, seen)
        _check_node_unfused(node, host[id(node)], [host[id(k)] for k in node.kids])

    walk(root, set())
    unfused = host[id(root)]

    # fused: one generated kernel, bit-identical to the op-by-op result
    cp.set_config(fusion=True)
    fused = _eval(cp, root, dev_leaves, {})
    assert fused._fusion_node is not None
    _same(fused.get(), unfused)

    # fused sum at the root (row sums for 2-D results, else the whole array)
    axis = 1 if (unfused.ndim == 2 and seed % 2 == 0) else None
    if unfused.dtype.kind == "i":                          # int32 sums to int64, exactly
        s = cp.sum(_eval(cp, root, dev_leaves, {}), axis=axis).get()
        _same(s, np.sum(unfused, axis=axis))
    elif np.all(np.isfinite(unfused)):
        # the sum accumulates in float64: within one unit in the last place
        # of the result, plus float64 rounding over the terms
        s = cp.sum(_eval(cp, root, dev_leaves, {}), axis=axis).get()
        assert np.asarray(s).dtype == unfused.dtype
        want = np.sum(unfused.astype(np.float64), axis=axis)
        mag = np.sum(np.abs(unfused.astype(np.float64)), axis=axis)
        tol = np.spacing(np.abs(want).astype(unfused.dtype)).astype(np.float64) + 1e-13 * mag
        assert np.all(np.abs(np.asarray(s, np.float64) - want) <= tol)
    # the leaves are untouched
    for h, d in leaves:
        if np.ndim(h):
            _same(d.get(), np.ascontiguousarray(h))


def _int_tree(rng, leaves, depth, pool):
    if depth == 0 or rng.random() < 0.25:
        return Node("leaf", leaf=int(rng.integers(len(leaves))))
    if pool and rng.random() < 0.15:
        return pool[int(rng.integers(len(pool)))]
    r = rng.random()
    if r < 0.2:
        op = str(rng.choice(["neg", "abs", "rshift", "lshift", "not"]))
        kid = _int_tree(rng, leaves, depth - 1, pool)
        if kid.kind == "leaf" and np.ndim(leaves[kid.leaf][0]) == 0:
            return kid
        node = Node("iun", op, [kid], bound=float(rng.integers(0, 8)))
    elif r < 0.35:
        # floor_divide / mod by a signed divisor in [-13, -1] u [1, 13]
        a = _int_tree(rng, leaves, depth - 1, pool)
        b = _int_tree(rng, leaves, depth - 1, pool)
        c = _int_tree(rng, leaves, depth - 1, pool)
        if any(k.kind == "leaf" and np.ndim(leaves[k.leaf][0]) == 0 for k in (b, c)):
            return a
        node = Node("idiv", str(rng.choice(["floordiv", "mod"])), [a, b, c])
    else:
        op = str(rng.choice(list(I_BINARY)))
        a = _int_tree(rng, leaves, depth - 1, pool)
        b = _int_tree(rng, leaves, depth - 1, pool)
        if (a.kind == "leaf" and np.ndim(leaves[a.leaf][0]) == 0
                and b.kind == "leaf" and np.ndim(leaves[b.leaf][0]) == 0):
            return a
        node = Node("ibin", op, [a, b])
    pool.append(node)
    return node


def _ieval(m, node, leaf_vals, memo):
    key = id(node)
    if key in memo:
        return memo[key]
    if node.kind == "leaf":
        v = leaf_vals[node.leaf]
    else:
        k = [_ieval(m, c, leaf_vals, memo) for c in node.kids]
        if node.kind == "iun":
            s = int(node.bound)
            v = {"neg": lambda: -k[0], "abs": lambda: m.abs(k[0]),
                 "rshift": lambda: m.right_shift(k[0], s + 3),
                 "lshift": lambda: m.left_shift(k[0], s),
                 "not": lambda: ~k[0]}[node.op]()
        elif node.kind == "idiv":
            d = m.mod(m.abs(k[1]), 13) + 1                 # 1 .. 13
            d = m.where(k[2] > 0, d, -d)
            v = m.floor_divide(k[0], d) if node.op == "floordiv" else m.mod(k[0], d)
        else:
            v = I_BINARY[node.op](m, k[0], k[1])
    memo[key] = v
    return v


@pytest.mark.parametrize("seed", range(24))
def test_random_int32_dag(seed):
    rng = np.random.default_rng(5000 + seed)
    R, C = SHAPES[(seed + 3) % len(SHAPES)]
    leaves = _make_leaves(rng, R, C, np.int32, int(rng.integers(2, 6)))
    root = None
    while root is None or root.kind == "leaf":
        root = _int_tree(rng, leaves, int(rng.integers(2, 5)), [])
    with np.errstate(all="ignore"):
        want = np.asarray(_ieval(np, root, [h for h, _ in leaves], {}))
    assert want.dtype == np.int32
    for fusion in (True, False):
        cp.set_config(fusion=fusion)
        got = _ieval(cp, root, [d for _, d in leaves], {})
        _same(got.get(), want)
