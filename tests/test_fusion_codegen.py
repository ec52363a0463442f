"""Fusion engine on the CPU: DAG linearisation, dimension collapsing and
generated HIP source compiled by hiprtc for gfx950 (no device needed)."""
import numpy as np
import pytest

from macmetalpy_amd import _fusion as F
from macmetalpy_amd._backend import DeviceBuffer, rtc_build


def _FakeBuf(ptr, nbytes):  # borrowed: never handed to mmp_free
    return DeviceBuffer(ptr, nbytes, owned=False)


def _leaf(shape, dtype=np.float32, strides=None, ptr=0x10000):
    st = strides if strides is not None else F._c_contig_strides(tuple(shape))
    return F.InputNode(_FakeBuf(ptr, 0), shape, dtype, st)


def _compile(root, mode="map", keep_last=False, vec=True):
    prog = F._Program(root)
    cshape, outer, cols, leaf_str, kinds = F._plan(prog, root._shape, keep_last)
    out_dt = root._dtype
    vec = vec and F._vec_ok(prog, kinds, leaf_str, outer, cols, 0x20000, out_dt.itemsize, mode)
    src = F.generate_source(prog, kinds, len(outer), out_dt if mode == "map" else np.dtype(np.float32),
                            vec, mode)
    code = rtc_build(src, F.RTC_OPTIONS)
    assert code[:4] == b"\x7fELF"
    return prog, cshape, kinds, vec, src


def test_c1_expression_compiles_vectorised():
    x = _leaf((1 << 20,))
    sq = F.UnaryOpNode("square_op", x, x._shape, np.float32)
    e = F.UnaryOpNode("exp_op", F.UnaryOpNode("neg_op", sq, x._shape, np.float32), x._shape, np.float32)
    s = F.UnaryOpNode("sqrt_op", F.UnaryOpNode("abs_op", x, x._shape, np.float32), x._shape, np.float32)
    root = F.BinaryOpNode("add_op", s, e, x._shape, np.float32)
    prog, cshape, kinds, vec, src = _compile(root)
    assert len(prog.arrays) == 1  # x loaded once
    assert cshape == [1 << 20] and kinds == ["c"] and vec
    assert "__builtin_nontemporal_load" in src


def test_c5_broadcast_scalar_and_row_sum_compile():
    x = _leaf((64, 128))
    r = _leaf((1, 128), ptr=0x30000)
    one = F.ScalarNode(1.0, np.float32)
    shp = (64, 128)
    xr = F.BinaryOpNode("mul_op", x, r, shp, np.float32)
    t = F.UnaryOpNode("tanh_op", F.BinaryOpNode("add_op", xr, one, shp, np.float32), shp, np.float32)
    e = F.UnaryOpNode("exp_op", F.UnaryOpNode("neg_op", F.UnaryOpNode("abs_op", x, shp, np.float32),
                                                shp, np.float32), shp, np.float32)
    l = F.UnaryOpNode("log1p_op", F.BinaryOpNode("mul_op", x, x, shp, np.float32), shp, np.float32)
    root = F.BinaryOpNode("sub_op", F.BinaryOpNode("mul_op", t, e, shp, np.float32), l, shp, np.float32)
    prog, cshape, kinds, vec, src = _compile(root)
    assert len(prog.arrays) == 2 and len(prog.scalars) == 1
    assert cshape == [64, 128]          # r's stride-0 row prevents collapsing
    _compile(root, mode="sum", keep_last=True, vec=False)


def test_collapse_rules():
    shape, st = F._collapse([4, 5, 6], [[30, 6, 1], [0, 0, 1]])
    assert shape == [4, 5, 6] or shape == [20, 6]
    shape, st = F._collapse([4, 5, 6], [[30, 6, 1], [30, 6, 1]])
    assert shape == [120] and st == [[1], [1]]
    shape, st = F._collapse([4, 1, 6], [[6, 6, 1]], keep_last=True)
    assert shape == [4, 6]
    shape, st = F._collapse([4, 5, 6], [[30, 6, 1]], keep_last=True)
    assert shape == [20, 6]


@pytest.mark.parametrize("dtype", [np.float16, np.float64, np.int32, np.uint16, np.bool_])
def test_dtypes_casts_compares_compile(dtype):
    a = _leaf((33, 7), dtype)
    b = _leaf((7,), np.float32, ptr=0x40000)
    if np.dtype(dtype) == np.bool_:
        root = F.BinaryOpNode("eq_op", a, F.CastNode(b, np.bool_), (33, 7), np.bool_)
    else:
        cast = F.CastNode(a, np.float64)
        root = F.BinaryOpNode("lt_op", cast, F.CastNode(b, np.float64), (33, 7), np.bool_)
    _compile(root)


def test_strided_leaf_disables_vector_path():
    x = _leaf((100, 64), strides=(128, 2))
    root = F.UnaryOpNode("sin_op", x, (100, 64), np.float32)
    prog, cshape, kinds, vec, src = _compile(root)
    assert kinds == ["s"] and not vec


_INT_DTYPES = [np.bool_, np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64]
_ALL_DTYPES = _INT_DTYPES + [np.float16, np.float32, np.float64]


@pytest.mark.parametrize("dtype", _INT_DTYPES)
def test_bitwise_and_shift_ops_compile(dtype):
    shp = (4, 256)
    a = _leaf(shp, dtype)
    b = _leaf(shp, dtype, ptr=0x30000)
    root = F.BinaryOpNode("bit_xor_op", F.BinaryOpNode("bit_and_op", a, b, shp, dtype),
                          F.BinaryOpNode("bit_or_op", a, F.UnaryOpNode("invert_op", b, shp, dtype),
                                         shp, dtype), shp, dtype)
    if dtype is not np.bool_:  # numpy shifts bool as int8
        root = F.BinaryOpNode("rshift_op", F.BinaryOpNode("lshift_op", root, b, shp, dtype), a,
                              shp, dtype)
    prog, cshape, kinds, vec, src = _compile(root)
    assert vec and len(prog.arrays) == 2
    for fn in ("op_bitwise_and", "op_bitwise_or", "op_bitwise_xor", "op_invert"):
        assert fn in src


@pytest.mark.parametrize("dtype", _ALL_DTYPES)
def test_predicates_logical_and_where_compile(dtype):
    shp = (3, 512)
    x = _leaf(shp, dtype)
    y = _leaf((1, 512), dtype, ptr=0x30000)
    bool_ = np.dtype(np.bool_)
    preds = [F.UnaryOpNode(op, x, shp, bool_)
             for op in ("isnan_op", "isinf_op", "isfinite_op", "signbit_op", "logical_not_op")]
    c = preds[0]
    for p in preds[1:]:
        c = F.BinaryOpNode("logical_xor_op", c, p, shp, bool_)
    c = F.BinaryOpNode("logical_or_op", F.BinaryOpNode("logical_and_op", x, y, shp, bool_), c,
                       shp, bool_)
    root = F.WhereNode(c, x, F.ScalarNode(1, dtype), shp, dtype)
    prog, cshape, kinds, vec, src = _compile(root)
    assert kinds == ["c", "c"] and cshape == [3, 512]  # y's rows are stride 0
    assert "? t" in src and "op_isnan" in src


def test_where_cond_cast_and_mixed_leaves():
    shp = (1000,)
    cond = F.CastNode(_leaf(shp, np.float32), np.bool_)
    x = _leaf(shp, np.int64, ptr=0x30000)
    root = F.WhereNode(cond, x, F.ScalarNode(-1, np.int64), shp, np.int64)
    prog, cshape, kinds, vec, src = _compile(root)
    assert len(prog.arrays) == 2 and len(prog.scalars) == 1
    assert "mmp_convert<bool, float>" in src


def test_vectorised_sum_epilogue_compiles():
    shp = (64, 1024)
    x = _leaf(shp, np.float32)
    r = _leaf((1, 1024), np.float32, ptr=0x30000)
    root = F.BinaryOpNode("gt_op", F.BinaryOpNode("mul_op", x, r, shp, np.float32),
                          F.ScalarNode(0.5, np.float32), shp, np.bool_)
    prog, cshape, kinds, vec, src = _compile(root, mode="sum", keep_last=True, vec=True)
    assert vec and "__builtin_nontemporal_load" in src and "& ~3LL" in src
    # an odd row length keeps the scalar loop
    y = _leaf((64, 1023), np.float32)
    prog, cshape, kinds, vec, src = _compile(F.UnaryOpNode("abs_op", y, (64, 1023), np.float32),
                                             mode="sum", keep_last=True, vec=True)
    assert not vec
