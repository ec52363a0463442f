"""Fusion engine on the CPU: DAG linearisation, dimension collapsing and
generated HIP source compiled by hiprtc for gfx950 (no device needed)."""
import numpy as np
import pytest

from macmetalpy_amd import _fusion as F
from macmetalpy_amd._backend import DeviceBuffer, rtc_build


class _FakeBuf(DeviceBuffer):
    def __del__(self):
        pass


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
