"""Lazy fusion engine: expression DAG -> one HIP kernel (hiprtc), cached.

Reference: src/macmetalpy/_fusion.py.  The reference records unary ops (and
binary ops over already-lazy operands) as a DAG of ``InputNode`` /
``UnaryOpNode`` / ``BinaryOpNode`` (:37-71), limits depth to 16 (:24), and
on materialisation emits one MSL ``fused_op`` kernel over same-shape,
same-dtype, contiguous inputs (:297-409), caching the text by topology
(:408-436).  Scalars and broadcasts are materialised into full arrays
before they reach the DAG (ndarray.py:1026, 1062-1065).

This engine keeps the node names, the depth cap and the materialisation
triggers, and goes further:

* every elementwise op is lazy (binary roots too), scalars are ``ScalarNode``
  kernel arguments and broadcast operands are stride-0 views, so
  ``tanh(x*r + 1.0)`` with ``r`` of shape (1, N) reads ``x`` and ``r`` once;
* leaves may be strided views of any supported dtype; casts are nodes;
* a reduction over the last axis (or all axes) can be fused as an epilogue
  (``materialize_reduce``), accumulating in float64 per row;
* a DAG of a single op over contiguous operands runs the precompiled
  kernels of libmmp_hip.so (the reference's single-unary fast path,
  _fusion.py:452-464, generalised to binary and scalar forms);
* generated kernels evaluate the same csrc/mmp_ops.h functions with the same
  flags as the precompiled ones, so fused == unfused bit for bit.

Generated kernels are HBM-bound: each leaf is read once per output element
(a broadcast leaf is re-read from cache) and the output written once.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import numpy as np

from . import _abi
from ._backend import HipBackend
from ._config import get_config
from ._dtypes import ctype_name, dtype_code

__all__ = [
    "FusionNode", "InputNode", "ScalarNode", "UnaryOpNode", "BinaryOpNode", "CastNode",
    "WhereNode", "materialize", "materialize_reduce", "generate_source", "_MAX_DEPTH", "RTC_OPTIONS",
]

_MAX_DEPTH = 16
_MAX_LEAVES = 24
_BLOCK = 256
_UNROLL = 4
_ELEMS = 4  # consecutive elements per thread per unroll step (vector path)


def _map_unroll(kinds) -> int:
    """Unroll steps of a map kernel's workgroup tile (_BLOCK * _ELEMS
    elements each).  An expression with a single contiguous leaf and
    nothing else to read streams best in 1024-element tiles; two or more
    leaves (or a broadcast one) in 4096-element tiles.  Measured on MI355X
    at 2^28 elements (GB/s, two runs; tiles of 1024 / 2048 / 4096 / 8192):
    sqrt(|x|) + exp(-x*x) 6132-6487 / 6331-6400 / 6160-6214 / 5952-6066,
    x >> 3 (int32) 6355-6388 / 5886-5967 / 6001-6067 / 5431-5511, isnan
    6526-6581 / 6500-6518 / 6053-6191 / 6010-6074, clip 6373-6506 /
    6212-6275 / 6005-6033 / 6115-6145; a & b 6190-6203 / 6082-6126 /
    6354-6393 / 5798-5814, a * b + c 5938-5965 / 5998-6004 / 6100-6143 /
    5818-5830, X * r with a broadcast row 5951-6035 / 5854-5904 / 6023-6030
    / 5855-5912.  The native gate applies the same rule (native_gate.cpp,
    map_tile)."""
    return 1 if len(kinds) == 1 and kinds[0] == "c" else _UNROLL


def _map_tile(kinds) -> int:
    return _BLOCK * _ELEMS * _map_unroll(kinds)
# Workgroups of a row-sum launch, split over its rows (a row gets at most
# one per 4096 elements).  Measured on 2^28 float32 reduced whole:
# any(a > 3) / count_nonzero 6.7 TB/s at 1024, 5.9-6.0 at 2048, 5.7 at 512;
# sum(a * b) 6.8-6.9 at all three.
_SUM_BLOCKS = 1024
_SUM_UNROLL = 4     # vector steps per thread unrolled in the row-sum loop

_CSRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc")
# Same numerics flags as the precompiled library (csrc/build.py).
RTC_OPTIONS = ("-O3 -std=c++17 -ffp-contract=off "
               "-Xclang -target-feature -Xclang -packed-fp32-ops")

_ops_header_text: Optional[str] = None


def _ops_header() -> str:
    global _ops_header_text
    if _ops_header_text is None:
        with open(os.path.join(_CSRC, "mmp_ops.h")) as f:
            _ops_header_text = f.read().replace("#pragma once", "")
    return _ops_header_text


# ---------------------------------------------------------------- nodes
class FusionNode:
    __slots__ = ("_shape", "_dtype", "_depth", "_buffers", "_nleaves")


class InputNode(FusionNode):
    """A device-resident array view (buffer, element offset, strides)."""
    __slots__ = ("_buffer", "_offset", "_strides")

    def __init__(self, buffer, shape, dtype, strides, offset=0):
        self._buffer = buffer
        self._shape = tuple(shape)
        self._dtype = np.dtype(dtype)
        self._strides = tuple(strides)
        self._offset = int(offset)
        self._depth = 0
        self._buffers = (buffer,)
        self._nleaves = 1


class ScalarNode(FusionNode):
    """A scalar kernel argument: its value converted to ``dtype`` (NumPy's
    conversion), held as the little-endian bits of that value."""
    __slots__ = ("_bits",)

    def __init__(self, value, dtype):
        self._dtype = np.dtype(dtype)
        raw = np.array(value, dtype=self._dtype).tobytes()
        self._bits = int.from_bytes(raw.ljust(8, b"\0"), "little")
        self._shape = ()
        self._depth = 0
        self._buffers = ()
        self._nleaves = 0

    @property
    def _value(self):
        """The value as a 0-d array of ``dtype``."""
        raw = self._bits.to_bytes(8, "little")[:self._dtype.itemsize]
        return np.frombuffer(raw, dtype=self._dtype).reshape(())


def _merge_buffers(*nodes):
    seen, out = set(), []
    for n in nodes:
        for b in n._buffers:
            if id(b) not in seen:
                seen.add(id(b))
                out.append(b)
    return tuple(out)


class UnaryOpNode(FusionNode):
    __slots__ = ("_op_name", "_input")

    def __init__(self, op_name, input_node, shape, dtype):
        self._op_name = op_name
        self._input = input_node
        self._shape = tuple(shape)
        self._dtype = np.dtype(dtype)
        self._depth = input_node._depth + 1
        self._buffers = input_node._buffers
        self._nleaves = input_node._nleaves


class CastNode(FusionNode):
    __slots__ = ("_input",)

    def __init__(self, input_node, dtype):
        self._input = input_node
        self._shape = input_node._shape
        self._dtype = np.dtype(dtype)
        self._depth = input_node._depth  # free: folded into the consumer
        self._buffers = input_node._buffers
        self._nleaves = input_node._nleaves


class BinaryOpNode(FusionNode):
    __slots__ = ("_op_name", "_lhs", "_rhs")

    def __init__(self, op_name, lhs, rhs, shape, dtype):
        self._op_name = op_name
        self._lhs = lhs
        self._rhs = rhs
        self._shape = tuple(shape)
        self._dtype = np.dtype(dtype)
        self._depth = max(lhs._depth, rhs._depth) + 1
        self._buffers = _merge_buffers(lhs, rhs)
        self._nleaves = lhs._nleaves + rhs._nleaves


class WhereNode(FusionNode):
    """``cond ? x : y`` (reference where_shader, _kernels.py:984-1000);
    ``cond`` is a bool node, ``x`` and ``y`` have the result dtype."""
    __slots__ = ("_cond", "_x", "_y")

    def __init__(self, cond, x, y, shape, dtype):
        self._cond = cond
        self._x = x
        self._y = y
        self._shape = tuple(shape)
        self._dtype = np.dtype(dtype)
        self._depth = max(cond._depth, x._depth, y._depth) + 1
        self._buffers = _merge_buffers(cond, x, y)
        self._nleaves = cond._nleaves + x._nleaves + y._nleaves


# ---------------------------------------------------------- DAG analysis
def _c_contig_strides(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc *= s
    return tuple(reversed(st))


def _bcast_strides(shape, strides, target):
    diff = len(target) - len(shape)
    out = [0] * diff
    for s, st, t in zip(shape, strides, target[diff:]):
        out.append(st if (s == t and s != 1) else 0)
    return out


class _Program:
    """Post-order linearisation of a DAG with deduplicated leaves."""

    def __init__(self, root):
        self.root = root
        self.arrays = []      # InputNode leaves (unique views)
        self.scalars = []     # ScalarNode leaves
        self.steps = []       # (kind, payload...) per SSA value
        self.dtypes = []      # dtype per SSA value
        self._memo = {}
        self._leaf_index = {}
        self.result = self._visit(root)

    def _visit(self, node):
        nid = id(node)
        idx = self._memo.get(nid)
        if idx is not None:
            return idx
        cls = type(node)
        if cls is InputNode:
            key = (id(node._buffer), node._offset, node._strides, node._shape, node._dtype)
            k = self._leaf_index.get(key)
            if k is None:
                k = len(self.arrays)
                self._leaf_index[key] = k
                self.arrays.append(node)
            step = ("load", k)
        elif cls is UnaryOpNode:
            step = ("unary", node._op_name, self._visit(node._input))
        elif cls is BinaryOpNode:
            step = ("binary", node._op_name, self._visit(node._lhs), self._visit(node._rhs))
        elif cls is ScalarNode:
            step = ("scalar", len(self.scalars))
            self.scalars.append(node)
        elif cls is CastNode:
            step = ("cast", self._visit(node._input))
        elif cls is WhereNode:
            step = ("where", self._visit(node._cond), self._visit(node._x),
                    self._visit(node._y))
        else:
            raise TypeError(f"unknown fusion node {cls.__name__}")
        self.steps.append(step)
        self.dtypes.append(node._dtype)
        idx = len(self.steps) - 1
        self._memo[nid] = idx
        return idx


def _collapse(shape, stride_lists, keep_last=False):
    """Merge adjacent dims contiguous for every operand; drop size-1 dims.
    Returns (shape, [strides per operand]).  With keep_last, the last dim
    is never merged with the dims before it."""
    n = len(shape)
    cshape, cstr = [], [[] for _ in stride_lists]
    for d in range(n):
        is_last = keep_last and d == n - 1
        if shape[d] == 1 and not is_last:
            continue
        mergeable = bool(cshape) and not is_last and all(
            sl[-1] == st[d] * shape[d] for sl, st in zip(cstr, stride_lists))
        if mergeable:
            cshape[-1] *= shape[d]
            for sl, st in zip(cstr, stride_lists):
                sl[-1] = st[d]
        else:
            cshape.append(shape[d])
            for sl, st in zip(cstr, stride_lists):
                sl.append(st[d])
    return cshape, cstr


# --------------------------------------------------------------- codegen
_ARG_FIELDS_CACHE: dict = {}


def _param_struct(n_in, n_sc, n_outer):
    key = (n_in, n_sc, n_outer)
    cls = _ARG_FIELDS_CACHE.get(key)
    if cls is None:
        fields = [
            ("ptr", ctypes.c_uint64 * max(1, n_in)),
            ("outp", ctypes.c_uint64),
            ("sbits", ctypes.c_uint64 * max(1, n_sc)),
            ("n", ctypes.c_int64),
            ("rows", ctypes.c_int64),
            ("cols", ctypes.c_int64),
            ("colblocks", ctypes.c_int64),
            ("oshape", ctypes.c_int64 * max(1, n_outer)),
            ("ostride", ctypes.c_int64 * max(1, n_in * n_outer)),
            ("lstride", ctypes.c_int64 * max(1, n_in)),
            ("scale", ctypes.c_double),
        ]
        cls = type(f"FusedParams_{n_in}_{n_sc}_{n_outer}", (ctypes.Structure,),
                   {"_fields_": fields})
        _ARG_FIELDS_CACHE[key] = cls
    return cls


_STRUCT_DECL = """
struct P {{
  unsigned long long ptr[{nin}];
  unsigned long long outp;
  unsigned long long sbits[{nsc}];
  long long n, rows, cols, colblocks;
  long long oshape[{nout}];
  long long ostride[{nio}];
  long long lstride[{nin}];
  double scale;
}};
"""

_BITS_T = {1: "unsigned char", 2: "unsigned short", 4: "unsigned int", 8: "unsigned long long"}


def _acc_type(dtype):
    """Accumulator of a fused sum: float64, uint64 for unsigned inputs,
    else int64 (NumPy sums bool and signed integers as int64)."""
    if dtype.kind == "f":
        return "double", np.dtype(np.float64)
    if dtype.kind == "u":
        return "mmp_u64", np.dtype(np.uint64)
    return "mmp_i64", np.dtype(np.int64)


_FAST_DTYPES = (np.dtype(np.float32), np.dtype(np.float16))


def _op_fn(table, op_name, dtype, fast):
    """mmp_ops.h function for ``op_name`` computing in ``dtype``; the
    ``_fast`` form under fast_math for float32 / float16."""
    fn = table[op_name]
    if fast and op_name in _abi.FAST_MATH_OPS and dtype in _FAST_DTYPES:
        return fn + "_fast"
    return fn


_NONNEG_UNARY = frozenset(("abs_op", "absolute_op", "fabs_op", "square_op", "sqrt_op", "exp_op",
                           "exp2_op", "cosh_op"))


def _sign_facts(prog: _Program):
    """Per SSA value, (never below zero, never above zero) as far as the
    expression shows it, NaN aside: |x|, x*x, exp(...) are >= 0, their
    negations <= 0, products and sums of known signs follow (scalar leaves
    count as unknown: kernels are cached by structure, and a scalar's value
    is a launch parameter).  Lets the
    code generator call the forms of exp and log1p without the cases their
    argument cannot reach (bit for bit the same results)."""
    facts, canon = [], []
    for i, step in enumerate(prog.steps):
        kind, f = step[0], (False, False)
        canon.append(("load", step[1]) if kind == "load" else i)
        if prog.dtypes[i].kind != "f":
            facts.append(f)
            continue
        if kind == "cast":
            f = facts[step[1]] if prog.dtypes[step[1]].kind == "f" else f
        elif kind == "unary":
            a = facts[step[2]]
            if step[1] in _NONNEG_UNARY:
                f = (True, False)
            elif step[1] in ("neg_op", "negative_op"):
                f = (a[1], a[0])
        elif kind == "where":
            a, b = facts[step[2]], facts[step[3]]
            f = (a[0] and b[0], a[1] and b[1])
        elif kind == "binary":
            op, a, b = step[1], facts[step[2]], facts[step[3]]
            if op == "mul_op":
                if canon[step[2]] == canon[step[3]]:
                    f = (True, False)
                else:
                    f = ((a[0] and b[0]) or (a[1] and b[1]), (a[0] and b[1]) or (a[1] and b[0]))
            elif op == "add_op":
                f = (a[0] and b[0], a[1] and b[1])
            elif op == "sub_op":
                f = (a[0] and b[1], a[1] and b[0])
        facts.append(f)
    return facts


def generate_source(prog: _Program, kinds, nouter, out_dtype, vec, mode, fast=False):
    """HIP source for ``prog``.

    kinds[k]: last-dim stride class of array leaf k ('c' unit, 'b' zero,
    's' general).  nouter: number of outer (row) dims (0 = 1-D launch).
    mode: 'map' (elementwise, contiguous output), 'sum' (row-sum epilogue).
    fast: use the fast_math forms of the transcendentals.
    """
    nin, nsc = len(prog.arrays), len(prog.scalars)
    L = []
    L.append(_ops_header())
    L.append(_STRUCT_DECL.format(nin=max(1, nin), nsc=max(1, nsc), nout=max(1, nouter),
                                 nio=max(1, nin * nouter)))
    ct = [ctype_name(a._dtype) for a in prog.arrays]
    out_ct = ctype_name(out_dtype)
    if mode == "sum":
        acc_ct, _ = _acc_type(prog.dtypes[prog.result])
    # vector types for the vectorised path
    vtypes = {}
    if vec:
        for t in set(ct + ([out_ct] if mode == "map" else [])):
            vt = "v4_" + t.replace(" ", "_")
            st = "unsigned char" if t == "bool" else t
            vtypes[t] = vt
            L.append(f"typedef {st} {vt} __attribute__((ext_vector_type(4)));")

    signs = _sign_facts(prog)

    def expr_lines(load_expr, indent):
        """Statements computing every SSA value; load_expr(k) -> leaf k."""
        out = []
        for i, step in enumerate(prog.steps):
            t = ctype_name(prog.dtypes[i])
            kind = step[0]
            if kind == "load":
                rhs = load_expr(step[1])
            elif kind == "scalar":
                rhs = f"s{step[1]}"
            elif kind == "cast":
                src_t = ctype_name(prog.dtypes[step[1]])
                rhs = f"mmp_convert<{t}, {src_t}>(t{step[1]})"
            elif kind == "unary":
                fn = _op_fn(_abi.UNARY_FN, step[1], prog.dtypes[i], fast)
                if fn == "op_exp" and signs[step[2]][1]:
                    fn = "op_exp_nonpos"
                elif fn == "op_log1p" and signs[step[2]][0]:
                    fn = "op_log1p_nonneg"
                rhs = f"{fn}(t{step[2]})"
            elif kind == "where":
                rhs = f"(t{step[1]} ? t{step[2]} : t{step[3]})"
            elif step[1] in _abi.COMPARE_OPS:
                rhs = f"(t{step[2]} {_abi.COMPARE_OPS[step[1]][1]} t{step[3]})"
            else:
                rhs = f"{_op_fn(_abi.BINARY_FN, step[1], prog.dtypes[i], fast)}(t{step[2]}, t{step[3]})"
            out.append(f"{indent}const {t} t{i} = {rhs};")
        return out

    L.append(f'extern "C" __global__ __launch_bounds__({_BLOCK}) void fused_op(P p) {{')
    for k in range(nin):
        L.append(f"  const {ct[k]}* __restrict__ in{k} = (const {ct[k]}*)p.ptr[{k}];")
    for j, sc in enumerate(prog.scalars):
        t = ctype_name(sc._dtype)
        bt = _BITS_T[sc._dtype.itemsize]
        if t == "bool":
            L.append(f"  const bool s{j} = (p.sbits[{j}] & 1ull) != 0;")
        else:
            L.append(f"  const {t} s{j} = __builtin_bit_cast({t}, ({bt})p.sbits[{j}]);")
    # row setup
    if nouter == 0:
        L.append("  const long long row = 0; const long long cb = blockIdx.x;")
        for k in range(nin):
            L.append(f"  const long long ro{k} = 0;")
    else:
        # workgroup ids, colblocks and the outer extents are below 2^31
        # (HIP's grid limit), so the index splits divide in 32 bits: a
        # 64-bit division is ~130 scalar instructions per wave
        L.append("  const unsigned cbk = (unsigned)p.colblocks;")
        L.append("  const unsigned rowu = blockIdx.x / cbk;")
        L.append("  const long long row = rowu;")
        L.append("  const long long cb = blockIdx.x - rowu * cbk;")
        for k in range(nin):
            L.append(f"  long long ro{k} = 0;")
        L.append("  { unsigned r = rowu;")
        for d in range(nouter - 1, -1, -1):
            L.append(f"    {{ const unsigned q = r / (unsigned)p.oshape[{d}]; "
                     f"const long long ix = r - q * (unsigned)p.oshape[{d}];")
            for k in range(nin):
                L.append(f"      ro{k} += ix * p.ostride[{k * nouter + d}];")
            L.append("      r = q; }")
        L.append("  }")
    L.append("  const long long cols = p.cols;")
    tile = _map_tile(kinds)
    unroll = _map_unroll(kinds)

    def scalar_load(k, col):
        if kinds[k] == "c":
            return f"in{k}[ro{k} + {col}]"
        if kinds[k] == "b":
            return f"in{k}[ro{k}]"
        return f"in{k}[ro{k} + {col} * p.lstride[{k}]]"

    res = f"t{prog.result}"
    if mode == "map":
        L.append("  const long long obase = row * cols;")
        L.append(f"  const long long c0 = cb * {tile}LL;")
        L.append(f"  const long long c1 = c0 + {tile}LL < cols ? c0 + {tile}LL : cols;")
        if vec:
            L.append(f"  if (c0 + {tile}LL <= cols) {{")
            for k in range(nin):
                if kinds[k] == "c":
                    L.append(f"    {vtypes[ct[k]]} l{k}[{unroll}];")
            L.append(f"    #pragma unroll\n    for (int u = 0; u < {unroll}; ++u) {{")
            L.append(f"      const long long c = c0 + ((long long)u * {_BLOCK} + threadIdx.x) * {_ELEMS};")
            for k in range(nin):
                if kinds[k] == "c":
                    L.append(f"      l{k}[u] = __builtin_nontemporal_load((const {vtypes[ct[k]]}*)(in{k} + ro{k} + c));")
            L.append("    }")
            for k in range(nin):
                if kinds[k] == "b":
                    L.append(f"    const {ct[k]} bc{k} = in{k}[ro{k}];")
            L.append(f"    #pragma unroll\n    for (int u = 0; u < {unroll}; ++u) {{")
            L.append(f"      const long long c = c0 + ((long long)u * {_BLOCK} + threadIdx.x) * {_ELEMS};")
            L.append(f"      {vtypes[out_ct]} r;")
            L.append(f"      #pragma unroll\n      for (int e = 0; e < {_ELEMS}; ++e) {{")

            def vload(k):
                if kinds[k] == "c":
                    return f"({ct[k]})l{k}[u][e]"
                return f"bc{k}"
            L.extend(expr_lines(vload, "        "))
            L.append(f"        r[e] = {res};")
            L.append("      }")
            L.append(f"      __builtin_nontemporal_store(r, ({vtypes[out_ct]}*)(({out_ct}*)p.outp + obase + c));")
            L.append("    }")
            L.append("    return;")
            L.append("  }")
        L.append(f"  for (long long c = c0 + threadIdx.x; c < c1; c += {_BLOCK}) {{")
        L.extend(expr_lines(lambda k: scalar_load(k, "c"), "    "))
        L.append(f"    (({out_ct}*)p.outp)[obase + c] = {res};")
        L.append("  }")
        L.append("}")
    else:  # row-sum epilogue
        L.append(f"  {acc_ct} acc = 0;")
        L.append("  const unsigned cbk_ = (unsigned)p.colblocks;")
        if vec:
            # column ranges are multiples of 4 elements, so every 16-byte
            # (or narrower) vector load of a contiguous leaf is aligned
            L.append("  const long long span = cols + p.colblocks - 1;")
            L.append("  const long long per = ((span < 0x100000000LL ? (long long)((unsigned)span / cbk_) "
                     ": span / p.colblocks) + 3) & ~3LL;")
        else:
            L.append("  const long long span = cols + p.colblocks - 1;")
            L.append("  const long long per = span < 0x100000000LL ? (long long)((unsigned)span / cbk_) "
                     ": span / p.colblocks;")
        L.append("  const long long c0 = cb * per;")
        L.append("  const long long c1 = c0 + per < cols ? c0 + per : cols;")
        if vec:
            for k in range(nin):
                if kinds[k] == "b":
                    L.append(f"  const {ct[k]} bc{k} = in{k}[ro{k}];")
            L.append(f"  #pragma unroll {_SUM_UNROLL}")
            L.append(f"  for (long long c = c0 + threadIdx.x * {_ELEMS}; c < c1; "
                     f"c += {_BLOCK * _ELEMS}) {{")
            for k in range(nin):
                if kinds[k] == "c":
                    L.append(f"    const {vtypes[ct[k]]} l{k} = __builtin_nontemporal_load("
                             f"(const {vtypes[ct[k]]}*)(in{k} + ro{k} + c));")
            L.append(f"    #pragma unroll\n    for (int e = 0; e < {_ELEMS}; ++e) {{")

            def vload_sum(k):
                if kinds[k] == "c":
                    return f"({ct[k]})l{k}[e]"
                return f"bc{k}"
            L.extend(expr_lines(vload_sum, "      "))
            L.append(f"      acc += ({acc_ct}){res};")
            L.append("    }")
            L.append("  }")
        else:
            L.append(f"  for (long long c = c0 + threadIdx.x; c < c1; c += {_BLOCK}) {{")
            L.extend(expr_lines(lambda k: scalar_load(k, "c"), "    "))
            L.append(f"    acc += ({acc_ct}){res};")
            L.append("  }")
        L.append("  // wave64 butterfly, then one value per wave through LDS")
        L.append("  #pragma unroll\n  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);")
        L.append(f"  __shared__ {acc_ct} red[{_BLOCK // 64}];")
        L.append("  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;")
        L.append("  __syncthreads();")
        L.append("  if (threadIdx.x == 0) {")
        L.append(f"    {acc_ct} s = red[0];")
        L.append(f"    for (int w = 1; w < {_BLOCK // 64}; ++w) s += red[w];")
        L.append("    if (p.colblocks == 1) {")
        if _acc_type(prog.dtypes[prog.result])[0] == "double":
            L.append(f"      (({out_ct}*)p.outp)[row] = mmp_convert<{out_ct}, double>(s * p.scale);")
            L.append("    } else {")
            L.append("      ((double*)p.outp)[row * p.colblocks + cb] = s * p.scale;")
        else:
            L.append(f"      (({out_ct}*)p.outp)[row] = mmp_convert<{out_ct}, {acc_ct}>(s);")
            L.append("    } else {")
            L.append(f"      (({acc_ct}*)p.outp)[row * p.colblocks + cb] = s;")
        L.append("    }")
        L.append("  }")
        L.append("}")
    return "\n".join(L) + "\n"


# ------------------------------------------------------------ execution
_kernel_cache: dict = {}
_cache_lock = threading.Lock()


def clear_kernel_caches() -> None:
    """Forget every compiled-kernel handle (by source and by structure)."""
    with _cache_lock:
        _kernel_cache.clear()
        _struct_cache.clear()


def _kernel_for(src: str) -> int:
    k = _kernel_cache.get(src)
    if k is None:
        k = HipBackend().compile(src, "fused_op", RTC_OPTIONS)
        with _cache_lock:
            _kernel_cache[src] = k
    return k


# Kernels by program structure: the generated source is a function of the
# SSA steps (op names and operand indices), the value dtypes, the leaves'
# dtypes and stride classes, the number of outer dimensions, the output
# dtype, the vector flag and the mode -- so a repeated expression skips
# source generation (about 30 us of Python per call) as well as compilation.
_struct_cache: dict = {}


def _kernel_for_program(prog, kinds, nouter, out_dtype, vec, mode) -> int:
    fast = get_config().fast_math
    key = (tuple(prog.steps), tuple(prog.dtypes), tuple(a._dtype for a in prog.arrays),
           tuple(kinds), nouter, out_dtype, vec, mode, fast)
    k = _struct_cache.get(key)
    if k is None:
        k = _kernel_for(generate_source(prog, kinds, nouter, out_dtype, vec, mode, fast))
        with _cache_lock:
            _struct_cache[key] = k
    return k


def _leaf_ptr(node: InputNode) -> int:
    return node._buffer.ptr + node._offset * node._dtype.itemsize


def _scalar_bits(sc: ScalarNode) -> int:
    return sc._bits


def _plan(prog: _Program, shape, keep_last):
    """Collapse the iteration space and classify leaves."""
    strides = [_bcast_strides(a._shape, a._strides, shape) for a in prog.arrays]
    out_st = list(_c_contig_strides(shape))
    cshape, cstr = _collapse(list(shape), strides + [out_st], keep_last=keep_last)
    leaf_str = cstr[:-1]
    if not cshape:
        cshape = [1]
        leaf_str = [[0] for _ in leaf_str]
    cols = cshape[-1]
    outer = cshape[:-1]
    kinds = []
    for st in leaf_str:
        ls = st[-1] if st else 0
        kinds.append("c" if ls == 1 else ("b" if ls == 0 else "s"))
    return cshape, outer, cols, leaf_str, kinds


def _fill_params(prog, P, outer, cols, leaf_str, out_ptr, colblocks, scale):
    nin, nouter = len(prog.arrays), len(outer)
    p = P()
    for k, a in enumerate(prog.arrays):
        p.ptr[k] = _leaf_ptr(a)
        p.lstride[k] = leaf_str[k][-1] if leaf_str[k] else 0
        for d in range(nouter):
            p.ostride[k * nouter + d] = leaf_str[k][d]
    for j, sc in enumerate(prog.scalars):
        p.sbits[j] = _scalar_bits(sc)
    rows = 1
    for d, s in enumerate(outer):
        p.oshape[d] = s
        rows *= s
    p.outp = out_ptr
    p.rows = rows
    p.cols = cols
    p.n = rows * cols
    p.colblocks = colblocks
    p.scale = scale
    return p, rows


def _vec_ok(prog, kinds, leaf_str, outer, cols, out_ptr, out_itemsize, mode):
    """Whether every leaf can be read (and, for 'map', the output written)
    4 elements at a time with aligned vector accesses."""
    if cols % _ELEMS:
        return False
    if mode == "map" and out_ptr % (_ELEMS * out_itemsize):
        return False
    for k, a in enumerate(prog.arrays):
        if kinds[k] == "s":
            return False
        if kinds[k] == "c":
            align = _ELEMS * a._dtype.itemsize
            if _leaf_ptr(a) % align:
                return False
            if any(st % _ELEMS for st in leaf_str[k][:-1]):
                return False
    return True


def _check_grid(nblocks: int) -> None:
    """HIP counts at most 2^32 - 1 work-items per grid dimension; the
    generated kernels also split workgroup ids in 32-bit arithmetic."""
    if nblocks * _BLOCK > 0xFFFFFFFF:
        raise ValueError("fused launch too large")


def run_map(root: FusionNode, out_buffer, out_ptr: int) -> None:
    """Evaluate ``root`` into the C-contiguous output at ``out_ptr``."""
    prog = _Program(root)
    shape = root._shape
    cshape, outer, cols, leaf_str, kinds = _plan(prog, shape, keep_last=False)
    out_dtype = root._dtype
    vec = _vec_ok(prog, kinds, leaf_str, outer, cols, out_ptr, out_dtype.itemsize, "map")
    kern = _kernel_for_program(prog, kinds, len(outer), out_dtype, vec, "map")
    tile = _map_tile(kinds)
    colblocks = -(-cols // tile)
    P = _param_struct(len(prog.arrays), len(prog.scalars), len(outer))
    p, rows = _fill_params(prog, P, outer, cols, leaf_str, out_ptr, colblocks, 1.0)
    nblocks = rows * colblocks
    if nblocks == 0:
        return
    _check_grid(nblocks)
    HipBackend().launch(kern, (nblocks, 1, 1), (_BLOCK, 1, 1), [p])


def _run_sum_py(root: FusionNode, axis_last: bool, out_dtype, out_ptr: int, mean: bool):
    """Fused reduction epilogue: sum (or mean) of ``root`` over its last axis
    (axis_last=True) or over all elements, written to ``out_ptr``."""
    from ._backend import HipBackend as _HB
    be = _HB()
    prog = _Program(root)
    shape = tuple(root._shape)
    if not axis_last:
        # reduce everything: rows are the collapsed outer dims, then the
        # per-row partials are summed by the precompiled reduction.
        cshape, outer, cols, leaf_str, kinds = _plan(prog, shape, keep_last=False)
    else:
        cshape, outer, cols, leaf_str, kinds = _plan(prog, shape, keep_last=True)
    rows = 1
    for s in outer:
        rows *= s
    count = cols if axis_last else max(1, int(np.prod(shape)) if shape else 1)
    scale = (1.0 / count) if mean else 1.0
    acc_ct, acc_dt = _acc_type(root._dtype)
    # enough blocks to fill 256 CUs; at least 4K elements per block
    want = max(1, _SUM_BLOCKS // max(1, rows))
    colblocks = max(1, min(want, -(-cols // 4096)))
    final_direct = axis_last and colblocks == 1
    P = _param_struct(len(prog.arrays), len(prog.scalars), len(outer))
    vec = _vec_ok(prog, kinds, leaf_str, outer, cols, 0, 0, "sum")
    kern = _kernel_for_program(prog, kinds, len(outer), out_dtype if final_direct else acc_dt,
                               vec, "sum")
    if final_direct:
        p, rows = _fill_params(prog, P, outer, cols, leaf_str, out_ptr, 1, scale)
        _check_grid(rows)
        be.launch(kern, (rows, 1, 1), (_BLOCK, 1, 1), [p])
        return None
    _check_grid(rows * colblocks)
    part = be.create_buffer(rows * colblocks, acc_dt)
    p, rows = _fill_params(prog, P, outer, cols, leaf_str, part.ptr, colblocks, scale)
    be.launch(kern, (rows * colblocks, 1, 1), (_BLOCK, 1, 1), [p])
    outer_n, length = (rows, colblocks) if axis_last else (1, rows * colblocks)
    be.reduce(_abi.REDUCE_SUM, dtype_code(acc_dt), dtype_code(out_dtype), outer_n, length, 1,
              part.ptr, out_ptr)
    return part  # keep alive until the stream passes it (pool is stream-ordered)


def is_precompiled_unary(node) -> bool:
    return (isinstance(node, UnaryOpNode) and _abi.precompiled_unary_ok(node._op_name, node._dtype)
            and isinstance(node._input, InputNode)
            and node._input._dtype == node._dtype
            and node._input._shape == node._shape
            and node._input._strides == _c_contig_strides(node._shape))


def _contig_leaf(n, shape, dtype):
    return (isinstance(n, InputNode) and n._dtype == dtype and n._shape == tuple(shape)
            and n._strides == _c_contig_strides(shape))


def materialize_node(node: FusionNode, out_ptr: int) -> None:
    """Compute ``node`` into the contiguous output at ``out_ptr``."""
    be = HipBackend()
    n = 1
    for s in node._shape:
        n *= s
    if n == 0:
        return
    if (get_config().fast_math and getattr(node, "_op_name", None) in _abi.FAST_MATH_OPS
            and node._dtype in _FAST_DTYPES):
        run_map(node, None, out_ptr)  # the generated kernel carries the fast form
        return
    if is_precompiled_unary(node):
        code = _abi.UNARY_OPS[node._op_name][0]
        be.unary(code, dtype_code(node._dtype), n, _leaf_ptr(node._input), out_ptr)
        return
    if isinstance(node, BinaryOpNode) and node._op_name in _abi.BINARY_OPS:
        a, b = node._lhs, node._rhs
        code = _abi.BINARY_OPS[node._op_name][0]
        dc = dtype_code(node._dtype)
        if _contig_leaf(a, node._shape, node._dtype) and _contig_leaf(b, node._shape, node._dtype):
            be.binary(code, dc, n, _leaf_ptr(a), _leaf_ptr(b), out_ptr)
            return
        if (_contig_leaf(a, node._shape, node._dtype) and isinstance(b, ScalarNode)
                and b._dtype == node._dtype):
            be.binary_scalar(code, dc, n, _leaf_ptr(a), b._value, 1, out_ptr)
            return
        if (isinstance(a, ScalarNode) and a._dtype == node._dtype
                and _contig_leaf(b, node._shape, node._dtype)):
            be.binary_scalar(code, dc, n, _leaf_ptr(b), a._value, 0, out_ptr)
            return
    if isinstance(node, CastNode) and isinstance(node._input, InputNode):
        src = node._input
        be.copy(dtype_code(src._dtype), dtype_code(node._dtype), src._shape, _leaf_ptr(src),
                src._strides, out_ptr)
        return
    run_map(node, None, out_ptr)


def compile_for_native(root, kinds, nouter, out_dtype, vec, mode="map") -> int:
    """Kernel handle of the generated kernel for ``root`` ('map' or 'sum'
    mode) with the iteration plan the native gate computed (leaf stride
    classes ``kinds``, ``nouter`` outer dims, output dtype, vector flag);
    the DAG is linearised here in the same order as there."""
    prog = _Program(root)
    return _kernel_for_program(prog, list(kinds), nouter, np.dtype(out_dtype), bool(vec), mode)


def _materialize_py(arr) -> None:
    """Evaluate a lazy ndarray in place (reference: _fusion.py:443-486):
    afterwards ``arr._buffer`` holds the result and ``arr._fusion_node`` is
    None.  The native gate (``_native.materialize``, bound to
    ``materialize`` by the package) handles the common cases and calls this
    for the rest."""
    node = arr._fusion_node
    if node is None:
        return
    be = HipBackend()
    buf = be.create_buffer(arr.size, arr._dtype)
    materialize_node(node, buf.ptr)
    arr._buffer = buf
    arr._fusion_node = None
    arr._np_data = None
    arr._offset = 0
    arr._strides = _c_contig_strides(arr._shape)


# Replaced by the native gate's versions when the package is set up.
materialize = _materialize_py
run_sum = _run_sum_py
