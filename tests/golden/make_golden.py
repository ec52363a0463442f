"""Write tests/golden/hot_path_vectors.npz: small input/expected-output
vectors for every hot-path operation, computed by the oracle (the NumPy
restatement of the reference's CPU path, oracle/reference_cpu.py).

The reference's own tests store no fixtures; they compare against NumPy at
run time.  Where they use literal values, those literals are included here
with their source (file:line of grantkl/MacMetalPy v0.1.3):

* tests/test_math_ops.py:446-453 and tests/test_math_ext.py:302-307 --
  mod with negative operands ([-7, 7, -7, 7] % [3, -3, -3, 3]);
* tests/test_untested_math.py:227-232 -- float32 floor_divide with
  negatives ([-7.5, 7.5, -7.5] // [2, -2, -2]);
* tests/test_error_handling.py:107-114 -- 1-D @ 1-D of arange(3) = 5;
* tests/test_edge_shapes.py:367-378 -- sum of 1e6 ones = 1e6.

Run from the repository root: ``python tests/golden/make_golden.py``.
Everything is seeded, so re-running reproduces the file bit for bit (for
the same NumPy version; 2.2.6 wrote the committed one).
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import reference_cpu as ref  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hot_path_vectors.npz")

F32_SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 2.0, 3.0, 1e-3, -1e-3, 100.0, -100.0,
                         1e-30, 1e-40, -1e-40, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan,
                         np.pi, -np.pi, 1e4, 88.0, -88.0, 0.9999, 1.0001],
                        dtype=np.float32)
INT32_EDGE = np.array([0, 1, -1, 7, -7, 1000, -1000, 2**31 - 1, -2**31, 123456789,
                       -123456789, 2**30, -2**30], dtype=np.int32)


def vectors() -> dict[str, np.ndarray]:
    v: dict[str, np.ndarray] = {}
    g = np.random.default_rng(20251201)

    # -- C2b: integer floor_divide / mod: edge pairs (divisor 0 -> 0 as NumPy),
    #    INT_MIN // -1 (wraps), and a random sample of the workload's ranges
    a = np.repeat(INT32_EDGE, INT32_EDGE.size)
    b = np.tile(INT32_EDGE, INT32_EDGE.size)
    rs = g.integers(-2**30, 2**30, 4096, dtype=np.int32)
    rb = (g.integers(1, 1000, 4096, endpoint=True, dtype=np.int32)
          * np.where(g.random(4096) < 0.5, -1, 1).astype(np.int32))
    a = np.concatenate([a, rs]).astype(np.int32)
    b = np.concatenate([b, rb]).astype(np.int32)
    v["floor_divide_i32/a"], v["floor_divide_i32/b"] = a, b
    v["floor_divide_i32/out"] = ref.floor_divide(a, b)
    v["mod_i32/out"] = ref.mod(a, b)

    # reference test literals (tests/test_math_ops.py:446-453, test_math_ext.py:302-307)
    v["lit_mod/a"] = np.array([-7, 7, -7, 7], dtype=np.int32)
    v["lit_mod/b"] = np.array([3, -3, -3, 3], dtype=np.int32)
    v["lit_mod/out"] = np.array([2, -2, -1, 1], dtype=np.int32)
    # tests/test_untested_math.py:227-232
    v["lit_floordiv_f32/a"] = np.array([-7.5, 7.5, -7.5], dtype=np.float32)
    v["lit_floordiv_f32/b"] = np.array([2.0, -2.0, -2.0], dtype=np.float32)
    v["lit_floordiv_f32/out"] = np.array([-4.0, -4.0, 3.0], dtype=np.float32)

    # -- C2a: float32 add and the unary table on special values + a sample
    x = np.concatenate([F32_SPECIALS, g.standard_normal(2048, dtype=np.float32) * 4]).astype(np.float32)
    y = np.concatenate([F32_SPECIALS[::-1], g.standard_normal(2048, dtype=np.float32)]).astype(np.float32)
    v["f32/x"], v["f32/y"] = x, y
    v["add_f32/out"] = ref.binary("add_op", x, y)
    for op in ("sin_op", "exp_op", "log1p_op", "tanh_op", "sqrt_op", "abs_op", "neg_op"):
        v[f"{op}_f32/out"] = ref.unary(op, x)

    # -- C1 / C5 fused expressions on small inputs
    x1 = g.standard_normal(4099, dtype=np.float32)
    v["c1/x"] = x1
    v["c1/out"] = ref.fused_elementwise(x1)
    x5 = g.standard_normal((37, 301), dtype=np.float32)
    r5 = g.uniform(0.5, 2.0, (1, 301)).astype(np.float32)
    v["c5/x"], v["c5/r"] = x5, r5
    v["c5/out_f64"] = ref.fusion_chain_f64(x5, r5)

    # -- C3a: sum / mean / argmax (float64-accumulated expectations)
    m = g.standard_normal((65, 515), dtype=np.float32)
    m[3, 17] = m[3, 400] = 50.0          # tie: first index wins
    m[7, 5] = np.nan                     # NaN row: argmax is the first NaN
    v["c3/m"] = m
    clean = np.where(np.isnan(m), 0.0, m).astype(np.float32)  # the sums use m without its NaN
    v["sum_all/out_f64"] = np.array(ref.sum_f64(clean))
    v["sum_axis1/out_f64"] = ref.sum_f64(clean, axis=1)
    v["mean_axis1/out_f64"] = ref.mean_f64(clean, axis=1)
    v["argmax_axis1/out"] = ref.argmax(m, axis=1).astype(np.int64)
    v["argmax_all/out"] = np.array(ref.argmax(m), dtype=np.int64)
    v["lit_sum_ones/n"] = np.array(1_000_000, dtype=np.int64)   # tests/test_edge_shapes.py:367-378

    # -- C3b: cumsum int32 -> int64 (exact) and float32 (float64 carry)
    ci = g.integers(-100, 100, 20001, endpoint=True, dtype=np.int32)
    cf = g.random(20001, dtype=np.float32)
    v["cumsum_i32/x"], v["cumsum_i32/out"] = ci, ref.cumsum(ci)
    v["cumsum_f32/x"], v["cumsum_f32/out_f64"] = cf, ref.cumsum_f64(cf)

    # -- C4: matmul (float64 products of the rounded inputs)
    for name, dt, (mm, nn, kk) in (("f32", np.float32, (96, 80, 112)),
                                   ("f16", np.float16, (128, 64, 96))):
        A = (g.standard_normal((mm, kk)) / np.sqrt(kk)).astype(dt)
        B = (g.standard_normal((kk, nn)) / np.sqrt(kk)).astype(dt)
        v[f"matmul_{name}/a"], v[f"matmul_{name}/b"] = A, B
        v[f"matmul_{name}/out_f64"] = ref.matmul_f64(A, B)
    # tests/test_error_handling.py:107-114: arange(3) @ arange(3) == 5
    v["lit_inner/x"] = np.arange(3, dtype=np.float32)
    v["lit_inner/out"] = np.array(5.0, dtype=np.float32)
    return v


def main() -> None:
    v = vectors()
    np.savez_compressed(OUT, **v)
    total = sum(a.nbytes for a in v.values())
    print(f"wrote {OUT}: {len(v)} arrays, {total} bytes uncompressed")


if __name__ == "__main__":
    main()
