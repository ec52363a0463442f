"""ORACLE -- test infrastructure only, never part of the product.

A CPU restatement of what the reference (grantkl/MacMetalPy v0.1.3)
computes on its CPU/NumPy fallback path for the array-compute hot path.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or, in bench.py, as
the timed CPU baseline) -- the device path in ``macmetalpy_amd`` never calls
it and fails loudly without its HIP library.

Modules
-------
reference_cpu   NumPy restatement of the reference's fallback tables
                (src/macmetalpy/ndarray.py:74-111, math_ops.py:540-548,
                reductions.py:74-163, 381-418, 661-681, linalg_top.py:94-111)
                plus float64-accumulated references for tolerance checks.
c_oracle        ctypes loader of ``oracle/c/oracle.c``: an independent C
                restatement of the integer ops (NumPy floor division and
                remainder, int32 -> int64 cumsum, argmax with the first-NaN
                rule) used to pin the NumPy restatement.

Pinning (tests/test_oracle.py): every function is checked against
mathematics the reference's own tests rely on -- the division identity and
remainder sign rules with brute force over all small pairs, hand-derived
answers for the literal inputs of the reference's tests
(tests/test_math_ops.py:446-453, test_untested_math.py:227-232,
test_math_ext.py:302-307, test_ndarray_gaps.py:659-681,
test_edge_shapes.py:367-378, test_error_handling.py:107-114), closed forms
(sums and prefix sums of ones / aranges, identity matmuls), ULP bounds of
float32 transcendentals against float64 evaluation, and the C restatement.
No function is left "parity unpinned".
"""
