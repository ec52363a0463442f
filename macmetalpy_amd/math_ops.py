"""Module-level math names of the reference (src/macmetalpy/math_ops.py).

The elementwise functions live in ``ufunc_ops``; this module re-exports the
names the reference defines here (sqrt, exp, log, abs, power, sin, tanh,
square, negative, mod, ...) plus ``dot``.
"""
from __future__ import annotations

from .linalg_top import dot  # noqa: F401
from .ufunc_ops import (  # noqa: F401
    abs, arccos, arcsin, arctan, ceil, cos, cosh, exp, floor, log, log2, log10, mod,
    negative, power, remainder, sign, sin, sinh, sqrt, square, tan, tanh,
)
