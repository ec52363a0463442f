"""NumPy ufunc -> device function map for ``ndarray.__array_ufunc__``
(reference ndarray.py:2681-2720 looks names up on the package)."""
from __future__ import annotations

import numpy as np

_TABLE = None


def lookup(ufunc):
    global _TABLE
    if _TABLE is None:
        from . import ufunc_ops
        t = {}
        for name in ufunc_ops.__all__:
            u = getattr(np, name, None)
            if isinstance(u, np.ufunc):
                t[u] = getattr(ufunc_ops, name)
        from .linalg_top import matmul
        t[np.matmul] = matmul
        _TABLE = t
    return _TABLE.get(ufunc)
