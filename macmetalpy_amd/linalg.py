"""``cp.linalg`` namespace: ``matmul`` (reference linalg.py:234-240, which
calls np.linalg.matmul on the CPU) runs on the device.  The reference's
other linalg functions are NumPy-on-CPU wrappers outside the device path and
are not provided."""
from __future__ import annotations

from .linalg_top import matmul  # noqa: F401

__all__ = ["matmul"]


def __getattr__(name):
    raise AttributeError(f"macmetalpy_amd.linalg.{name} is not implemented on the device "
                         "(only matmul is)")
