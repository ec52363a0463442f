"""NumPy broadcasting rules (reference: src/macmetalpy/_broadcasting.py:8-76).

Unlike the reference, whose GPU path materialises broadcasts with a
``broadcast_nd`` kernel (ndarray.py:515-545), broadcast operands here are
described by stride-0 views (``broadcast_strides``) that kernels index
directly.
"""
from __future__ import annotations

__all__ = ["broadcast_shapes", "broadcast_strides", "needs_broadcast"]


def broadcast_shapes(*shapes: tuple[int, ...]) -> tuple[int, ...]:
    if not shapes:
        return ()
    ndim = max(len(s) for s in shapes)
    out = []
    for axis in range(-ndim, 0):
        dims = [s[axis] if len(s) >= -axis else 1 for s in shapes]
        non_one = {d for d in dims if d != 1}
        if len(non_one) > 1:
            raise ValueError(f"Shape mismatch: cannot broadcast shapes {shapes}")
        out.append(non_one.pop() if non_one else 1)
    return tuple(out)


def broadcast_strides(shape, target_shape, strides) -> tuple[int, ...]:
    """Element strides of ``shape``/``strides`` viewed as ``target_shape``:
    stretched and prepended dimensions get stride 0."""
    diff = len(target_shape) - len(shape)
    if diff < 0:
        raise ValueError(f"cannot broadcast {shape} to {target_shape}")
    out = [0] * diff
    for size, tsize, st in zip(shape, target_shape[diff:], strides):
        if size == tsize:
            out.append(st if size != 1 else 0)
        elif size == 1:
            out.append(0)
        else:
            raise ValueError(f"Cannot broadcast dimension {size} to {tsize}")
    return tuple(out)


def needs_broadcast(shape1, shape2) -> bool:
    return tuple(shape1) != tuple(shape2)
