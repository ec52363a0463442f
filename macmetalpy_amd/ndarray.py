"""Device-resident N-dimensional array for the MI355X.

Reference: src/macmetalpy/ndarray.py (class ``ndarray`` :236-2783).  The
state model is the reference's (:245-368):

* ``_np_data``  -- host-resident NumPy storage (creation / random results
  stay on the host until a device op needs them; ``_ensure_gpu`` uploads);
* ``_buffer``   -- a ``DeviceBuffer`` in HBM, viewed through ``_shape``,
  ``_strides`` (in elements), ``_offset`` (in elements) and ``_dtype``;
* ``_fusion_node`` -- a pending expression DAG (lazy result).

Differences, all deliberate: no size thresholds send work to NumPy; views
of lazy arrays evaluate them first (the reference's ``transpose``/``ravel``
drop the DAG, ndarray.py:661-722); ``get()`` is a device-to-host copy (HBM
is not unified memory); ``@`` follows NumPy for N-D operands (batched)
instead of raising for 3-D (ndarray.py:1422-1423).
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

from . import _abi
from . import _elementwise as ew
from . import _fusion as _fusion_mod
from ._backend import HipBackend
from ._dtypes import dtype_code, resolve_dtype

__all__ = ["ndarray", "_wrap_np", "_c_contiguous_strides"]

_STRIDE_CACHE: dict = {}


def _c_contiguous_strides(shape: Tuple[int, ...]) -> Tuple[int, ...]:
    """C-contiguous element strides (reference ndarray.py:215-232)."""
    s = _STRIDE_CACHE.get(shape)
    if s is not None:
        return s
    st, acc = [], 1
    for d in reversed(shape):
        st.append(acc)
        acc *= d
    res = tuple(reversed(st))
    if len(_STRIDE_CACHE) < 512:
        _STRIDE_CACHE[shape] = res
    return res


def _prod(shape) -> int:
    p = 1
    for s in shape:
        p *= s
    return p


def _normalize_axis(axis: int, ndim: int) -> int:
    if not -ndim <= axis < max(ndim, 1):
        raise np.exceptions.AxisError(axis, ndim)
    return axis % ndim if ndim else 0


class ndarray:
    """MI355X array with the reference's ``cp.ndarray`` interface."""

    _fusion_node = None
    __array_priority__ = 100

    # ------------------------------------------------------------ init
    def __init__(self, buffer, shape, dtype, strides=None, offset=0, base=None):
        self._buffer = buffer
        self._np_data: Optional[np.ndarray] = None
        self._shape = tuple(int(s) for s in shape)
        self._dtype = np.dtype(dtype)
        self._strides = tuple(strides) if strides is not None else _c_contiguous_strides(self._shape)
        self._offset = int(offset)
        self._base = base

    @classmethod
    def _from_buffer(cls, buffer, shape, dtype, strides=None, offset=0, base=None) -> "ndarray":
        return cls(buffer, shape, dtype, strides=strides, offset=offset, base=base)

    @classmethod
    def _from_np_direct(cls, np_array) -> "ndarray":
        """Host-resident array (reference ndarray.py:284-331).  The dtype is
        resolved by the device policy (int8 -> int16, float64 per config)."""
        if type(np_array) is not np.ndarray:
            np_array = np.asarray(np_array)
        target = resolve_dtype(np_array.dtype)
        if np_array.dtype != target:
            np_array = np_array.astype(target)
        arr = cls.__new__(cls)
        arr._buffer = None
        arr._np_data = np_array
        arr._shape = np_array.shape
        arr._dtype = target
        arr._strides = _c_contiguous_strides(np_array.shape)
        arr._offset = 0
        arr._base = None
        return arr

    @classmethod
    def _lazy(cls, node) -> "ndarray":
        arr = cls.__new__(cls)
        arr._buffer = None
        arr._np_data = None
        arr._shape = tuple(node._shape)
        arr._dtype = node._dtype
        arr._strides = _c_contiguous_strides(arr._shape)
        arr._offset = 0
        arr._base = None
        arr._fusion_node = node
        return arr

    @classmethod
    def _empty_device(cls, shape, dtype) -> "ndarray":
        shape = tuple(int(s) for s in shape)
        buf = HipBackend().create_buffer(_prod(shape), dtype)
        return cls(buf, shape, dtype)

    # ------------------------------------------------------- residency
    def _materialize_if_lazy(self) -> None:
        if self._fusion_node is not None:
            _fusion_mod.materialize(self)

    def _ensure_gpu(self) -> "ndarray":
        """Upload host-resident data (reference ndarray.py:352-368)."""
        self._materialize_if_lazy()
        if self._np_data is not None:
            data = np.ascontiguousarray(self._np_data)
            self._buffer = HipBackend().array_to_buffer(data)
            self._np_data = None
            self._strides = _c_contiguous_strides(self._shape)
            self._offset = 0
        return self

    def _is_c_contiguous(self) -> bool:
        return self._strides == _c_contiguous_strides(self._shape)

    def _is_device_contiguous(self) -> bool:
        return (self._fusion_node is None and self._np_data is None
                and self._buffer is not None and self._is_c_contiguous())

    def _ensure_contiguous(self) -> "ndarray":
        """Self if C-contiguous on the device, else a contiguous device copy."""
        self._materialize_if_lazy()
        if self._np_data is not None:
            return self._ensure_gpu()
        if self._is_c_contiguous():
            return self
        return self._contiguous_copy()

    @property
    def _ptr(self) -> int:
        return self._buffer.ptr + self._offset * self._dtype.itemsize

    def _contiguous_copy(self, dtype=None) -> "ndarray":
        """Strided (or casting) device copy (reference ndarray.py:483-513)."""
        self._ensure_gpu()
        dtype = self._dtype if dtype is None else np.dtype(dtype)
        out = ndarray._empty_device(self._shape, dtype)
        if self.size:
            HipBackend().copy(dtype_code(self._dtype), dtype_code(dtype), self._shape,
                              self._ptr, self._strides, out._ptr)
        return out

    def _broadcast_copy(self, shape, dtype) -> "ndarray":
        """Contiguous copy broadcast to ``shape`` (the reference's
        broadcast_nd kernel, _kernel_cache.py:74-97) with a cast."""
        from ._broadcasting import broadcast_strides
        self._ensure_gpu()
        st = broadcast_strides(self._shape, tuple(shape), self._strides)
        out = ndarray._empty_device(shape, dtype)
        if out.size:
            HipBackend().copy(dtype_code(self._dtype), dtype_code(dtype), tuple(shape),
                              self._ptr, st, out._ptr)
        return out

    # ----------------------------------------------------- host transfer
    def get(self, *, _force_copy: bool = False) -> np.ndarray:
        """Copy to host and return a NumPy array (reference ndarray.py:576-603)."""
        self._materialize_if_lazy()
        if self._np_data is not None:
            d = self._np_data
            return d.copy() if _force_copy else d
        src = self if self._is_c_contiguous() else self._contiguous_copy()
        be = HipBackend()
        out = be.host_empty(self._shape, self._dtype)
        be.read_buffer(src._buffer, src._offset * self._dtype.itemsize, out)
        return out

    def _get_view(self) -> np.ndarray:
        return self.get()

    def set(self, np_array) -> None:
        """Write host data into this array (reference ndarray.py:605-618)."""
        self._ensure_gpu()
        ew.flush_lazy(self._buffer)
        data = np.ascontiguousarray(np.broadcast_to(np.asarray(np_array, dtype=self._dtype),
                                                    self._shape))
        be = HipBackend()
        if self._is_c_contiguous():
            be.write_buffer(self._buffer, self._offset * self._dtype.itemsize, data)
        else:
            tmp = be.array_to_buffer(data)
            be.copy_strided(dtype_code(self._dtype), dtype_code(self._dtype), self._shape,
                            tmp.ptr, _c_contiguous_strides(self._shape), self._ptr,
                            self._strides)

    # ------------------------------------------------------- properties
    @property
    def shape(self):
        return self._shape

    @shape.setter
    def shape(self, value):
        self._assign(self.reshape(value))

    @property
    def dtype(self):
        return self._dtype

    @property
    def ndim(self) -> int:
        return len(self._shape)

    @property
    def size(self) -> int:
        return _prod(self._shape)

    @property
    def itemsize(self) -> int:
        return self._dtype.itemsize

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    @property
    def strides(self):
        """Byte strides (element strides x itemsize), as the reference."""
        return tuple(s * self.itemsize for s in self._strides)

    @property
    def T(self):
        return self.transpose()

    @property
    def mT(self):
        if self.ndim < 2:
            raise ValueError("matrix transpose with ndim < 2 is undefined")
        axes = list(range(self.ndim))
        axes[-2], axes[-1] = axes[-1], axes[-2]
        return self.transpose(axes)

    @property
    def base(self):
        return self._base

    @property
    def device(self):
        return "gpu"

    @property
    def real(self):
        return self

    @property
    def imag(self):
        from . import creation
        return creation.zeros(self._shape, dtype=self._dtype)

    @property
    def flags(self):
        return {"C_CONTIGUOUS": self._is_c_contiguous(), "OWNDATA": self._base is None}

    @property
    def flat(self):
        return iter(self.get().ravel())

    def _assign(self, other: "ndarray") -> None:
        self.__dict__.update(other.__dict__)

    # --------------------------------------------------------- views
    def reshape(self, *new_shape, order="C") -> "ndarray":
        if len(new_shape) == 1 and isinstance(new_shape[0], (tuple, list)):
            new_shape = tuple(new_shape[0])
        new_shape = tuple(int(s) for s in new_shape)
        if new_shape.count(-1) > 1:
            raise ValueError("can only specify one unknown dimension")
        if -1 in new_shape:
            known = _prod(s for s in new_shape if s != -1)
            if known == 0 or self.size % known:
                raise ValueError(f"cannot reshape array of size {self.size} into shape {new_shape}")
            new_shape = tuple(self.size // known if s == -1 else s for s in new_shape)
        if _prod(new_shape) != self.size:
            raise ValueError(f"cannot reshape array of size {self.size} into shape {new_shape}")
        if self._fusion_node is not None and self._shape == new_shape:
            return self
        # views of host-resident data live on the device, so that writes
        # through either alias reach the other
        src = self._ensure_contiguous()
        base = src._base if src._base is not None else src
        return ndarray(src._buffer, new_shape, self._dtype, offset=src._offset, base=base)

    def _view(self, shape, strides, offset) -> "ndarray":
        self._materialize_if_lazy()
        if self._np_data is not None:
            self._ensure_gpu()
        base = self._base if self._base is not None else self
        return ndarray(self._buffer, shape, self._dtype, strides=strides, offset=offset, base=base)

    def transpose(self, *axes) -> "ndarray":
        if len(axes) == 1 and (axes[0] is None or isinstance(axes[0], (tuple, list))):
            axes = axes[0]
        if not axes:
            axes = tuple(reversed(range(self.ndim)))
        axes = tuple(_normalize_axis(a, self.ndim) for a in axes)
        if sorted(axes) != list(range(self.ndim)):
            raise ValueError("axes don't match array")
        self._materialize_if_lazy()
        return self._view(tuple(self._shape[a] for a in axes),
                          tuple(self._strides[a] for a in axes), self._offset)

    def swapaxes(self, a1, a2) -> "ndarray":
        axes = list(range(self.ndim))
        a1, a2 = _normalize_axis(a1, self.ndim), _normalize_axis(a2, self.ndim)
        axes[a1], axes[a2] = axes[a2], axes[a1]
        return self.transpose(axes)

    def ravel(self, order="C") -> "ndarray":
        return self.reshape(-1)

    def flatten(self, order="C") -> "ndarray":
        return self.ravel().copy()

    def squeeze(self, axis=None) -> "ndarray":
        if axis is None:
            keep = [i for i, s in enumerate(self._shape) if s != 1]
        else:
            axes = (axis,) if isinstance(axis, int) else tuple(axis)
            axes = {_normalize_axis(a, self.ndim) for a in axes}
            for a in axes:
                if self._shape[a] != 1:
                    raise ValueError("cannot select an axis to squeeze out which has size not equal to one")
            keep = [i for i in range(self.ndim) if i not in axes]
        self._materialize_if_lazy()
        return self._view(tuple(self._shape[i] for i in keep),
                          tuple(self._strides[i] for i in keep), self._offset)

    def expand_dims(self, axis) -> "ndarray":
        from .manipulation import expand_dims
        return expand_dims(self, axis)

    # ------------------------------------------------------- indexing
    def _basic_index(self, key):
        """View for int/slice/None/Ellipsis keys, else None (reference
        ndarray.py:779-880)."""
        if not isinstance(key, tuple):
            key = (key,)
        for k in key:
            if isinstance(k, (bool, np.bool_)) or not (
                    isinstance(k, (int, np.integer, slice)) or k is None or k is Ellipsis):
                return None
        if sum(1 for k in key if k is Ellipsis) > 1:
            raise IndexError("an index can only have a single ellipsis ('...')")
        n_idx = sum(1 for k in key if k is not None and k is not Ellipsis)
        if n_idx > self.ndim:
            raise IndexError(f"too many indices for array: array is {self.ndim}-dimensional, "
                             f"but {n_idx} were indexed")
        if any(k is Ellipsis for k in key):
            i = next(j for j, k in enumerate(key) if k is Ellipsis)
            key = key[:i] + (slice(None),) * (self.ndim - n_idx) + key[i + 1:]
        shape, strides, offset, dim = [], [], self._offset, 0
        for k in key:
            if k is None:
                shape.append(1)
                strides.append(0)
                continue
            size, st = self._shape[dim], self._strides[dim]
            if isinstance(k, slice):
                start, stop, step = k.indices(size)
                length = len(range(start, stop, step))
                offset += start * st if length else 0
                shape.append(length)
                strides.append(st * step)
            else:
                idx = int(k)
                if not -size <= idx < size:
                    raise IndexError(f"index {idx} is out of bounds for axis {dim} with size {size}")
                offset += (idx % size) * st
            dim += 1
        shape.extend(self._shape[dim:])
        strides.extend(self._strides[dim:])
        return tuple(shape), tuple(strides), offset

    def __getitem__(self, key):
        if not _advanced_key(key):
            if self._np_data is not None:
                if _scalar_key(key, self.ndim):  # one element: read it where it is
                    return ndarray._from_np_direct(np.asarray(self._np_data[key]))
                self._ensure_gpu()  # a view: both aliases on the device
            basic = self._basic_index(key)
            if basic is not None:
                self._materialize_if_lazy()
                return self._view(*basic)
        # integer / boolean array indices: gathered on the device
        from . import indexing
        return indexing.getitem(self, key)

    def __setitem__(self, key, value):
        if _advanced_key(key):
            from . import indexing
            indexing.setitem(self, key, value)
            return
        if self._np_data is not None and not isinstance(value, ndarray):
            self._np_data[key] = value
            return
        self._ensure_gpu()
        basic = self._basic_index(key)
        if basic is None:
            raise IndexError("only integers, slices (`:`), ellipsis (`...`), numpy.newaxis "
                             "(`None`) and integer or boolean arrays are valid indices")
        shape, strides, offset = basic
        if _prod(shape) == 0:
            return
        ew.flush_lazy(self._buffer)
        target = ndarray(self._buffer, shape, self._dtype, strides=strides, offset=offset)
        from . import creation
        from ._broadcasting import broadcast_strides
        val = value if isinstance(value, ndarray) else creation.asarray(np.asarray(value))
        val._ensure_gpu()
        if val._buffer is self._buffer:
            val = val._contiguous_copy()
        vst = broadcast_strides(val._shape, shape, val._strides)
        HipBackend().copy_strided(dtype_code(val._dtype), dtype_code(self._dtype), shape,
                                  val._ptr, vst, target._ptr, strides)

    # --------------------------------------------------- arithmetic
    def __add__(self, o): return ew.binary("add_op", self, o)
    def __radd__(self, o): return ew.binary("add_op", o, self)
    def __sub__(self, o): return ew.binary("sub_op", self, o)
    def __rsub__(self, o): return ew.binary("sub_op", o, self)
    def __mul__(self, o): return ew.binary("mul_op", self, o)
    def __rmul__(self, o): return ew.binary("mul_op", o, self)
    def __truediv__(self, o): return ew.binary("div_op", self, o)
    def __rtruediv__(self, o): return ew.binary("div_op", o, self)
    def __floordiv__(self, o): return ew.binary("floor_divide_op", self, o)
    def __rfloordiv__(self, o): return ew.binary("floor_divide_op", o, self)
    def __mod__(self, o): return ew.binary("mod_op", self, o)
    def __rmod__(self, o): return ew.binary("mod_op", o, self)
    def __pow__(self, o): return ew.power(self, o)
    def __rpow__(self, o): return ew.binary("pow_op", o, self)
    def __neg__(self): return ew.unary("neg_op", self)
    def __pos__(self): return ew.unary("positive_op", self)
    def __abs__(self): return ew.unary("abs_op", self)

    def __and__(self, o): return ew.binary("bit_and_op", self, o)
    def __rand__(self, o): return ew.binary("bit_and_op", o, self)
    def __or__(self, o): return ew.binary("bit_or_op", self, o)
    def __ror__(self, o): return ew.binary("bit_or_op", o, self)
    def __xor__(self, o): return ew.binary("bit_xor_op", self, o)
    def __rxor__(self, o): return ew.binary("bit_xor_op", o, self)
    def __lshift__(self, o): return ew.binary("lshift_op", self, o)
    def __rlshift__(self, o): return ew.binary("lshift_op", o, self)
    def __rshift__(self, o): return ew.binary("rshift_op", self, o)
    def __rrshift__(self, o): return ew.binary("rshift_op", o, self)
    def __invert__(self): return ew.unary("invert_op", self)

    def __divmod__(self, o):
        return self // o, self % o

    def __matmul__(self, o):
        from .linalg_top import matmul
        return matmul(self, o)

    def __rmatmul__(self, o):
        from .linalg_top import matmul
        return matmul(o, self)

    def _inplace(self, result: "ndarray") -> "ndarray":
        """Write ``result`` into this array's memory (NumPy in-place
        semantics: views of ``self`` observe the update)."""
        if not np.can_cast(result._dtype, self._dtype, casting="same_kind"):
            raise TypeError(f"Cannot cast ufunc output from {result._dtype} to {self._dtype} "
                            "with casting rule 'same_kind'")
        if result._shape != self._shape:
            # the result has the broadcast shape of this array and the operand
            raise ValueError(f"non-broadcastable output operand with shape {self._shape} "
                             f"doesn't match the broadcast shape {result._shape}")
        if self._np_data is not None:
            self._ensure_gpu()
        ew.flush_lazy(self._buffer)
        res = result._ensure_contiguous()
        HipBackend().copy_strided(dtype_code(res._dtype), dtype_code(self._dtype), self._shape,
                                  res._ptr, _c_contiguous_strides(self._shape), self._ptr,
                                  self._strides)
        return self

    def __iadd__(self, o): return self._inplace(self.__add__(o))
    def __isub__(self, o): return self._inplace(self.__sub__(o))
    def __imul__(self, o): return self._inplace(self.__mul__(o))
    def __itruediv__(self, o): return self._inplace(self.__truediv__(o))
    def __ifloordiv__(self, o): return self._inplace(self.__floordiv__(o))
    def __imod__(self, o): return self._inplace(self.__mod__(o))
    def __ipow__(self, o): return self._inplace(self.__pow__(o))
    def __iand__(self, o): return self._inplace(self.__and__(o))
    def __ior__(self, o): return self._inplace(self.__or__(o))
    def __ixor__(self, o): return self._inplace(self.__xor__(o))
    def __ilshift__(self, o): return self._inplace(self.__lshift__(o))
    def __irshift__(self, o): return self._inplace(self.__rshift__(o))

    # ----------------------------------------------------- reductions
    def sum(self, axis=None, dtype=None, out=None, keepdims=False):
        from . import reductions
        return reductions.sum(self, axis=axis, dtype=dtype, out=out, keepdims=keepdims)

    def mean(self, axis=None, dtype=None, out=None, keepdims=False):
        from . import reductions
        return reductions.mean(self, axis=axis, dtype=dtype, out=out, keepdims=keepdims)

    def prod(self, axis=None, dtype=None, out=None, keepdims=False):
        from . import reductions
        return reductions.prod(self, axis=axis, dtype=dtype, out=out, keepdims=keepdims)

    def max(self, axis=None, out=None, keepdims=False):
        from . import reductions
        return reductions.max(self, axis=axis, out=out, keepdims=keepdims)

    def min(self, axis=None, out=None, keepdims=False):
        from . import reductions
        return reductions.min(self, axis=axis, out=out, keepdims=keepdims)

    def any(self, axis=None, out=None, keepdims=False):
        from . import reductions
        return reductions.any(self, axis=axis, out=out, keepdims=keepdims)

    def all(self, axis=None, out=None, keepdims=False):
        from . import reductions
        return reductions.all(self, axis=axis, out=out, keepdims=keepdims)

    def clip(self, min=None, max=None, out=None):
        from . import math_ops
        return math_ops.clip(self, min, max, out=out)

    def sort(self, axis=-1, kind=None, order=None):
        """Sort in place along ``axis`` (NumPy ndarray.sort)."""
        from . import sorting
        self._inplace(sorting.sort(self, axis=axis, kind=kind, order=order))

    def argsort(self, axis=-1, kind=None, order=None):
        from . import sorting
        return sorting.argsort(self, axis=axis, kind=kind, order=order)

    def nonzero(self):
        from .indexing import nonzero
        return nonzero(self)

    def take(self, indices, axis=None, out=None, mode="raise"):
        from .indexing import take
        return take(self, indices, axis=axis, out=out, mode=mode)

    def put(self, indices, values, mode="raise"):
        from .indexing import put
        return put(self, indices, values, mode=mode)

    def compress(self, condition, axis=None, out=None):
        from .indexing import compress
        return compress(condition, self, axis=axis, out=out)

    def searchsorted(self, v, side="left", sorter=None):
        from . import sorting
        return sorting.searchsorted(self, v, side=side, sorter=sorter)

    def argmax(self, axis=None, out=None, keepdims=False):
        from . import reductions
        return reductions.argmax(self, axis=axis, out=out, keepdims=keepdims)

    def argmin(self, axis=None, out=None, keepdims=False):
        from . import reductions
        return reductions.argmin(self, axis=axis, out=out, keepdims=keepdims)

    def cumsum(self, axis=None, dtype=None, out=None):
        from . import reductions
        return reductions.cumsum(self, axis=axis, dtype=dtype, out=out)

    def cumprod(self, axis=None, dtype=None, out=None):
        from . import reductions
        return reductions.cumprod(self, axis=axis, dtype=dtype, out=out)

    def var(self, axis=None, dtype=None, out=None, ddof=0, keepdims=False):
        from . import reductions
        return reductions.var(self, axis=axis, dtype=dtype, out=out, ddof=ddof, keepdims=keepdims)

    def std(self, axis=None, dtype=None, out=None, ddof=0, keepdims=False):
        from . import reductions
        return reductions.std(self, axis=axis, dtype=dtype, out=out, ddof=ddof, keepdims=keepdims)

    def dot(self, other):
        from .linalg_top import dot
        return dot(self, other)

    # --------------------------------------------------- conversions
    def astype(self, dtype, copy=True) -> "ndarray":
        """Cast (reference ndarray.py:2155-2197): a cast node when lazy,
        else the strided cast kernel."""
        dtype = resolve_dtype(dtype)
        if dtype == self._dtype and not copy:
            return self
        if self._np_data is not None:
            self._ensure_gpu()
        if self._fusion_node is not None:
            from ._fusion import CastNode
            out = ndarray._lazy(CastNode(self._fusion_node, dtype))
            ew.track_lazy(out)
            return out
        return self._contiguous_copy(dtype)

    def copy(self, order="C") -> "ndarray":
        if self._np_data is not None:
            return ndarray._from_np_direct(self._np_data.copy())
        self._materialize_if_lazy()
        return self._contiguous_copy()

    def fill(self, value) -> None:
        if self._np_data is not None:
            self._np_data.fill(value)
            return
        self._ensure_gpu()
        ew.flush_lazy(self._buffer)
        v = np.array(value).astype(self._dtype)
        if self._is_c_contiguous():
            HipBackend().fill(dtype_code(self._dtype), self.size, v, self._ptr)
        else:
            self[...] = v

    def item(self, *args):
        return self.get().item(*args)

    def tolist(self):
        return self.get().tolist()

    def __array__(self, dtype=None, copy=None):
        r = self.get()
        return r.astype(dtype) if dtype is not None else r

    def __float__(self):
        return float(self._scalar_value())

    def __int__(self):
        return int(self._scalar_value())

    def __index__(self):
        if not np.issubdtype(self._dtype, np.integer):
            raise TypeError("only integer arrays can be used as indices")
        return int(self._scalar_value())

    def __complex__(self):
        return complex(self._scalar_value())

    def __bool__(self):
        if self.size != 1:
            raise ValueError("The truth value of an array with more than one element is "
                             "ambiguous. Use a.any() or a.all()")
        return bool(self._scalar_value())

    def _scalar_value(self):
        if self.size != 1:
            raise TypeError("only length-1 arrays can be converted to Python scalars")
        return self.get().reshape(-1)[0]

    def __len__(self):
        if not self._shape:
            raise TypeError("len() of unsized object")
        return self._shape[0]

    def __iter__(self):
        if not self._shape:
            raise TypeError("iteration over a 0-d array")
        for i in range(self._shape[0]):
            yield self[i]

    def __repr__(self):
        return repr(self.get()).replace("array(", "array(", 1)

    def __str__(self):
        return str(self.get())

    def __reduce__(self):
        return (_reconstruct, (self.get(),))

    __hash__ = None

    # ------------------------------------------------------ comparisons
    # Device comparisons through the fusion engine (bool results).
    def __lt__(self, o): return ew.binary("lt_op", self, o)
    def __le__(self, o): return ew.binary("le_op", self, o)
    def __gt__(self, o): return ew.binary("gt_op", self, o)
    def __ge__(self, o): return ew.binary("ge_op", self, o)
    def __eq__(self, o): return ew.binary("eq_op", self, o)
    def __ne__(self, o): return ew.binary("ne_op", self, o)

    # ------------------------------------------------- numpy protocols
    def __array_ufunc__(self, ufunc, method, *inputs, **kwargs):
        """Route NumPy ufunc calls on device arrays to the device ops
        (reference ndarray.py:2681-2720, which falls back to NumPy on the
        host): ``__call__`` with ``out=`` / ``dtype=`` / ``where=`` (with
        ``out``), ``reduce`` and ``accumulate`` of the ufuncs that have a
        reduction or scan.  Anything else returns NotImplemented, so NumPy
        raises TypeError rather than computing on the host."""
        from . import _ufunc_table
        return _ufunc_table.dispatch(ufunc, method, inputs, kwargs)

    def __array_namespace__(self, *, api_version=None):
        import macmetalpy_amd
        return macmetalpy_amd

    def __array_function__(self, func, types, args, kwargs):
        """NumPy functions called with device arrays run this library's
        function of the same name (``numpy.linalg`` ones the ``linalg``
        namespace's), as the reference dispatches (ndarray.py:2722-2729);
        a function without a device counterpart returns NotImplemented, so
        NumPy raises TypeError instead of computing on the host."""
        import macmetalpy_amd as mod
        name = getattr(func, "__name__", "")
        where = getattr(func, "__module__", "") or ""
        if where.startswith("numpy.linalg"):
            target = getattr(mod.linalg, name, None)
        elif where.startswith("numpy.fft"):
            target = getattr(mod.fft, name, None)
        else:
            target = getattr(mod, name, None)
        if target is None or target is func or not callable(target):
            return NotImplemented
        return target(*args, **kwargs)

    @classmethod
    def __class_getitem__(cls, item):
        return cls

    def __contains__(self, value):
        return bool((self == value).any())

    def __copy__(self):
        return self.copy()

    def __deepcopy__(self, memo):
        return self.copy()

    def __delitem__(self, key):
        raise ValueError("cannot delete array elements")

    def __imatmul__(self, o):
        from .linalg_top import matmul
        r = matmul(self, o)
        if tuple(r.shape) != self._shape:
            raise ValueError("matmul: in-place result would change the array's shape")
        return self._inplace(r)

    def __rdivmod__(self, o):
        return o // self, o % self

    def __dlpack__(self, *, stream=None, max_version=None, dl_device=None, copy=None):
        """A host copy's DLPack capsule (as the reference exports)."""
        return self.get().__dlpack__()

    def __dlpack_device__(self):
        return (1, 0)

    # ---------------------------------------------- more NumPy methods
    def view(self, dtype=None, type=None):
        """Same device bytes read as another dtype; a different item size
        needs a contiguous last axis whose byte length it divides."""
        import builtins
        self._materialize_if_lazy()
        if self._np_data is not None:
            self._ensure_gpu()
        if dtype is None or (isinstance(dtype, builtins.type) and issubclass(dtype, ndarray)):
            return ndarray(self._buffer, self._shape, self._dtype, self._strides, self._offset,
                           self._base if self._base is not None else self)
        new = np.dtype(dtype)
        from ._dtypes import dtype_code
        dtype_code(new)
        old = self._dtype.itemsize
        base = self._base if self._base is not None else self
        if new.itemsize == old:
            return ndarray(self._buffer, self._shape, new, self._strides, self._offset, base)
        if not self._shape or self._strides[-1] != 1:
            raise ValueError("To change to a dtype of a different size, the last axis must be "
                             "contiguous")
        nbytes_last = self._shape[-1] * old
        if nbytes_last % new.itemsize:
            raise ValueError("When changing to a smaller dtype, its size must be a divisor of the "
                             "size of original dtype" if new.itemsize < old else
                             "When changing to a larger dtype, its size must be a divisor of the "
                             "total size in bytes of the last axis of the array.")
        if (self._offset * old) % new.itemsize or any((st * old) % new.itemsize
                                                      for st in self._strides[:-1]):
            raise ValueError("the array's offset or strides are not a multiple of the new "
                             "dtype's size")
        shape = self._shape[:-1] + (nbytes_last // new.itemsize,)
        strides = tuple(st * old // new.itemsize for st in self._strides[:-1]) + (1,)
        return ndarray(self._buffer, shape, new, strides, self._offset * old // new.itemsize, base)

    def byteswap(self, inplace=False):
        """Byte order reversed per element with shifts on the unsigned view."""
        size = self._dtype.itemsize
        if size == 1 or self._dtype == np.bool_:
            r = self.copy()
        else:
            ut = {2: np.uint16, 4: np.uint32, 8: np.uint64}[size]
            u = self._ensure_contiguous().view(ut)
            acc = None
            for k in range(size):
                byte = (u >> ut(8 * k)) & ut(0xFF)
                part = byte << ut(8 * (size - 1 - k))
                acc = part if acc is None else (acc | part)
            r = acc.astype(ut).view(self._dtype)
        if inplace:
            self[...] = r
            return self
        return r

    def partition(self, kth, axis=-1, kind="introselect", order=None):
        """In place; a full sort satisfies every kth."""
        from .extras import partition
        self[...] = partition(self, kth, axis=axis)

    def argpartition(self, kth, axis=-1, kind="introselect", order=None):
        from .extras import argpartition
        return argpartition(self, kth, axis=axis)

    def choose(self, choices, out=None, mode="raise"):
        from .extras import choose
        return choose(self, choices, out=out, mode=mode)

    def conj(self):
        return self.copy()

    conjugate = conj

    def diagonal(self, offset=0, axis1=0, axis2=1):
        from .manipulation import diagonal
        return diagonal(self, offset, axis1, axis2)

    def trace(self, offset=0, axis1=0, axis2=1, dtype=None, out=None):
        from .manipulation import trace
        return trace(self, offset, axis1, axis2, dtype, out)

    def ptp(self, axis=None, out=None, keepdims=False):
        from .manipulation import ptp
        return ptp(self, axis=axis, out=out, keepdims=keepdims)

    def repeat(self, repeats, axis=None):
        from .manipulation import repeat
        return repeat(self, repeats, axis=axis)

    def round(self, decimals=0, out=None):
        from .extras import round as _round
        return _round(self, decimals, out=out)

    def resize(self, *new_shape, refcheck=True):
        """In place, as NumPy's method: the flat data kept, zeros appended."""
        if len(new_shape) == 1 and not isinstance(new_shape[0], (int, np.integer)):
            new_shape = tuple(new_shape[0])
        shp = tuple(int(x) for x in new_shape)
        from .creation import zeros
        n = _prod(shp)
        out = zeros((n,), dtype=self._dtype)
        k = min(n, self.size)
        if k:
            out[:k] = self.ravel()[:k]
        out = out.reshape(shp)._ensure_contiguous()
        self._buffer, self._np_data = out._buffer, None
        self._shape, self._strides, self._offset, self._base = out._shape, out._strides, 0, None
        self._fusion_node = None

    def itemset(self, *args):
        if not args:
            raise ValueError("itemset must have at least one argument")
        *idx, value = args
        if not idx:
            self.reshape(-1)[0:1] = value
        elif len(idx) == 1 and isinstance(idx[0], (int, np.integer)):
            flat = self.ravel()
            flat[idx[0]] = value
            if flat._buffer is not self._buffer:
                self[...] = flat.reshape(self._shape)
        else:
            self[tuple(idx[0]) if len(idx) == 1 else tuple(idx)] = value

    def setflags(self, write=None, align=None, uic=None):
        """Device arrays stay writeable and aligned; the flags are accepted."""
        return None

    def to_device(self, device, /, *, stream=None):
        return self

    @property
    def data(self):
        """Device address of the first element (an integer), for callers
        handing the buffer to their own kernels."""
        self._ensure_gpu()
        return self._ptr

    def getfield(self, dtype, offset=0):
        if offset != 0 or np.dtype(dtype).itemsize != self._dtype.itemsize:
            raise NotImplementedError("getfield needs offset 0 and an equal item size")
        return self.view(dtype).copy()

    def setfield(self, val, dtype, offset=0):
        if offset != 0 or np.dtype(dtype).itemsize != self._dtype.itemsize:
            raise NotImplementedError("setfield needs offset 0 and an equal item size")
        self.view(dtype)[...] = val

    def tobytes(self, order="C"):
        return self.get().tobytes(order)

    tostring = tobytes

    def tofile(self, fid, sep="", format="%s"):
        self.get().tofile(fid, sep=sep, format=format)

    def dump(self, file):
        self.get().dump(file)

    def dumps(self):
        return self.get().dumps()


def _scalar_key(key, ndim) -> bool:
    """Whether ``key`` is one integer per dimension (selects one element)."""
    items = key if isinstance(key, tuple) else (key,)
    return len(items) == ndim and all(
        isinstance(k, (int, np.integer)) and not isinstance(k, (bool, np.bool_)) for k in items)


def _advanced_key(key) -> bool:
    """Whether ``key`` holds an integer or boolean array (or a sequence or a
    boolean scalar), i.e. needs NumPy's advanced indexing."""
    items = key if isinstance(key, tuple) else (key,)
    for k in items:
        if isinstance(k, (ndarray, np.ndarray, list, bool, np.bool_)):
            return True
        if isinstance(k, tuple):
            return True
    return False


def _reconstruct(np_array):
    return ndarray._from_np_direct(np_array)


def _wrap_np(np_array) -> ndarray:
    return ndarray._from_np_direct(np_array)
