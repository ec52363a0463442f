"""Names of the reference's namespace that compute no array data on the
device: dtype aliases and the scalar-type hierarchy, printing, file I/O,
datetime helpers, error-state and buffer settings, and Python-callable
wrappers.

The reference re-exports NumPy's objects for these (dtype_utils.py,
format_ops.py, io.py, utils.py, functional.py, config_ops.py).  Arrays pass
through the host only where the operation is host work by nature: text and
file formats are read and written by NumPy and the data is uploaded once,
printing formats a host copy, and ``vectorize`` / ``frompyfunc`` call a
Python function per element.  ``fromfunction`` evaluates its function on
device index grids.
"""
from __future__ import annotations

import os

import numpy as np

from .ndarray import ndarray

# ----------------------------------------------------- dtypes and scalars
False_ = np.False_
True_ = np.True_
ScalarType = np.ScalarType
byte, ubyte, short, ushort = np.byte, np.ubyte, np.short, np.ushort
intc, uintc, uint, longlong, ulonglong = np.intc, np.uintc, np.uint, np.longlong, np.ulonglong
int_, intp, uintp = np.int64, np.intp, np.uintp
int8, uint8 = np.int8, np.uint8
single, double, half, longdouble = np.single, np.double, np.half, np.longdouble
float_, longfloat = np.float64, np.longdouble
csingle, cdouble, clongdouble = np.csingle, np.cdouble, np.clongdouble
complex64, complex128, complex_, cfloat = np.complex64, np.complex128, np.complex128, np.complex128
singlecomplex, longcomplex, clongfloat = np.complex64, np.clongdouble, np.clongdouble
bytes_, str_, object_, void = np.bytes_, np.str_, np.object_, np.void
datetime64, timedelta64 = np.datetime64, np.timedelta64
generic, number, integer, signedinteger = np.generic, np.number, np.integer, np.signedinteger
unsignedinteger, inexact, floating, complexfloating = (np.unsignedinteger, np.inexact,
                                                       np.floating, np.complexfloating)
character, flexible = np.character, np.flexible
dtype = np.dtype
sctypeDict = np.sctypeDict
typecodes = np.typecodes
little_endian = np.little_endian
euler_gamma = np.euler_gamma
issubdtype = np.issubdtype
isdtype = np.isdtype
mintypecode = np.mintypecode
typename = np.typename
iterable = np.iterable
broadcast = np.broadcast
flatiter = np.flatiter
ndindex = np.ndindex


def _dt(x):
    return x.dtype if isinstance(x, ndarray) else np.asarray(x).dtype


def common_type(*arrays):
    """NumPy's rule on the arrays' dtypes: integers count as float64,
    otherwise the widest float."""
    best = np.float16
    for a in arrays:
        d = _dt(a)
        if d.kind in "iub":
            t = np.float64
        elif d.kind == "f":
            t = d.type
        elif d.kind == "c":
            t = d.type
        else:
            raise TypeError("can't get common type for non-numeric array")
        best = np.result_type(best, t).type
    return best


def min_scalar_type(a):
    return np.min_scalar_type(a.get() if isinstance(a, ndarray) else a)


def iscomplexobj(x):
    return _dt(x).kind == "c"


def isrealobj(x):
    return not iscomplexobj(x)


def isfortran(a):
    """Device arrays are C-ordered, so never Fortran-only contiguous."""
    return False


def _extent(a):
    a._materialize_if_lazy()
    if a._buffer is None:
        return None
    lo = hi = a._offset
    for n, s in zip(a.shape, a._strides):
        if n == 0:
            return a._buffer, 0, 0
        if s >= 0:
            hi += (n - 1) * s
        else:
            lo += (n - 1) * s
    item = a.dtype.itemsize
    return a._buffer, lo * item, (hi + 1) * item


def may_share_memory(a, b, max_work=None):
    """Whether the two arrays' byte ranges in one device buffer overlap."""
    if not (isinstance(a, ndarray) and isinstance(b, ndarray)):
        return False
    ea, eb = _extent(a), _extent(b)
    if ea is None or eb is None or ea[0] is not eb[0]:
        return False
    return ea[1] < eb[2] and eb[1] < ea[2]


def shares_memory(a, b, max_work=None):
    """Exact for views along one axis; overlapping extents otherwise."""
    return may_share_memory(a, b)


# -------------------------------------------------------------- printing
def _h(a):
    return a.get() if isinstance(a, ndarray) else a


def array2string(a, *args, **kwargs):
    return np.array2string(_h(a), *args, **kwargs)


def array_repr(arr, max_line_width=None, precision=None, suppress_small=None):
    return np.array_repr(_h(arr), max_line_width, precision, suppress_small)


def array_str(a, max_line_width=None, precision=None, suppress_small=None):
    return np.array_str(_h(a), max_line_width, precision, suppress_small)


set_printoptions = np.set_printoptions
get_printoptions = np.get_printoptions
printoptions = np.printoptions
format_float_positional = np.format_float_positional
format_float_scientific = np.format_float_scientific
base_repr = np.base_repr
binary_repr = np.binary_repr
info = np.info

# Floating-point error state and the ufunc buffer size belong to NumPy's
# host loops; device kernels follow IEEE semantics without traps.
errstate = np.errstate
seterr = np.seterr
geterr = np.geterr
seterrcall = np.seterrcall
geterrcall = np.geterrcall
getbufsize = np.getbufsize
setbufsize = np.setbufsize


def get_include():
    """Directory of the C header of the device library (mmp_hip.h)."""
    return os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")


def show_config():
    from ._backend import lib_path
    print(f"macmetalpy_amd: HIP library {lib_path()}, target gfx950")


def show_runtime():
    from ._backend import lib_path
    print(f"macmetalpy_amd: HIP library {lib_path()} "
          f"({'present' if os.path.exists(lib_path()) else 'missing'})")


# ------------------------------------------------------------------- I/O
def _up(x):
    from .creation import asarray
    return asarray(x) if isinstance(x, np.ndarray) else x


def save(file, arr, allow_pickle=True):
    np.save(file, _h(arr), allow_pickle=allow_pickle)


def savez(file, *args, **kwds):
    np.savez(file, *[_h(a) for a in args], **{k: _h(v) for k, v in kwds.items()})


def savez_compressed(file, *args, **kwds):
    np.savez_compressed(file, *[_h(a) for a in args], **{k: _h(v) for k, v in kwds.items()})


class _NpzOnDevice:
    """Mapping over an .npz archive that uploads each member when read."""

    def __init__(self, npz):
        self._npz = npz

    def __getitem__(self, key):
        return _up(self._npz[key])

    def keys(self):
        return self._npz.keys()

    @property
    def files(self):
        return self._npz.files

    def __iter__(self):
        return iter(self._npz.files)

    def __len__(self):
        return len(self._npz.files)

    def __contains__(self, key):
        return key in self._npz.files

    def items(self):
        return [(k, self[k]) for k in self._npz.files]

    def close(self):
        self._npz.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def load(file, mmap_mode=None, allow_pickle=False, fix_imports=True, encoding="ASCII", *,
         max_header_size=None):
    kw = {} if max_header_size is None else {"max_header_size": max_header_size}
    r = np.load(file, mmap_mode=mmap_mode, allow_pickle=allow_pickle, fix_imports=fix_imports,
                encoding=encoding, **kw)
    if isinstance(r, np.lib.npyio.NpzFile):
        return _NpzOnDevice(r)
    return _up(np.asarray(r)) if isinstance(r, np.ndarray) else r


def loadtxt(fname, *args, **kwargs):
    return _up(np.loadtxt(fname, *args, **kwargs))


def savetxt(fname, X, *args, **kwargs):
    np.savetxt(fname, _h(X), *args, **kwargs)


def genfromtxt(fname, *args, **kwargs):
    return _up(np.genfromtxt(fname, *args, **kwargs))


def fromfile(file, dtype=float, count=-1, sep="", offset=0):
    return _up(np.fromfile(file, dtype=dtype, count=count, sep=sep, offset=offset))


def fromregex(file, regexp, dtype, encoding=None):
    return _up(np.fromregex(file, regexp, dtype, encoding=encoding))


def frombuffer(buffer, dtype=float, count=-1, offset=0):
    return _up(np.frombuffer(buffer, dtype=dtype, count=count, offset=offset).copy())


def fromstring(string, dtype=float, count=-1, *, sep):
    return _up(np.fromstring(string, dtype=dtype, count=count, sep=sep))


def fromiter(iter, dtype, count=-1):
    return _up(np.fromiter(iter, dtype=dtype, count=count))


def from_dlpack(x, /, *, device=None, copy=None):
    """Host DLPack producers (NumPy arrays, CPU tensors) are uploaded."""
    return _up(np.from_dlpack(x))


def fromfunction(function, shape, *, dtype=float, **kwargs):
    """Calls the function once with device index grids (NumPy's contract:
    one array per dimension, each holding its coordinate)."""
    from .extras import indices
    grids = indices(tuple(shape), dtype=dtype)
    return function(*[grids[i] for i in range(len(shape))], **kwargs)


memmap = np.memmap

# --------------------------------------------------------- datetime (host)
busday_count = np.busday_count
busday_offset = np.busday_offset
busdaycalendar = np.busdaycalendar
is_busday = np.is_busday
datetime_as_string = np.datetime_as_string
datetime_data = np.datetime_data

# ------------------------------------------------------- legacy host types
matrix = np.matrix
asmatrix = np.asmatrix
bmat = np.bmat
recarray = np.recarray
record = np.record


# ------------------------------------------------- Python callables per element
class vectorize:
    """Calls a Python function per element, as NumPy's vectorize does (on
    host copies of the arguments), and returns device arrays."""

    def __init__(self, pyfunc=None, otypes=None, doc=None, excluded=None, cache=False,
                 signature=None):
        self._v = np.vectorize(pyfunc, otypes=otypes, doc=doc, excluded=excluded, cache=cache,
                               signature=signature)
        self.__doc__ = self._v.__doc__

    def __call__(self, *args, **kwargs):
        r = self._v(*[_h(a) for a in args], **{k: _h(v) for k, v in kwargs.items()})
        if isinstance(r, tuple):
            return tuple(_up(np.asarray(x)) for x in r)
        return _up(np.asarray(r))


def frompyfunc(func, /, nin, nout, *, identity=None):
    uf = np.frompyfunc(func, nin, nout) if identity is None else \
        np.frompyfunc(func, nin, nout, identity=identity)

    def call(*args, **kwargs):
        r = uf(*[_h(a) for a in args], **kwargs)
        if isinstance(r, tuple):
            return tuple(_up(np.asarray(x)) for x in r)
        return _up(np.asarray(r)) if isinstance(r, np.ndarray) else r

    call.__name__ = getattr(func, "__name__", "frompyfunc")
    return call


def nditer(op, *args, **kwargs):
    """Iteration over host copies of the operands (read-only)."""
    ops = [_h(o) for o in op] if isinstance(op, (list, tuple)) else _h(op)
    return np.nditer(ops, *args, **kwargs)


def sort_complex(a):
    raise TypeError("sort_complex needs complex dtypes, which the device arrays do not hold")


# NumPy 1.x's error object: [buffer size, mask, callback], the mask holding
# one 3-bit mode per condition (divide, over, under, invalid at bits 0, 3,
# 6, 9; modes ignore, warn, raise, call, print, log = 0..5).  NumPy 2
# dropped these functions; they are rebuilt on seterr / setbufsize.
_ERR_MODES = ("ignore", "warn", "raise", "call", "print", "log")
_ERR_FIELDS = (("divide", 0), ("over", 3), ("under", 6), ("invalid", 9))


def geterrobj():
    state = np.geterr()
    mask = 0
    for name, shift in _ERR_FIELDS:
        mask |= _ERR_MODES.index(state[name]) << shift
    return [np.getbufsize(), mask, np.geterrcall()]


def seterrobj(errobj):
    bufsize, mask, callback = errobj
    np.setbufsize(bufsize)
    np.seterr(**{name: _ERR_MODES[(mask >> shift) & 7] for name, shift in _ERR_FIELDS})
    np.seterrcall(callback)


def set_numeric_ops(**ops):
    """Removed in NumPy 2; accepted and ignored (an empty mapping back)."""
    return {}
