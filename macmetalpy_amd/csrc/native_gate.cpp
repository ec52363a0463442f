// native_gate.cpp -- CPython extension `macmetalpy_amd._native`: the host
// dispatch path of elementwise ops, in C.
//
// Reference: src/macmetalpy/_accelerator.c:549-858 (fast_binary /
// fast_unary / fast_reduce) gates every op in C before the Python path:
// CPU-resident arrays below the size thresholds of ndarray.py:41-44 go to
// NumPy, everything else returns None and continues in Python.  Here the
// device runs every size, so the gate's job is the other half of that
// contract -- do the common case natively, hand everything else back:
//
//  * unary(op, x) / binary(op, a, b): when the operands are ndarrays whose
//    shapes broadcast, or an array and a Python int / float, build the lazy
//    fusion node and the result array in C (the result dtype comes from a
//    table the Python path fills on first use).  A host-resident operand
//    (an array made from NumPy data, the case the reference's C gate
//    answers on the CPU) with C-contiguous data is uploaded here first,
//    through mmp_h2d's page-locked staging, so small host arrays reach the
//    same device kernels without a pass through Python;
//  * reduce(code, x, axis): whole-array or last-axis reductions of a
//    contiguous array (host-resident ones uploaded the same way);
//  * materialize(arr): evaluate a lazy array -- one precompiled kernel for
//    a single op over contiguous operands (mmp_unary / mmp_binary /
//    mmp_binary_scalar), else the generated fused kernel, looked up by the
//    program's structure in a C++ table, with its parameter block packed
//    here and launched through mmp_rtc_launch;
//  * DeviceBuffer: the owning handle of one device allocation, freed with
//    mmp_free when the last reference goes.
//
// Anything else (shapes that do not broadcast, host data that is not
// C-contiguous, depth or leaf caps, casts of leaves to a new dtype at the
// root, float16 scalars, unfused mode ...) calls the Python implementation,
// which stays the single definition of the semantics.  The generated kernel
// for a structure seen for the first time is compiled by a Python callback
// from the same DAG, traversed in the same order as here, so leaves,
// scalars and the parameter block agree.  Library functions are reached through pointers
// handed over by the ctypes binding (one loaded copy of libmmp_hip.so).
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <structmember.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

// ------------------------------------------------------ library entry points
typedef int (*fn_alloc_t)(size_t, void **);
typedef int (*fn_free_t)(void *);
typedef int (*fn_unary_t)(int, int, int64_t, const void *, void *);
typedef int (*fn_binary_t)(int, int, int64_t, const void *, const void *, void *);
typedef int (*fn_binary_scalar_t)(int, int, int64_t, const void *, const void *, int, void *);
typedef int (*fn_launch_t)(void *, const uint32_t *, const uint32_t *, uint32_t, void **);
typedef int (*fn_reduce_t)(int, int, int, int64_t, int64_t, int64_t, const void *, void *);
typedef int (*fn_argreduce_t)(int, int, int64_t, int64_t, int64_t, const void *, int64_t *);
typedef int (*fn_d2h_t)(void *, const void *, size_t);
typedef int (*fn_h2d_t)(void *, const void *, size_t);

fn_alloc_t p_alloc = nullptr;
fn_free_t p_free = nullptr;
fn_unary_t p_unary = nullptr;
fn_binary_t p_binary = nullptr;
fn_binary_scalar_t p_binary_scalar = nullptr;
fn_launch_t p_launch = nullptr;
fn_reduce_t p_reduce = nullptr;
fn_argreduce_t p_argreduce = nullptr;
fn_d2h_t p_d2h = nullptr;
fn_h2d_t p_h2d = nullptr;

// ------------------------------------------------------------ DeviceBuffer
struct DevBuf {
  PyObject_HEAD
  unsigned long long ptr;
  long long nbytes;
  int owned;                  // free with mmp_free at the end (else: borrowed memory)
  PyObject *lazy_dependents;  // list of weakrefs to lazy arrays reading it, or NULL
  PyObject *weakreflist;
};

void devbuf_dealloc(DevBuf *self) {
  if (self->weakreflist) PyObject_ClearWeakRefs((PyObject *)self);
  if (self->ptr && self->owned && p_free) p_free((void *)(uintptr_t)self->ptr);
  self->ptr = 0;
  Py_CLEAR(self->lazy_dependents);
  Py_TYPE(self)->tp_free((PyObject *)self);
}

int devbuf_init(DevBuf *self, PyObject *args, PyObject *kw) {
  unsigned long long ptr = 0;
  long long nbytes = 0;
  int owned = 1;
  static const char *kwlist[] = {"ptr", "nbytes", "owned", nullptr};
  if (!PyArg_ParseTupleAndKeywords(args, kw, "KL|p", (char **)kwlist, &ptr, &nbytes, &owned))
    return -1;
  self->ptr = ptr;
  self->nbytes = nbytes;
  self->owned = owned;
  return 0;
}

PyObject *devbuf_repr(DevBuf *self) {
  char buf[96];
  std::snprintf(buf, sizeof buf, "DeviceBuffer(0x%llx, %lld bytes)", self->ptr, self->nbytes);
  return PyUnicode_FromString(buf);
}

PyObject *devbuf_get_deps(DevBuf *self, void *) {
  PyObject *v = self->lazy_dependents ? self->lazy_dependents : Py_None;
  Py_INCREF(v);
  return v;
}

int devbuf_set_deps(DevBuf *self, PyObject *v, void *) {
  Py_CLEAR(self->lazy_dependents);
  if (v && v != Py_None) {
    Py_INCREF(v);
    self->lazy_dependents = v;
  }
  return 0;
}

PyMemberDef devbuf_members[] = {
    {(char *)"ptr", T_ULONGLONG, offsetof(DevBuf, ptr), 0, (char *)"device address"},
    {(char *)"nbytes", T_LONGLONG, offsetof(DevBuf, nbytes), 0, (char *)"size in bytes"},
    {nullptr, 0, 0, 0, nullptr}};

PyGetSetDef devbuf_getset[] = {
    {(char *)"lazy_dependents", (getter)devbuf_get_deps, (setter)devbuf_set_deps,
     (char *)"weak references to lazy arrays whose expression reads this buffer", nullptr},
    {nullptr, nullptr, nullptr, nullptr, nullptr}};

PyTypeObject DevBufType = {PyVarObject_HEAD_INIT(nullptr, 0)};

// ------------------------------------------------------------- state
PyTypeObject *T_ndarray = nullptr, *T_input = nullptr, *T_cast = nullptr, *T_unary = nullptr,
             *T_binary = nullptr, *T_scalar = nullptr, *T_where = nullptr;
PyObject *py_unary_fb = nullptr, *py_binary_fb = nullptr, *py_materialize_fb = nullptr,
         *py_run_sum_fb = nullptr, *py_reduce_dt = nullptr;
PyObject *py_compile_map = nullptr, *py_check = nullptr, *py_unary_dt = nullptr,
         *py_binary_dt = nullptr, *py_prune = nullptr, *py_ensure_device = nullptr;
PyObject *cfg_obj = nullptr;
constexpr int kNDT = 10;
PyObject *dtypes[kNDT] = {};
int itemsize[kNDT] = {1, 2, 2, 4, 4, 8, 8, 2, 4, 8};
enum { D_BOOL = 0, D_I16, D_U16, D_I32, D_U32, D_I64, D_U64, D_F16, D_F32, D_F64 };
long max_depth = 16, max_leaves = 24;
long sum_blocks = 1024;  // workgroups of a fused row-sum launch (init key "sum_blocks")

// slot descriptors of the fusion node classes
PyObject *d_shape, *d_dtype, *d_depth, *d_buffers, *d_nleaves;
PyObject *d_in_buffer, *d_in_offset, *d_in_strides, *d_sc_bits;
PyObject *d_un_op, *d_un_input, *d_cast_input, *d_bin_op, *d_bin_lhs, *d_bin_rhs;
PyObject *d_wh_cond, *d_wh_x, *d_wh_y;

// interned attribute names
PyObject *s_buffer, *s_np_data, *s_shape, *s_dtype, *s_strides, *s_offset, *s_base, *s_fnode,
    *s_fusion, *s_fast_math;

// op tables (ids assigned by init)
constexpr int kMaxOps = 160;
PyObject *op_ids = nullptr;  // dict name -> id
int n_ops = 0;
int unary_code[kMaxOps], binary_code[kMaxOps];
bool fast_op[kMaxOps];
bool int_unary_op[kMaxOps];  // mmp_unary also defines the op for integer dtypes
int8_t un_rdt[kMaxOps][kNDT], un_idt[kMaxOps][kNDT];
int8_t bin_rdt[kMaxOps][kNDT][kNDT], bin_odt[kMaxOps][kNDT][kNDT];
// array dtype x scalar kind (0 float, 1 int) x scalar side (0 left, 1 right):
// type resolution need not be symmetric (ldexp takes a float first)
int8_t bsc_rdt[kMaxOps][kNDT][2][2], bsc_odt[kMaxOps][kNDT][2][2];

std::unordered_map<std::string, void *> g_kernels;  // structure key -> kernel handle
unsigned long long stat_native_ops = 0, stat_native_mat = 0, stat_fallback = 0, stat_uploads = 0;

// ------------------------------------------------------------ helpers
inline PyObject *dget(PyObject *descr, PyObject *obj) {  // new reference
  return Py_TYPE(descr)->tp_descr_get(descr, obj, (PyObject *)Py_TYPE(obj));
}
inline int dset(PyObject *descr, PyObject *obj, PyObject *v) {
  return Py_TYPE(descr)->tp_descr_set(descr, obj, v);
}
inline long long dget_ll(PyObject *descr, PyObject *obj) {
  PyObject *v = dget(descr, obj);
  if (!v) return -1;
  long long r = PyLong_AsLongLong(v);
  Py_DECREF(v);
  return r;
}

inline int dtype_index(PyObject *dt) {
  for (int i = 0; i < kNDT; ++i)
    if (dtypes[i] == dt) return i;
  return -1;
}

inline PyObject *inst_dict(PyObject *o) {
  PyObject **dp = _PyObject_GetDictPtr(o);
  return dp ? *dp : nullptr;
}

// borrowed; NULL if absent
inline PyObject *iget(PyObject *dict, PyObject *name) { return dict ? PyDict_GetItem(dict, name) : nullptr; }

bool cfg_flag(PyObject *name) {
  PyObject *d = inst_dict(cfg_obj);
  PyObject *v = iget(d, name);
  return v == Py_True;
}

bool shape_size(PyObject *shape, long long *n) {
  if (!PyTuple_CheckExact(shape)) return false;
  long long s = 1;
  for (Py_ssize_t i = 0; i < PyTuple_GET_SIZE(shape); ++i) {
    long long v = PyLong_AsLongLong(PyTuple_GET_ITEM(shape, i));
    if (v < 0) {
      PyErr_Clear();
      return false;
    }
    s *= v;
  }
  *n = s;
  return true;
}

PyObject *contig_strides(PyObject *shape) {
  const Py_ssize_t nd = PyTuple_GET_SIZE(shape);
  PyObject *t = PyTuple_New(nd);
  if (!t) return nullptr;
  long long acc = 1;
  for (Py_ssize_t i = nd - 1; i >= 0; --i) {
    PyObject *v = PyLong_FromLongLong(acc);
    if (!v) {
      Py_DECREF(t);
      return nullptr;
    }
    PyTuple_SET_ITEM(t, i, v);
    acc *= PyLong_AsLongLong(PyTuple_GET_ITEM(shape, i));
  }
  return t;
}

bool is_contig(PyObject *shape, PyObject *strides) {
  if (!PyTuple_CheckExact(strides) || PyTuple_GET_SIZE(strides) != PyTuple_GET_SIZE(shape))
    return false;
  long long acc = 1;
  for (Py_ssize_t i = PyTuple_GET_SIZE(shape) - 1; i >= 0; --i) {
    if (PyLong_AsLongLong(PyTuple_GET_ITEM(strides, i)) != acc) return false;
    acc *= PyLong_AsLongLong(PyTuple_GET_ITEM(shape, i));
  }
  return true;
}

PyObject *alloc_slots(PyTypeObject *t) { return t->tp_alloc(t, 0); }

// ------------------------------------------------------- node builders
// Each returns a new reference or NULL with an exception set.
PyObject *new_input(PyObject *buffer, PyObject *shape, PyObject *dtype, PyObject *strides,
                    PyObject *offset) {
  PyObject *n = alloc_slots(T_input);
  if (!n) return nullptr;
  PyObject *bufs = PyTuple_Pack(1, buffer);
  PyObject *zero = PyLong_FromLong(0), *one = PyLong_FromLong(1);
  int bad = !bufs || !zero || !one || dset(d_in_buffer, n, buffer) || dset(d_shape, n, shape) ||
            dset(d_dtype, n, dtype) || dset(d_in_strides, n, strides) ||
            dset(d_in_offset, n, offset) || dset(d_depth, n, zero) || dset(d_buffers, n, bufs) ||
            dset(d_nleaves, n, one);
  Py_XDECREF(bufs);
  Py_XDECREF(zero);
  Py_XDECREF(one);
  if (bad) {
    Py_DECREF(n);
    return nullptr;
  }
  return n;
}

PyObject *new_cast(PyObject *input, PyObject *dtype) {
  PyObject *n = alloc_slots(T_cast);
  if (!n) return nullptr;
  PyObject *shape = dget(d_shape, input), *depth = dget(d_depth, input),
           *bufs = dget(d_buffers, input), *nl = dget(d_nleaves, input);
  int bad = !shape || !depth || !bufs || !nl || dset(d_cast_input, n, input) ||
            dset(d_shape, n, shape) || dset(d_dtype, n, dtype) || dset(d_depth, n, depth) ||
            dset(d_buffers, n, bufs) || dset(d_nleaves, n, nl);
  Py_XDECREF(shape);
  Py_XDECREF(depth);
  Py_XDECREF(bufs);
  Py_XDECREF(nl);
  if (bad) {
    Py_DECREF(n);
    return nullptr;
  }
  return n;
}

PyObject *new_unary(PyObject *op, PyObject *input, PyObject *shape, PyObject *dtype) {
  PyObject *n = alloc_slots(T_unary);
  if (!n) return nullptr;
  const long long dep = dget_ll(d_depth, input);
  PyObject *depth = PyLong_FromLongLong(dep + 1);
  PyObject *bufs = dget(d_buffers, input), *nl = dget(d_nleaves, input);
  int bad = !depth || !bufs || !nl || dset(d_un_op, n, op) || dset(d_un_input, n, input) ||
            dset(d_shape, n, shape) || dset(d_dtype, n, dtype) || dset(d_depth, n, depth) ||
            dset(d_buffers, n, bufs) || dset(d_nleaves, n, nl);
  Py_XDECREF(depth);
  Py_XDECREF(bufs);
  Py_XDECREF(nl);
  if (bad) {
    Py_DECREF(n);
    return nullptr;
  }
  return n;
}

PyObject *merge_buffers(PyObject *a, PyObject *b) {  // tuples; identity dedup, order kept
  const Py_ssize_t na = PyTuple_GET_SIZE(a), nb = PyTuple_GET_SIZE(b);
  std::vector<PyObject *> out;
  out.reserve(na + nb);
  for (Py_ssize_t i = 0; i < na + nb; ++i) {
    PyObject *x = i < na ? PyTuple_GET_ITEM(a, i) : PyTuple_GET_ITEM(b, i - na);
    bool seen = false;
    for (PyObject *y : out) seen = seen || y == x;
    if (!seen) out.push_back(x);
  }
  PyObject *t = PyTuple_New((Py_ssize_t)out.size());
  if (!t) return nullptr;
  for (size_t i = 0; i < out.size(); ++i) {
    Py_INCREF(out[i]);
    PyTuple_SET_ITEM(t, (Py_ssize_t)i, out[i]);
  }
  return t;
}

PyObject *new_binary(PyObject *op, PyObject *lhs, PyObject *rhs, PyObject *shape, PyObject *dtype) {
  PyObject *n = alloc_slots(T_binary);
  if (!n) return nullptr;
  const long long da = dget_ll(d_depth, lhs), db = dget_ll(d_depth, rhs);
  const long long la = dget_ll(d_nleaves, lhs), lb = dget_ll(d_nleaves, rhs);
  PyObject *depth = PyLong_FromLongLong((da > db ? da : db) + 1);
  PyObject *nl = PyLong_FromLongLong(la + lb);
  PyObject *ba = dget(d_buffers, lhs), *bb = dget(d_buffers, rhs);
  PyObject *bufs = (ba && bb) ? merge_buffers(ba, bb) : nullptr;
  int bad = !depth || !nl || !bufs || dset(d_bin_op, n, op) || dset(d_bin_lhs, n, lhs) ||
            dset(d_bin_rhs, n, rhs) || dset(d_shape, n, shape) || dset(d_dtype, n, dtype) ||
            dset(d_depth, n, depth) || dset(d_buffers, n, bufs) || dset(d_nleaves, n, nl);
  Py_XDECREF(depth);
  Py_XDECREF(nl);
  Py_XDECREF(ba);
  Py_XDECREF(bb);
  Py_XDECREF(bufs);
  if (bad) {
    Py_DECREF(n);
    return nullptr;
  }
  return n;
}

PyObject *new_scalar(unsigned long long bits, PyObject *dtype) {
  PyObject *n = alloc_slots(T_scalar);
  if (!n) return nullptr;
  PyObject *shape = PyTuple_New(0), *zero = PyLong_FromLong(0), *bufs = PyTuple_New(0);
  PyObject *b = PyLong_FromUnsignedLongLong(bits);
  int bad = !shape || !zero || !bufs || !b || dset(d_sc_bits, n, b) || dset(d_dtype, n, dtype) ||
            dset(d_shape, n, shape) || dset(d_depth, n, zero) || dset(d_buffers, n, bufs) ||
            dset(d_nleaves, n, zero);
  Py_XDECREF(shape);
  Py_XDECREF(zero);
  Py_XDECREF(bufs);
  Py_XDECREF(b);
  if (bad) {
    Py_DECREF(n);
    return nullptr;
  }
  return n;
}

// Lazy result array around `node` (ndarray._lazy) registered with the
// buffers it reads (track_lazy).
PyObject *new_lazy_array(PyObject *node, PyObject *shape, PyObject *dtype) {
  PyObject *arr = T_ndarray->tp_alloc(T_ndarray, 0);
  if (!arr) return nullptr;
  PyObject *d = PyDict_New();
  PyObject *strides = contig_strides(shape);
  PyObject *zero = PyLong_FromLong(0);
  if (!d || !strides || !zero) {
    Py_XDECREF(d);
    Py_XDECREF(strides);
    Py_XDECREF(zero);
    Py_DECREF(arr);
    return nullptr;
  }
  PyObject **dp = _PyObject_GetDictPtr(arr);
  *dp = d;
  int bad = PyDict_SetItem(d, s_buffer, Py_None) || PyDict_SetItem(d, s_np_data, Py_None) ||
            PyDict_SetItem(d, s_shape, shape) || PyDict_SetItem(d, s_dtype, dtype) ||
            PyDict_SetItem(d, s_strides, strides) || PyDict_SetItem(d, s_offset, zero) ||
            PyDict_SetItem(d, s_base, Py_None) || PyDict_SetItem(d, s_fnode, node);
  Py_DECREF(strides);
  Py_DECREF(zero);
  if (bad) {
    Py_DECREF(arr);
    return nullptr;
  }
  // track_lazy
  PyObject *bufs = dget(d_buffers, node);
  if (!bufs) {
    Py_DECREF(arr);
    return nullptr;
  }
  PyObject *ref = PyWeakref_NewRef(arr, nullptr);
  if (!ref) {
    Py_DECREF(bufs);
    Py_DECREF(arr);
    return nullptr;
  }
  for (Py_ssize_t i = 0; i < PyTuple_GET_SIZE(bufs); ++i) {
    PyObject *b = PyTuple_GET_ITEM(bufs, i);
    if (Py_TYPE(b) != &DevBufType) continue;
    DevBuf *db = (DevBuf *)b;
    if (!db->lazy_dependents) {
      db->lazy_dependents = PyList_New(1);
      if (!db->lazy_dependents) {
        bad = 1;
        break;
      }
      Py_INCREF(ref);
      PyList_SET_ITEM(db->lazy_dependents, 0, ref);
      continue;
    }
    if (PyList_Append(db->lazy_dependents, ref)) {
      bad = 1;
      break;
    }
    if (PyList_GET_SIZE(db->lazy_dependents) > 64) {
      PyObject *r = PyObject_CallOneArg(py_prune, db->lazy_dependents);
      if (!r) {
        bad = 1;
        break;
      }
      Py_DECREF(r);
    }
  }
  Py_DECREF(ref);
  Py_DECREF(bufs);
  if (bad) {
    Py_DECREF(arr);
    return nullptr;
  }
  return arr;
}

int check_status(int st, const char *what) {
  if (st == 0) return 0;
  PyObject *r = PyObject_CallFunction(py_check, "is", st, what);
  Py_XDECREF(r);
  if (!PyErr_Occurred()) PyErr_Format(PyExc_RuntimeError, "%s failed (status %d)", what, st);
  return -1;
}

PyObject *new_devbuf(long long nbytes) {
  void *p = nullptr;
  if (check_status(p_alloc((size_t)(nbytes > 0 ? nbytes : 1), &p), "mmp_alloc")) return nullptr;
  DevBuf *b = PyObject_New(DevBuf, &DevBufType);
  if (!b) {
    p_free(p);
    return nullptr;
  }
  b->ptr = (unsigned long long)(uintptr_t)p;
  b->nbytes = nbytes;
  b->owned = 1;
  b->lazy_dependents = nullptr;
  b->weakreflist = nullptr;
  return (PyObject *)b;
}

// Host-resident ndarray (dict `xd`, `_np_data` set): upload its data into a
// new device buffer and make the array device-resident in place, as
// ndarray._ensure_gpu does (reference ndarray.py:352-368, where the first
// GPU use of an array created from NumPy data copies it into the shared
// buffer).  The data must be C-contiguous with the array's item size;
// mmp_h2d stages small copies through page-locked memory and returns
// without waiting for the device.  1 = uploaded, 0 = not handled here (the
// Python path uploads), -1 = error.
int upload_host(PyObject *xd) {
  PyObject *np = iget(xd, s_np_data), *dtype = iget(xd, s_dtype), *shape = iget(xd, s_shape);
  if (!np || np == Py_None || !dtype || !shape) return 0;
  if (!p_h2d) {  // the device is not set up yet: set it up (that binds the library)
    PyObject *r = PyObject_CallNoArgs(py_ensure_device);
    if (!r) return -1;
    Py_DECREF(r);
    if (!p_h2d) return 0;
  }
  const int dt = dtype_index(dtype);
  long long n = 0;
  if (dt < 0 || !shape_size(shape, &n)) return 0;
  Py_buffer view;
  if (PyObject_GetBuffer(np, &view, PyBUF_C_CONTIGUOUS) != 0) {  // strided data: Python copies
    PyErr_Clear();
    return 0;
  }
  const long long bytes = n * itemsize[dt];
  if (view.len != bytes || view.itemsize != itemsize[dt]) {
    PyBuffer_Release(&view);
    return 0;
  }
  PyObject *buf = new_devbuf(bytes);
  if (!buf) {
    PyBuffer_Release(&view);
    return -1;
  }
  const int st =
      bytes ? p_h2d((void *)(uintptr_t)((DevBuf *)buf)->ptr, view.buf, (size_t)bytes) : 0;
  PyBuffer_Release(&view);
  if (check_status(st, "mmp_h2d")) {
    Py_DECREF(buf);
    return -1;
  }
  PyObject *strides = contig_strides(shape), *zero = PyLong_FromLong(0);
  const int bad = !strides || !zero || PyDict_SetItem(xd, s_buffer, buf) ||
                  PyDict_SetItem(xd, s_np_data, Py_None) || PyDict_SetItem(xd, s_strides, strides) ||
                  PyDict_SetItem(xd, s_offset, zero);
  Py_XDECREF(strides);
  Py_XDECREF(zero);
  Py_DECREF(buf);
  if (bad) return -1;
  ++stat_uploads;
  return 1;
}

// Operand node of ndarray `x` (dict `xd`) read as dtype index `want`:
// 1 = ok (*out new ref), 0 = not handled here (fall back), -1 = error.
int operand_node(PyObject *xd, int want, PyObject **out) {
  PyObject *node = iget(xd, s_fnode);
  PyObject *dtype = iget(xd, s_dtype);
  if (!dtype) return 0;
  if (node && node != Py_None) {
    if (Py_TYPE(node) != T_input && Py_TYPE(node) != T_unary && Py_TYPE(node) != T_binary &&
        Py_TYPE(node) != T_cast && Py_TYPE(node) != T_scalar && Py_TYPE(node) != T_where)
      return 0;
    const long long dep = dget_ll(d_depth, node), nl = dget_ll(d_nleaves, node);
    if (dep < 0 || nl < 0) {
      PyErr_Clear();
      return 0;
    }
    if (dep + 1 > max_depth || nl > max_leaves) return 0;  // Python materialises first
    Py_INCREF(node);
  } else {
    PyObject *np = iget(xd, s_np_data);
    if (np && np != Py_None) {
      const int up = upload_host(xd);
      if (up <= 0) return up;
    }
    PyObject *buf = iget(xd, s_buffer);
    if (!buf || buf == Py_None) return 0;
    PyObject *shape = iget(xd, s_shape), *strides = iget(xd, s_strides), *off = iget(xd, s_offset);
    if (!shape || !strides || !off) return 0;
    node = new_input(buf, shape, dtype, strides, off);
    if (!node) return -1;
  }
  PyObject *ndt = dget(d_dtype, node);
  if (!ndt) {
    Py_DECREF(node);
    return -1;
  }
  const bool same = ndt == dtypes[want];
  Py_DECREF(ndt);
  if (!same) {
    PyObject *c = new_cast(node, dtypes[want]);
    Py_DECREF(node);
    if (!c) return -1;
    node = c;
  }
  *out = node;
  return 1;
}

int op_id_of(PyObject *op) {
  PyObject *v = PyDict_GetItem(op_ids, op);
  return v ? (int)PyLong_AsLong(v) : -1;
}

PyObject *fallback2(PyObject *fn, PyObject *a, PyObject *b) {
  ++stat_fallback;
  PyObject *args[2] = {a, b};
  return PyObject_Vectorcall(fn, args, 2, nullptr);
}

PyObject *fallback3(PyObject *fn, PyObject *a, PyObject *b, PyObject *c) {
  ++stat_fallback;
  PyObject *args[3] = {a, b, c};
  return PyObject_Vectorcall(fn, args, 3, nullptr);
}

// ------------------------------------------------------------- unary
PyObject *gate_unary(PyObject *, PyObject *const *args, Py_ssize_t nargs) {
  if (nargs != 2) {
    PyErr_SetString(PyExc_TypeError, "unary(op_name, x)");
    return nullptr;
  }
  PyObject *op = args[0], *x = args[1];
  if (Py_TYPE(x) != T_ndarray || !cfg_flag(s_fusion)) return fallback2(py_unary_fb, op, x);
  const int id = op_id_of(op);
  PyObject *xd = inst_dict(x);
  PyObject *dtype = iget(xd, s_dtype), *shape = iget(xd, s_shape);
  const int di = dtype ? dtype_index(dtype) : -1;
  long long n = 0;
  if (id < 0 || di < 0 || !shape || !shape_size(shape, &n) || n == 0)
    return fallback2(py_unary_fb, op, x);
  if (un_rdt[id][di] < 0) {
    PyObject *r = PyObject_CallFunctionObjArgs(py_unary_dt, op, dtype, nullptr);
    if (!r) {
      PyErr_Clear();
      return fallback2(py_unary_fb, op, x);
    }
    const int rd = PyTuple_Check(r) && PyTuple_GET_SIZE(r) == 2 ? dtype_index(PyTuple_GET_ITEM(r, 0)) : -1;
    const int id2 = rd >= 0 ? dtype_index(PyTuple_GET_ITEM(r, 1)) : -1;
    Py_DECREF(r);
    if (rd < 0 || id2 < 0) return fallback2(py_unary_fb, op, x);
    un_rdt[id][di] = (int8_t)rd;
    un_idt[id][di] = (int8_t)id2;
  }
  PyObject *in = nullptr;
  const int st = operand_node(xd, un_idt[id][di], &in);
  if (st < 0) return nullptr;
  if (st == 0) return fallback2(py_unary_fb, op, x);
  PyObject *rdt = dtypes[un_rdt[id][di]];
  PyObject *node = new_unary(op, in, shape, rdt);
  Py_DECREF(in);
  if (!node) return nullptr;
  PyObject *arr = new_lazy_array(node, shape, rdt);
  Py_DECREF(node);
  ++stat_native_ops;
  return arr;
}

// Python int / float operand: kind 0 float, 1 int; false if not handled.
bool scalar_kind(PyObject *v, int *kind) {
  if (PyFloat_CheckExact(v)) {
    *kind = 0;
    return true;
  }
  if (PyLong_CheckExact(v)) {
    *kind = 1;
    return true;
  }
  return false;
}

// Bits of Python scalar `v` converted to dtype index `dt` (NumPy's
// conversion of an in-range value); false if not handled here.
bool scalar_bits(PyObject *v, int kind, int dt, unsigned long long *bits) {
  if (kind == 0) {
    const double d = PyFloat_AS_DOUBLE(v);
    if (dt == D_F64) {
      std::memcpy(bits, &d, 8);
      return true;
    }
    if (dt == D_F32) {
      const float f = (float)d;
      unsigned u;
      std::memcpy(&u, &f, 4);
      *bits = u;
      return true;
    }
    return false;  // float16 (and int targets) through Python
  }
  int overflow = 0;
  const long long x = PyLong_AsLongLongAndOverflow(v, &overflow);
  if (overflow || (x == -1 && PyErr_Occurred())) {
    PyErr_Clear();
    return false;
  }
  switch (dt) {
    case D_F64: {
      if (x > (1LL << 53) || x < -(1LL << 53)) return false;
      const double d = (double)x;
      std::memcpy(bits, &d, 8);
      return true;
    }
    case D_F32: {
      if (x > (1LL << 24) || x < -(1LL << 24)) return false;
      const float f = (float)x;
      unsigned u;
      std::memcpy(&u, &f, 4);
      *bits = u;
      return true;
    }
    case D_I16:
      if (x < -32768 || x > 32767) return false;
      *bits = (unsigned long long)(uint16_t)(int16_t)x;
      return true;
    case D_U16:
      if (x < 0 || x > 65535) return false;
      *bits = (unsigned long long)x;
      return true;
    case D_I32:
      if (x < -2147483648LL || x > 2147483647LL) return false;
      *bits = (unsigned long long)(uint32_t)(int32_t)x;
      return true;
    case D_U32:
      if (x < 0 || x > 4294967295LL) return false;
      *bits = (unsigned long long)x;
      return true;
    case D_I64:
      *bits = (unsigned long long)x;
      return true;
    case D_U64:
      if (x < 0) return false;
      *bits = (unsigned long long)x;
      return true;
    default:
      return false;
  }
}

// NumPy broadcasting of two shape tuples; NULL (exception set) if they
// do not broadcast.
PyObject *broadcast_shape(PyObject *sa, PyObject *sb) {
  const Py_ssize_t na = PyTuple_GET_SIZE(sa), nb = PyTuple_GET_SIZE(sb);
  const Py_ssize_t nd = na > nb ? na : nb;
  PyObject *t = PyTuple_New(nd);
  if (!t) return nullptr;
  for (Py_ssize_t i = 0; i < nd; ++i) {
    const Py_ssize_t ia = i - (nd - na), ib = i - (nd - nb);
    const long long x = ia >= 0 ? PyLong_AsLongLong(PyTuple_GET_ITEM(sa, ia)) : 1;
    const long long y = ib >= 0 ? PyLong_AsLongLong(PyTuple_GET_ITEM(sb, ib)) : 1;
    if (x != y && x != 1 && y != 1) {
      Py_DECREF(t);
      PyErr_SetString(PyExc_ValueError, "shapes do not broadcast");
      return nullptr;
    }
    PyObject *v = PyLong_FromLongLong(x == 1 ? y : x);
    if (!v) {
      Py_DECREF(t);
      return nullptr;
    }
    PyTuple_SET_ITEM(t, i, v);
  }
  return t;
}

// ------------------------------------------------------------- binary
PyObject *gate_binary(PyObject *, PyObject *const *args, Py_ssize_t nargs) {
  if (nargs != 3) {
    PyErr_SetString(PyExc_TypeError, "binary(op_name, a, b)");
    return nullptr;
  }
  PyObject *op = args[0], *a = args[1], *b = args[2];
  if (!cfg_flag(s_fusion)) return fallback3(py_binary_fb, op, a, b);
  const int id = op_id_of(op);
  const bool a_arr = Py_TYPE(a) == T_ndarray, b_arr = Py_TYPE(b) == T_ndarray;
  if (id < 0 || (!a_arr && !b_arr)) return fallback3(py_binary_fb, op, a, b);
  if (a_arr && b_arr) {
    PyObject *ad = inst_dict(a), *bd = inst_dict(b);
    PyObject *dta = iget(ad, s_dtype), *dtb = iget(bd, s_dtype);
    PyObject *sa = iget(ad, s_shape), *sb = iget(bd, s_shape);
    const int ia = dta ? dtype_index(dta) : -1, ib = dtb ? dtype_index(dtb) : -1;
    long long n = 0;
    if (ia < 0 || ib < 0 || !sa || !sb || !shape_size(sa, &n) || n == 0)
      return fallback3(py_binary_fb, op, a, b);
    PyObject *shape = sa;  // borrowed, or the new broadcast shape below
    PyObject *bshape = nullptr;
    if (sa != sb) {
      const int eq = PyObject_RichCompareBool(sa, sb, Py_EQ);
      if (eq < 0) return nullptr;
      if (!eq) {
        bshape = broadcast_shape(sa, sb);
        if (!bshape) {
          PyErr_Clear();  // incompatible: Python raises NumPy's error
          return fallback3(py_binary_fb, op, a, b);
        }
        if (!shape_size(bshape, &n) || n == 0) {
          Py_DECREF(bshape);
          return fallback3(py_binary_fb, op, a, b);
        }
        shape = bshape;
      }
    }
    if (bin_rdt[id][ia][ib] < 0) {
      PyObject *r = PyObject_CallFunctionObjArgs(py_binary_dt, op, dta, dtb, nullptr);
      if (!r) {
        PyErr_Clear();
        return fallback3(py_binary_fb, op, a, b);
      }
      const int rd = PyTuple_Check(r) && PyTuple_GET_SIZE(r) == 2 ? dtype_index(PyTuple_GET_ITEM(r, 0)) : -1;
      const int od = rd >= 0 ? dtype_index(PyTuple_GET_ITEM(r, 1)) : -1;
      Py_DECREF(r);
      if (rd < 0 || od < 0) return fallback3(py_binary_fb, op, a, b);
      bin_rdt[id][ia][ib] = (int8_t)rd;
      bin_odt[id][ia][ib] = (int8_t)od;
    }
    const int rd = bin_rdt[id][ia][ib], od = bin_odt[id][ia][ib];
    PyObject *an = nullptr, *bn = nullptr, *node = nullptr, *arr = nullptr;
    int st;
    // integer powers need the host's negative-exponent check
    if (binary_code[id] == 6 && rd != D_F16 && rd != D_F32 && rd != D_F64) goto back;
    st = operand_node(ad, od, &an);
    if (st <= 0) {
      if (st < 0) goto err;
      goto back;
    }
    st = operand_node(bd, od, &bn);
    if (st <= 0) {
      if (st < 0) goto err;
      goto back;
    }
    if (dget_ll(d_nleaves, an) + dget_ll(d_nleaves, bn) > max_leaves) goto back;
    node = new_binary(op, an, bn, shape, dtypes[rd]);
    if (!node) goto err;
    arr = new_lazy_array(node, shape, dtypes[rd]);
    Py_DECREF(node);
    Py_XDECREF(an);
    Py_XDECREF(bn);
    Py_XDECREF(bshape);
    if (arr) ++stat_native_ops;
    return arr;
  back:
    Py_XDECREF(an);
    Py_XDECREF(bn);
    Py_XDECREF(bshape);
    return fallback3(py_binary_fb, op, a, b);
  err:
    Py_XDECREF(an);
    Py_XDECREF(bn);
    Py_XDECREF(bshape);
    return nullptr;
  }
  // one array and a Python int / float
  PyObject *arr_o = a_arr ? a : b, *sc = a_arr ? b : a;
  int kind = 0;
  if (!scalar_kind(sc, &kind)) return fallback3(py_binary_fb, op, a, b);
  PyObject *xd = inst_dict(arr_o);
  PyObject *dt = iget(xd, s_dtype), *shape = iget(xd, s_shape);
  const int di = dt ? dtype_index(dt) : -1;
  long long n = 0;
  if (di < 0 || di == D_BOOL || !shape || !shape_size(shape, &n) || n == 0)
    return fallback3(py_binary_fb, op, a, b);
  const int side = a_arr ? 1 : 0;
  if (bsc_rdt[id][di][kind][side] < 0) {
    // the result dtype of an array with a weak Python scalar does not depend
    // on the scalar's value once the value fits (checked per call below)
    PyObject *sample = kind ? PyLong_FromLong(1) : PyFloat_FromDouble(1.0);
    if (!sample) return nullptr;
    PyObject *r = side ? PyObject_CallFunctionObjArgs(py_binary_dt, op, dt, sample, nullptr)
                       : PyObject_CallFunctionObjArgs(py_binary_dt, op, sample, dt, nullptr);
    Py_DECREF(sample);
    if (!r) {
      PyErr_Clear();
      return fallback3(py_binary_fb, op, a, b);
    }
    const int rd = PyTuple_Check(r) && PyTuple_GET_SIZE(r) == 2 ? dtype_index(PyTuple_GET_ITEM(r, 0)) : -1;
    const int od = rd >= 0 ? dtype_index(PyTuple_GET_ITEM(r, 1)) : -1;
    Py_DECREF(r);
    if (rd < 0 || od < 0) return fallback3(py_binary_fb, op, a, b);
    bsc_rdt[id][di][kind][side] = (int8_t)rd;
    bsc_odt[id][di][kind][side] = (int8_t)od;
  }
  const int rd = bsc_rdt[id][di][kind][side], od = bsc_odt[id][di][kind][side];
  if (binary_code[id] == 6 && rd != D_F16 && rd != D_F32 && rd != D_F64)
    return fallback3(py_binary_fb, op, a, b);
  // an int scalar with an int array keeps the array dtype only if it fits;
  // scalar_bits refuses what does not fit (Python raises NumPy's error)
  unsigned long long bits = 0;
  if (!scalar_bits(sc, kind, od, &bits)) return fallback3(py_binary_fb, op, a, b);
  PyObject *an = nullptr;
  const int st = operand_node(xd, od, &an);
  if (st <= 0) {
    if (st < 0) return nullptr;
    return fallback3(py_binary_fb, op, a, b);
  }
  PyObject *sn = new_scalar(bits, dtypes[od]);
  if (!sn) {
    Py_DECREF(an);
    return nullptr;
  }
  PyObject *node = a_arr ? new_binary(op, an, sn, shape, dtypes[rd])
                         : new_binary(op, sn, an, shape, dtypes[rd]);
  Py_DECREF(an);
  Py_DECREF(sn);
  if (!node) return nullptr;
  PyObject *res = new_lazy_array(node, shape, dtypes[rd]);
  Py_DECREF(node);
  ++stat_native_ops;
  return res;
}

// ---------------------------------------------------------- materialize
struct Leaf {
  PyObject *node;  // InputNode (borrowed: kept alive by the DAG)
  unsigned long long ptr;
  int dt;
  std::vector<long long> shape, strides;
};

struct Prog {
  std::vector<Leaf> leaves;
  std::vector<unsigned long long> sbits;
  std::string key;                                  // structure of the steps
  std::vector<std::pair<PyObject *, int>> memo;     // node -> SSA index
  int nsteps = 0;
  bool ok = true;
};

bool tuple_ll(PyObject *t, std::vector<long long> *out) {
  if (!PyTuple_CheckExact(t)) return false;
  out->resize(PyTuple_GET_SIZE(t));
  for (Py_ssize_t i = 0; i < PyTuple_GET_SIZE(t); ++i) {
    (*out)[i] = PyLong_AsLongLong(PyTuple_GET_ITEM(t, i));
    if ((*out)[i] == -1 && PyErr_Occurred()) return false;
  }
  return true;
}

inline void put16(std::string *k, int v) {
  k->push_back((char)(v & 0xff));
  k->push_back((char)((v >> 8) & 0xff));
}

// Post-order SSA numbering with leaves deduplicated by (buffer, offset,
// strides, shape, dtype) -- the traversal of the Python _Program.
int visit(Prog &p, PyObject *node) {
  for (auto &m : p.memo)
    if (m.first == node) return m.second;
  if (!p.ok) return -1;
  PyTypeObject *t = Py_TYPE(node);
  PyObject *dto = dget(d_dtype, node);
  const int dt = dto ? dtype_index(dto) : -1;
  Py_XDECREF(dto);
  if (dt < 0) {
    p.ok = false;
    return -1;
  }
  std::string &k = p.key;
  if (t == T_input) {
    PyObject *buf = dget(d_in_buffer, node);
    PyObject *shp = dget(d_shape, node), *str = dget(d_in_strides, node);
    const long long off = dget_ll(d_in_offset, node);
    Leaf L;
    L.node = node;
    L.dt = dt;
    bool good = buf && Py_TYPE(buf) == &DevBufType && shp && str && off >= 0 &&
                tuple_ll(shp, &L.shape) && tuple_ll(str, &L.strides);
    if (good) L.ptr = ((DevBuf *)buf)->ptr + (unsigned long long)off * itemsize[dt];
    Py_XDECREF(buf);
    Py_XDECREF(shp);
    Py_XDECREF(str);
    if (!good) {
      PyErr_Clear();
      p.ok = false;
      return -1;
    }
    int li = -1;
    for (size_t i = 0; i < p.leaves.size(); ++i) {
      const Leaf &o = p.leaves[i];
      if (o.ptr == L.ptr && o.dt == L.dt && o.shape == L.shape && o.strides == L.strides) {
        // same buffer object too (pointer equality of the view start plus
        // equal layout is what the Python key compares, via id(buffer) and
        // the offset)
        PyObject *b1 = dget(d_in_buffer, o.node), *b2 = dget(d_in_buffer, node);
        const bool same = b1 == b2;
        Py_XDECREF(b1);
        Py_XDECREF(b2);
        if (same) {
          li = (int)i;
          break;
        }
      }
    }
    if (li < 0) {
      li = (int)p.leaves.size();
      p.leaves.push_back(std::move(L));
    }
    k.push_back('L');
    put16(&k, li);
  } else if (t == T_scalar) {
    PyObject *b = dget(d_sc_bits, node);
    if (!b) {
      PyErr_Clear();
      p.ok = false;
      return -1;
    }
    p.sbits.push_back(PyLong_AsUnsignedLongLongMask(b));
    Py_DECREF(b);
    k.push_back('S');
    put16(&k, (int)p.sbits.size() - 1);
  } else if (t == T_cast) {
    PyObject *in = dget(d_cast_input, node);
    const int a = in ? visit(p, in) : -1;
    Py_XDECREF(in);
    k.push_back('C');
    put16(&k, a);
  } else if (t == T_unary) {
    PyObject *op = dget(d_un_op, node), *in = dget(d_un_input, node);
    const int oid = op ? op_id_of(op) : -1;
    const int a = (in && oid >= 0) ? visit(p, in) : -1;
    Py_XDECREF(op);
    Py_XDECREF(in);
    if (oid < 0) p.ok = false;
    k.push_back('U');
    put16(&k, oid);
    put16(&k, a);
  } else if (t == T_binary) {
    PyObject *op = dget(d_bin_op, node), *l = dget(d_bin_lhs, node), *r = dget(d_bin_rhs, node);
    const int oid = op ? op_id_of(op) : -1;
    const int a = (l && oid >= 0) ? visit(p, l) : -1;
    const int b = (r && oid >= 0) ? visit(p, r) : -1;
    Py_XDECREF(op);
    Py_XDECREF(l);
    Py_XDECREF(r);
    if (oid < 0) p.ok = false;
    k.push_back('B');
    put16(&k, oid);
    put16(&k, a);
    put16(&k, b);
  } else if (t == T_where) {
    PyObject *c = dget(d_wh_cond, node), *x = dget(d_wh_x, node), *y = dget(d_wh_y, node);
    const int a = c ? visit(p, c) : -1;
    const int b = x ? visit(p, x) : -1;
    const int e = y ? visit(p, y) : -1;
    Py_XDECREF(c);
    Py_XDECREF(x);
    Py_XDECREF(y);
    k.push_back('W');
    put16(&k, a);
    put16(&k, b);
    put16(&k, e);
  } else {
    p.ok = false;
    return -1;
  }
  k.push_back((char)dt);
  const int idx = p.nsteps++;
  p.memo.emplace_back(node, idx);
  return idx;
}

// Collapse the iteration space (the Python _collapse): merge adjacent dims
// contiguous for every operand, drop size-1 dims; with keep_last the last
// dim stays separate (the reduced axis of a row reduction).
void collapse(const std::vector<long long> &shape, std::vector<std::vector<long long>> &st,
              bool keep_last, std::vector<long long> *cshape,
              std::vector<std::vector<long long>> *cst) {
  cshape->clear();
  cst->assign(st.size(), {});
  const size_t n = shape.size();
  for (size_t d = 0; d < n; ++d) {
    const bool is_last = keep_last && d == n - 1;
    if (shape[d] == 1 && !is_last) continue;
    bool merge = !cshape->empty() && !is_last;
    for (size_t k = 0; merge && k < st.size(); ++k)
      merge = (*cst)[k].back() == st[k][d] * shape[d];
    if (merge) {
      cshape->back() *= shape[d];
      for (size_t k = 0; k < st.size(); ++k) (*cst)[k].back() = st[k][d];
    } else {
      cshape->push_back(shape[d]);
      for (size_t k = 0; k < st.size(); ++k) (*cst)[k].push_back(st[k][d]);
    }
  }
}

bool contig_leaf(PyObject *n, PyObject *shape, int dt) {
  if (Py_TYPE(n) != T_input) return false;
  PyObject *dto = dget(d_dtype, n), *shp = dget(d_shape, n), *str = dget(d_in_strides, n);
  bool ok = dto && shp && str && dto == dtypes[dt];
  if (ok) {
    const int eq = shp == shape ? 1 : PyObject_RichCompareBool(shp, shape, Py_EQ);
    ok = eq == 1 && is_contig(shp, str);
  }
  Py_XDECREF(dto);
  Py_XDECREF(shp);
  Py_XDECREF(str);
  if (PyErr_Occurred()) PyErr_Clear();
  return ok;
}

unsigned long long leaf_ptr(PyObject *n, int dt) {
  PyObject *buf = dget(d_in_buffer, n);
  const long long off = dget_ll(d_in_offset, n);
  unsigned long long p = 0;
  if (buf && Py_TYPE(buf) == &DevBufType) p = ((DevBuf *)buf)->ptr + (unsigned long long)off * itemsize[dt];
  Py_XDECREF(buf);
  return p;
}

// Finish: the array now views `buf` (contiguous).
int finish(PyObject *arr, PyObject *arrd, PyObject *buf, PyObject *shape) {
  PyObject *strides = contig_strides(shape);
  PyObject *zero = PyLong_FromLong(0);
  int bad = !strides || !zero || PyDict_SetItem(arrd, s_buffer, buf) ||
            PyDict_SetItem(arrd, s_fnode, Py_None) || PyDict_SetItem(arrd, s_np_data, Py_None) ||
            PyDict_SetItem(arrd, s_offset, zero) || PyDict_SetItem(arrd, s_strides, strides);
  Py_XDECREF(strides);
  Py_XDECREF(zero);
  (void)arr;
  return bad ? -1 : 0;
}

constexpr int kBlock = 256;

// Linearised program plus its iteration plan (the Python _Program + _plan).
struct Plan {
  Prog p;
  std::vector<long long> cshape;
  std::vector<std::vector<long long>> cst;  // collapsed strides per leaf
  std::string kinds;                        // last-dim stride class per leaf
  long long cols = 1, rows = 1;
  size_t nouter = 0;
};

// Elements per workgroup of a generated map kernel: 1024 for a single
// contiguous leaf, else 4096 -- the rule of _fusion._map_unroll, which
// generates the kernel (its tile must match the launch).
long long map_tile(const std::string &kinds) {
  return kinds == "c" ? 256 * 4 * 1 : 256 * 4 * 4;
}

// 1 = planned, 0 = not handled here (fall back), -1 = error set.
int make_plan(PyObject *root, PyObject *shape, bool keep_last, Plan *pl) {
  Prog &p = pl->p;
  p.key.reserve(128);
  visit(p, root);
  if (!p.ok || PyErr_Occurred()) {
    PyErr_Clear();
    return 0;
  }
  std::vector<long long> oshape;
  if (!tuple_ll(shape, &oshape)) return -1;
  const size_t nin = p.leaves.size();
  std::vector<std::vector<long long>> st(nin + 1);
  for (size_t k = 0; k < nin; ++k) {
    const Leaf &L = p.leaves[k];
    if (L.shape.size() > oshape.size()) return 0;
    const size_t diff = oshape.size() - L.shape.size();
    st[k].assign(diff, 0);
    for (size_t d = 0; d < L.shape.size(); ++d) {
      const long long sz = L.shape[d], tt = oshape[diff + d];
      st[k].push_back((sz == tt && sz != 1) ? L.strides[d] : 0);
    }
  }
  st[nin].assign(oshape.size(), 0);
  long long acc = 1;
  for (size_t d = oshape.size(); d-- > 0;) {
    st[nin][d] = acc;
    acc *= oshape[d];
  }
  collapse(oshape, st, keep_last, &pl->cshape, &pl->cst);
  pl->cst.resize(nin);  // the output's collapsed strides are not needed
  if (pl->cshape.empty()) {
    pl->cshape.push_back(1);
    for (size_t k = 0; k < nin; ++k) pl->cst[k].assign(1, 0);
  }
  pl->cols = pl->cshape.back();
  pl->nouter = pl->cshape.size() - 1;
  pl->rows = 1;
  for (size_t d = 0; d < pl->nouter; ++d) pl->rows *= pl->cshape[d];
  pl->kinds.clear();
  for (size_t k = 0; k < nin; ++k) {
    const long long ls = pl->cst[k].empty() ? 0 : pl->cst[k].back();
    pl->kinds.push_back(ls == 1 ? 'c' : (ls == 0 ? 'b' : 's'));
  }
  return 1;
}

// Whether every leaf can be read 4 elements at a time with aligned vector
// loads (the Python _vec_ok); `out_ok` covers the output for map mode.
bool vec_ok(const Plan &pl, bool out_ok) {
  if (pl.cols % 4 || !out_ok) return false;
  for (size_t k = 0; k < pl.p.leaves.size(); ++k) {
    if (pl.kinds[k] == 's') return false;
    if (pl.kinds[k] == 'c') {
      if (pl.p.leaves[k].ptr % (4ull * itemsize[pl.p.leaves[k].dt])) return false;
      for (size_t d = 0; d + 1 < pl.cst[k].size(); ++d)
        if (pl.cst[k][d] % 4) return false;
    }
  }
  return true;
}

// Kernel for the plan (mode 'm' map, 's' row sum), by structure; compiled
// through the Python code generator the first time.
void *kernel_for(const Plan &pl, PyObject *root, int out_dt, bool vec, char mode, bool fast) {
  std::string key = pl.p.key;
  key.push_back('|');
  for (const Leaf &L : pl.p.leaves) key.push_back((char)L.dt);
  key += pl.kinds;
  key.push_back((char)pl.nouter);
  key.push_back((char)out_dt);
  key.push_back(vec ? 'v' : 's');
  key.push_back(fast ? 'f' : 'e');
  key.push_back(mode);
  auto it = g_kernels.find(key);
  if (it != g_kernels.end()) return it->second;
  PyObject *kt = PyUnicode_FromStringAndSize(pl.kinds.data(), (Py_ssize_t)pl.kinds.size());
  PyObject *r = kt ? PyObject_CallFunction(py_compile_map, "OOiOOs", root, kt, (int)pl.nouter,
                                           dtypes[out_dt], vec ? Py_True : Py_False,
                                           mode == 'm' ? "map" : "sum")
                   : nullptr;
  Py_XDECREF(kt);
  if (!r) return nullptr;
  void *kern = PyLong_AsVoidPtr(r);
  Py_DECREF(r);
  if (PyErr_Occurred()) return nullptr;
  if (!kern) {
    PyErr_SetString(PyExc_RuntimeError, "null kernel handle");
    return nullptr;
  }
  g_kernels.emplace(key, kern);
  return kern;
}

// Pack the generated kernel's parameter block (struct P: 8-byte fields
// ptr[nin], outp, sbits[nsc], n, rows, cols, colblocks, oshape[nouter],
// ostride[nin * nouter], lstride[nin], scale) and launch rows * colblocks
// workgroups of kBlock threads.  0 or -1 with an exception set.
int launch_plan(const Plan &pl, void *kern, unsigned long long outp, long long colblocks,
                double scale) {
  const size_t nin = pl.p.leaves.size(), nsc = pl.p.sbits.size(), nouter = pl.nouter;
  const size_t nin1 = nin ? nin : 1, nsc1 = nsc ? nsc : 1, nout1 = nouter ? nouter : 1,
               nio1 = (nin * nouter) != 0 ? nin * nouter : 1;
  std::vector<unsigned long long> P(nin1 + 1 + nsc1 + 4 + nout1 + nio1 + nin1 + 1, 0ull);
  size_t o = 0;
  const size_t o_ptr = o; o += nin1;
  const size_t o_out = o; o += 1;
  const size_t o_sb = o; o += nsc1;
  const size_t o_n = o; o += 4;
  const size_t o_osh = o; o += nout1;
  const size_t o_ost = o; o += nio1;
  const size_t o_lst = o; o += nin1;
  const size_t o_scale = o;
  for (size_t k = 0; k < nin; ++k) {
    P[o_ptr + k] = pl.p.leaves[k].ptr;
    P[o_lst + k] = (unsigned long long)(pl.cst[k].empty() ? 0 : pl.cst[k].back());
    for (size_t d = 0; d < nouter; ++d) P[o_ost + k * nouter + d] = (unsigned long long)pl.cst[k][d];
  }
  for (size_t j = 0; j < nsc; ++j) P[o_sb + j] = pl.p.sbits[j];
  for (size_t d = 0; d < nouter; ++d) P[o_osh + d] = (unsigned long long)pl.cshape[d];
  P[o_out] = outp;
  P[o_n + 0] = (unsigned long long)(pl.rows * pl.cols);
  P[o_n + 1] = (unsigned long long)pl.rows;
  P[o_n + 2] = (unsigned long long)pl.cols;
  P[o_n + 3] = (unsigned long long)colblocks;
  std::memcpy(&P[o_scale], &scale, 8);
  const unsigned long long nblocks = (unsigned long long)(pl.rows * colblocks);
  if (nblocks * kBlock > 0xffffffffull) {  // HIP's limit on work-items per grid dimension
    PyErr_SetString(PyExc_ValueError, "fused launch too large");
    return -1;
  }
  if (nblocks == 0) return 0;
  uint32_t grid[3] = {(uint32_t)nblocks, 1, 1}, block[3] = {kBlock, 1, 1};
  void *argv[1] = {P.data()};
  return check_status(p_launch(kern, grid, block, 0, argv), "mmp_rtc_launch");
}

PyObject *gate_materialize(PyObject *, PyObject *arr) {
  if (Py_TYPE(arr) != T_ndarray) return PyObject_CallOneArg(py_materialize_fb, arr);
  PyObject *arrd = inst_dict(arr);
  PyObject *node = iget(arrd, s_fnode);
  if (!node || node == Py_None) Py_RETURN_NONE;
  if (!p_launch) return PyObject_CallOneArg(py_materialize_fb, arr);
  PyTypeObject *t = Py_TYPE(node);
  if (t != T_unary && t != T_binary && t != T_where && t != T_cast)
    return PyObject_CallOneArg(py_materialize_fb, arr);
  Py_INCREF(node);  // the dict entry is replaced below
  PyObject *shape = dget(d_shape, node), *dto = dget(d_dtype, node);
  const int odt = dto ? dtype_index(dto) : -1;
  Py_XDECREF(dto);
  long long n = 0;
  if (!shape || odt < 0 || !shape_size(shape, &n) || n == 0 || t == T_cast) {
    Py_XDECREF(shape);
    Py_DECREF(node);
    PyErr_Clear();
    return PyObject_CallOneArg(py_materialize_fb, arr);
  }
  const bool fast = cfg_flag(s_fast_math);
  PyObject *result = nullptr;
  PyObject *buf = nullptr;
  // ---- one precompiled kernel
  int oid = -1;
  if (t == T_unary || t == T_binary) {
    PyObject *op = dget(t == T_unary ? d_un_op : d_bin_op, node);
    oid = op ? op_id_of(op) : -1;
    Py_XDECREF(op);
  }
  const bool fast_form = fast && oid >= 0 && fast_op[oid] && (odt == D_F32 || odt == D_F16);
  // mmp_unary defines every op for floats, the integer set for integers and
  // nothing for bool; the generated kernel covers the rest
  const bool unary_ok = oid >= 0 && unary_code[oid] >= 0 &&
                        (odt >= D_F16 || (odt != D_BOOL && int_unary_op[oid]));
  if (!fast_form && t == T_unary && unary_ok) {
    PyObject *in = dget(d_un_input, node);
    if (in && contig_leaf(in, shape, odt)) {
      const unsigned long long src = leaf_ptr(in, odt);
      buf = new_devbuf(n * itemsize[odt]);
      if (buf && !check_status(p_unary(unary_code[oid], odt, n, (const void *)(uintptr_t)src,
                                       (void *)(uintptr_t)((DevBuf *)buf)->ptr),
                               "mmp_unary"))
        result = Py_None;
    }
    Py_XDECREF(in);
    if (!result && PyErr_Occurred()) goto fail;
  }
  if (!result && !buf && !fast_form && t == T_binary && oid >= 0 && binary_code[oid] >= 0) {
    PyObject *l = dget(d_bin_lhs, node), *r = dget(d_bin_rhs, node);
    if (l && r) {
      const bool lc = contig_leaf(l, shape, odt), rc = contig_leaf(r, shape, odt);
      PyObject *ldt = dget(d_dtype, l), *rdt = dget(d_dtype, r);
      const bool ls = Py_TYPE(l) == T_scalar && ldt == dtypes[odt];
      const bool rs = Py_TYPE(r) == T_scalar && rdt == dtypes[odt];
      Py_XDECREF(ldt);
      Py_XDECREF(rdt);
      if ((lc && rc) || (lc && rs) || (ls && rc)) {
        buf = new_devbuf(n * itemsize[odt]);
        if (buf) {
          void *out = (void *)(uintptr_t)((DevBuf *)buf)->ptr;
          int st;
          if (lc && rc) {
            st = p_binary(binary_code[oid], odt, n, (const void *)(uintptr_t)leaf_ptr(l, odt),
                          (const void *)(uintptr_t)leaf_ptr(r, odt), out);
          } else {
            PyObject *sn = lc ? r : l;
            PyObject *bo = dget(d_sc_bits, sn);
            const unsigned long long bits = bo ? PyLong_AsUnsignedLongLongMask(bo) : 0;
            Py_XDECREF(bo);
            const unsigned long long arrp = leaf_ptr(lc ? l : r, odt);
            st = p_binary_scalar(binary_code[oid], odt, n, (const void *)(uintptr_t)arrp, &bits,
                                 lc ? 1 : 0, out);
          }
          if (!check_status(st, lc && rc ? "mmp_binary" : "mmp_binary_scalar")) result = Py_None;
        }
      }
    }
    Py_XDECREF(l);
    Py_XDECREF(r);
    if (!result && PyErr_Occurred()) goto fail;
  }
  if (!result) {
    if (buf) goto fail;  // allocated but failed: error already set
    // ---- generated kernel
    Plan pl;
    const int pst = make_plan(node, shape, false, &pl);
    if (pst <= 0) {
      if (pst < 0) goto fail;
      Py_DECREF(shape);
      Py_DECREF(node);
      return PyObject_CallOneArg(py_materialize_fb, arr);
    }
    buf = new_devbuf(n * itemsize[odt]);
    if (!buf) goto fail;
    const unsigned long long outp = ((DevBuf *)buf)->ptr;
    const bool vec = vec_ok(pl, outp % (4ull * itemsize[odt]) == 0);
    void *kern = kernel_for(pl, node, odt, vec, 'm', fast);
    if (!kern) goto fail;
    const long long tile = map_tile(pl.kinds);
    const long long colblocks = (pl.cols + tile - 1) / tile;
    if (launch_plan(pl, kern, outp, colblocks, 1.0)) goto fail;
    result = Py_None;
  }
  if (finish(arr, arrd, buf, shape)) goto fail;
  Py_DECREF(buf);
  Py_DECREF(shape);
  Py_DECREF(node);
  ++stat_native_mat;
  Py_RETURN_NONE;
fail:
  Py_XDECREF(buf);
  Py_XDECREF(shape);
  Py_DECREF(node);
  if (!PyErr_Occurred()) PyErr_SetString(PyExc_RuntimeError, "materialize failed");
  return nullptr;
}

// ------------------------------------------------------ fused row sum
// run_sum(root, axis_last, out_dtype, out_ptr, mean): the sum (or mean) of
// the lazy expression `root` over its last axis (axis_last) or over all of
// it, written to out_ptr -- the Python run_sum: generated kernel with a
// float64 / 64-bit integer row-sum epilogue, split over column blocks when
// there are few rows, then the precompiled reduction over the partials.
// Returns the partials' DeviceBuffer (kept alive by the caller until the
// stream passes it) or None.
PyObject *gate_run_sum(PyObject *, PyObject *const *args, Py_ssize_t nargs) {
  if (nargs != 5) {
    PyErr_SetString(PyExc_TypeError, "run_sum(root, axis_last, out_dtype, out_ptr, mean)");
    return nullptr;
  }
  PyObject *root = args[0], *out_dtype = args[2];
  const int axis_last = PyObject_IsTrue(args[1]), mean = PyObject_IsTrue(args[4]);
  const unsigned long long out_ptr = PyLong_AsUnsignedLongLong(args[3]);
  if (axis_last < 0 || mean < 0 || PyErr_Occurred()) return nullptr;
  const int odt = dtype_index(out_dtype);
  PyTypeObject *t = Py_TYPE(root);
  if (!p_launch || !p_reduce || odt < 0 ||
      (t != T_unary && t != T_binary && t != T_where && t != T_cast && t != T_input)) {
    ++stat_fallback;
    return PyObject_Vectorcall(py_run_sum_fb, args, 5, nullptr);
  }
  PyObject *shape = dget(d_shape, root), *rdto = dget(d_dtype, root);
  const int rdt = rdto ? dtype_index(rdto) : -1;
  Py_XDECREF(rdto);
  long long total = 0;
  Plan pl;
  int pst = (shape && rdt >= 0 && shape_size(shape, &total)) ? make_plan(root, shape, axis_last, &pl)
                                                             : 0;
  Py_XDECREF(shape);
  if (pst <= 0) {
    if (pst < 0) return nullptr;
    PyErr_Clear();
    ++stat_fallback;
    return PyObject_Vectorcall(py_run_sum_fb, args, 5, nullptr);
  }
  const long long count = axis_last ? pl.cols : (total > 1 ? total : 1);
  const double scale = mean ? 1.0 / (double)count : 1.0;
  const int acc = (rdt == D_F16 || rdt == D_F32 || rdt == D_F64)
                      ? D_F64
                      : ((rdt == D_U16 || rdt == D_U32 || rdt == D_U64) ? D_U64 : D_I64);
  long long want = sum_blocks / (pl.rows > 1 ? pl.rows : 1);
  if (want < 1) want = 1;
  long long colblocks = (pl.cols + 4095) / 4096;
  if (colblocks > want) colblocks = want;
  if (colblocks < 1) colblocks = 1;
  const bool final_direct = axis_last && colblocks == 1;
  const bool vec = vec_ok(pl, true);
  void *kern = kernel_for(pl, root, final_direct ? odt : acc, vec, 's', cfg_flag(s_fast_math));
  if (!kern) return nullptr;
  if (final_direct) {
    if (launch_plan(pl, kern, out_ptr, 1, scale)) return nullptr;
    ++stat_native_mat;
    Py_RETURN_NONE;
  }
  PyObject *part = new_devbuf(pl.rows * colblocks * 8);
  if (!part) return nullptr;
  const unsigned long long pp = ((DevBuf *)part)->ptr;
  if (launch_plan(pl, kern, pp, colblocks, scale)) {
    Py_DECREF(part);
    return nullptr;
  }
  const long long outer_n = axis_last ? pl.rows : 1;
  const long long length = axis_last ? colblocks : pl.rows * colblocks;
  if (check_status(p_reduce(0 /* MMP_R_SUM */, acc, odt, outer_n, length, 1,
                            (const void *)(uintptr_t)pp, (void *)(uintptr_t)out_ptr),
                   "mmp_reduce")) {
    Py_DECREF(part);
    return nullptr;
  }
  ++stat_native_mat;
  return part;
}

// ------------------------------------------------------------ reductions
// reduce(code, x, axis): sum / prod / max / min / mean (MMP_R_* codes 0-4)
// or argmax / argmin (5, 6) of a C-contiguous array over all elements
// (axis None) or its last axis, straight to mmp_reduce / mmp_argreduce --
// the reference's fast_reduce gate (_accelerator.c:549-858).  Host-resident
// data is uploaded first (upload_host).  Returns None (the caller takes the
// Python path) for anything else: lazy input, other axes, empty
// reductions.  argmax
// / argmin over everything return a Python int, as the Python path does.
constexpr int kRedCodes = 7;
int8_t red_odt[kRedCodes][kNDT];
void clear_dtype_tables();

PyObject *gate_reduce(PyObject *, PyObject *const *args, Py_ssize_t nargs) {
  if (nargs != 3) {
    PyErr_SetString(PyExc_TypeError, "reduce(code, x, axis)");
    return nullptr;
  }
  const long code = PyLong_AsLong(args[0]);
  PyObject *x = args[1], *axis = args[2];
  if (code < 0 || code >= kRedCodes || !p_reduce || Py_TYPE(x) != T_ndarray) {
    PyErr_Clear();
    Py_RETURN_NONE;
  }
  PyObject *xd = inst_dict(x);
  PyObject *node = iget(xd, s_fnode), *np = iget(xd, s_np_data);
  if ((!node || node == Py_None) && np && np != Py_None) {  // host data: upload here
    const int up = upload_host(xd);
    if (up < 0) return nullptr;
    if (up == 0) Py_RETURN_NONE;
    np = iget(xd, s_np_data);
  }
  PyObject *buf = iget(xd, s_buffer);
  PyObject *shape = iget(xd, s_shape), *strides = iget(xd, s_strides), *dto = iget(xd, s_dtype);
  PyObject *off = iget(xd, s_offset);
  if ((node && node != Py_None) || (np && np != Py_None) || !buf || Py_TYPE(buf) != &DevBufType ||
      !shape || !strides || !dto || !off || !PyTuple_CheckExact(shape))
    Py_RETURN_NONE;
  const int dt = dtype_index(dto);
  long long n = 0;
  if (dt < 0 || !shape_size(shape, &n) || n == 0 || !is_contig(shape, strides)) {
    PyErr_Clear();
    Py_RETURN_NONE;
  }
  const Py_ssize_t nd = PyTuple_GET_SIZE(shape);
  long long outer = 1, len = n;
  bool all = axis == Py_None;
  if (!all) {
    if (!PyLong_CheckExact(axis) || nd == 0) Py_RETURN_NONE;
    const long a = PyLong_AsLong(axis);
    if (a != -1 && a != nd - 1) Py_RETURN_NONE;
    len = PyLong_AsLongLong(PyTuple_GET_ITEM(shape, nd - 1));
    if (len == 0) Py_RETURN_NONE;
    outer = n / len;
  }
  if (red_odt[code][dt] < 0) {
    PyObject *c = PyLong_FromLong(code);
    PyObject *r = c ? PyObject_CallFunctionObjArgs(py_reduce_dt, c, dto, nullptr) : nullptr;
    Py_XDECREF(c);
    const int od = r ? dtype_index(r) : -1;
    Py_XDECREF(r);
    if (od < 0) {
      PyErr_Clear();
      Py_RETURN_NONE;
    }
    red_odt[code][dt] = (int8_t)od;
  }
  const int odt = red_odt[code][dt];
  const long long o = PyLong_AsLongLong(off);
  const unsigned long long src = ((DevBuf *)buf)->ptr + (unsigned long long)o * itemsize[dt];
  PyObject *res = new_devbuf(outer * itemsize[odt]);
  if (!res) return nullptr;
  void *dst = (void *)(uintptr_t)((DevBuf *)res)->ptr;
  const int st = code <= 4 ? p_reduce((int)code, dt, odt, outer, len, 1, (const void *)(uintptr_t)src, dst)
                           : p_argreduce((int)code, dt, outer, len, 1, (const void *)(uintptr_t)src,
                                         (int64_t *)dst);
  if (check_status(st, code <= 4 ? "mmp_reduce" : "mmp_argreduce")) {
    Py_DECREF(res);
    return nullptr;
  }
  ++stat_native_ops;
  if (all && code >= 5) {  // a Python int (synchronises, like the Python path)
    int64_t idx = 0;
    const int st2 = p_d2h(&idx, dst, 8);
    Py_DECREF(res);
    if (check_status(st2, "mmp_d2h")) return nullptr;
    return PyLong_FromLongLong(idx);
  }
  PyObject *oshape = all ? PyTuple_New(0) : PyTuple_GetSlice(shape, 0, nd - 1);
  PyObject *arr = oshape ? T_ndarray->tp_alloc(T_ndarray, 0) : nullptr;
  PyObject *d = arr ? PyDict_New() : nullptr;
  PyObject *ost = d ? contig_strides(oshape) : nullptr;
  PyObject *zero = ost ? PyLong_FromLong(0) : nullptr;
  int bad = !zero;
  if (!bad) {
    *_PyObject_GetDictPtr(arr) = d;
    d = nullptr;
    PyObject *ad = inst_dict(arr);
    bad = PyDict_SetItem(ad, s_buffer, res) || PyDict_SetItem(ad, s_np_data, Py_None) ||
          PyDict_SetItem(ad, s_shape, oshape) || PyDict_SetItem(ad, s_dtype, dtypes[odt]) ||
          PyDict_SetItem(ad, s_strides, ost) || PyDict_SetItem(ad, s_offset, zero) ||
          PyDict_SetItem(ad, s_base, Py_None) || PyDict_SetItem(ad, s_fnode, Py_None);
  }
  Py_XDECREF(d);
  Py_XDECREF(ost);
  Py_XDECREF(zero);
  Py_XDECREF(oshape);
  Py_DECREF(res);
  if (bad) {
    Py_XDECREF(arr);
    return nullptr;
  }
  return arr;
}

// ------------------------------------------------------------ setup
PyObject *descr(PyObject *cls, const char *name) {
  PyObject *d = PyObject_GetAttrString(cls, name);
  if (d && (!Py_TYPE(d)->tp_descr_get || !Py_TYPE(d)->tp_descr_set)) {
    Py_DECREF(d);
    PyErr_Format(PyExc_TypeError, "%s is not a slot", name);
    return nullptr;
  }
  return d;
}

PyObject *gate_init(PyObject *, PyObject *cfg) {
  if (!PyDict_Check(cfg)) {
    PyErr_SetString(PyExc_TypeError, "init(dict)");
    return nullptr;
  }
#define GETCFG(var, key)                                                       \
  do {                                                                         \
    PyObject *v_ = PyDict_GetItemString(cfg, key);                             \
    if (!v_) {                                                                 \
      PyErr_Format(PyExc_KeyError, "init: missing %s", key);                   \
      return nullptr;                                                          \
    }                                                                          \
    Py_INCREF(v_);                                                             \
    var = v_;                                                                  \
  } while (0)
  PyObject *o;
  GETCFG(o, "ndarray"); T_ndarray = (PyTypeObject *)o;
  GETCFG(o, "InputNode"); T_input = (PyTypeObject *)o;
  GETCFG(o, "CastNode"); T_cast = (PyTypeObject *)o;
  GETCFG(o, "UnaryOpNode"); T_unary = (PyTypeObject *)o;
  GETCFG(o, "BinaryOpNode"); T_binary = (PyTypeObject *)o;
  GETCFG(o, "ScalarNode"); T_scalar = (PyTypeObject *)o;
  GETCFG(o, "WhereNode"); T_where = (PyTypeObject *)o;
  GETCFG(py_unary_fb, "unary_py");
  GETCFG(py_binary_fb, "binary_py");
  GETCFG(py_materialize_fb, "materialize_py");
  GETCFG(py_run_sum_fb, "run_sum_py");
  GETCFG(py_reduce_dt, "reduce_dtype");
  GETCFG(py_compile_map, "compile_map");
  GETCFG(py_check, "check");
  GETCFG(py_unary_dt, "unary_dtypes");
  GETCFG(py_binary_dt, "binary_dtypes");
  GETCFG(py_prune, "prune");
  GETCFG(py_ensure_device, "ensure_device");
  GETCFG(cfg_obj, "config");
  PyObject *dts;
  GETCFG(dts, "dtypes");
  if (!PyTuple_Check(dts) || PyTuple_GET_SIZE(dts) != kNDT) {
    PyErr_SetString(PyExc_ValueError, "init: dtypes must be a 10-tuple");
    return nullptr;
  }
  for (int i = 0; i < kNDT; ++i) {
    dtypes[i] = PyTuple_GET_ITEM(dts, i);
    Py_INCREF(dtypes[i]);
  }
  PyObject *md, *ml;
  GETCFG(md, "max_depth");
  GETCFG(ml, "max_leaves");
  max_depth = PyLong_AsLong(md);
  max_leaves = PyLong_AsLong(ml);
  PyObject *sb;
  GETCFG(sb, "sum_blocks");
  sum_blocks = PyLong_AsLong(sb);
  if (sum_blocks < 1) sum_blocks = 1;
  PyObject *ops, *ucodes, *bcodes, *fastset, *intset;
  GETCFG(ops, "op_names");
  GETCFG(ucodes, "unary_codes");
  GETCFG(bcodes, "binary_codes");
  GETCFG(fastset, "fast_ops");
  GETCFG(intset, "int_unary_ops");
#undef GETCFG
  const Py_ssize_t nops = PySequence_Size(ops);
  if (nops < 0 || nops > kMaxOps) {
    PyErr_SetString(PyExc_ValueError, "init: too many ops");
    return nullptr;
  }
  Py_XDECREF(op_ids);
  op_ids = PyDict_New();
  n_ops = (int)nops;
  clear_dtype_tables();
  for (Py_ssize_t i = 0; i < nops; ++i) {
    PyObject *name = PySequence_GetItem(ops, i);
    PyObject *idv = PyLong_FromSsize_t(i);
    PyDict_SetItem(op_ids, name, idv);
    PyObject *uc = PyDict_GetItem(ucodes, name), *bc = PyDict_GetItem(bcodes, name);
    unary_code[i] = uc ? (int)PyLong_AsLong(uc) : -1;
    binary_code[i] = bc ? (int)PyLong_AsLong(bc) : -1;
    fast_op[i] = PySet_Contains(fastset, name) == 1;
    int_unary_op[i] = PySet_Contains(intset, name) == 1;
    Py_DECREF(name);
    Py_DECREF(idv);
  }
  g_kernels.clear();
  PyObject *fnode = (PyObject *)T_input;
  d_shape = descr(fnode, "_shape");
  d_dtype = descr(fnode, "_dtype");
  d_depth = descr(fnode, "_depth");
  d_buffers = descr(fnode, "_buffers");
  d_nleaves = descr(fnode, "_nleaves");
  d_in_buffer = descr(fnode, "_buffer");
  d_in_offset = descr(fnode, "_offset");
  d_in_strides = descr(fnode, "_strides");
  d_sc_bits = descr((PyObject *)T_scalar, "_bits");
  d_un_op = descr((PyObject *)T_unary, "_op_name");
  d_un_input = descr((PyObject *)T_unary, "_input");
  d_cast_input = descr((PyObject *)T_cast, "_input");
  d_bin_op = descr((PyObject *)T_binary, "_op_name");
  d_bin_lhs = descr((PyObject *)T_binary, "_lhs");
  d_bin_rhs = descr((PyObject *)T_binary, "_rhs");
  d_wh_cond = descr((PyObject *)T_where, "_cond");
  d_wh_x = descr((PyObject *)T_where, "_x");
  d_wh_y = descr((PyObject *)T_where, "_y");
  if (PyErr_Occurred()) return nullptr;
  Py_RETURN_NONE;
}

PyObject *gate_set_library(PyObject *, PyObject *fns) {
  if (fns == Py_None) {  // unbind: everything goes to the Python path
    p_alloc = nullptr;
    p_free = nullptr;
    p_unary = nullptr;
    p_binary = nullptr;
    p_binary_scalar = nullptr;
    p_launch = nullptr;
    p_reduce = nullptr;
    p_argreduce = nullptr;
    p_d2h = nullptr;
    p_h2d = nullptr;
    g_kernels.clear();
    Py_RETURN_NONE;
  }
  if (!PyDict_Check(fns)) {
    PyErr_SetString(PyExc_TypeError, "set_library(dict name -> address)");
    return nullptr;
  }
  auto addr = [&](const char *name) -> void * {
    PyObject *v = PyDict_GetItemString(fns, name);
    return v ? PyLong_AsVoidPtr(v) : nullptr;
  };
  p_alloc = (fn_alloc_t)addr("mmp_alloc");
  p_free = (fn_free_t)addr("mmp_free");
  p_unary = (fn_unary_t)addr("mmp_unary");
  p_binary = (fn_binary_t)addr("mmp_binary");
  p_binary_scalar = (fn_binary_scalar_t)addr("mmp_binary_scalar");
  p_launch = (fn_launch_t)addr("mmp_rtc_launch");
  p_reduce = (fn_reduce_t)addr("mmp_reduce");
  p_argreduce = (fn_argreduce_t)addr("mmp_argreduce");
  p_d2h = (fn_d2h_t)addr("mmp_d2h");
  p_h2d = (fn_h2d_t)addr("mmp_h2d");
  if (PyErr_Occurred()) return nullptr;
  if (!p_alloc || !p_free || !p_unary || !p_binary || !p_binary_scalar || !p_launch ||
      !p_reduce || !p_argreduce || !p_d2h || !p_h2d) {
    p_launch = nullptr;
    PyErr_SetString(PyExc_ValueError, "set_library: missing entry points");
    return nullptr;
  }
  Py_RETURN_NONE;
}

// The result-dtype tables follow the float64 policy of the configuration
// (set_config(float64_behavior=..., default_float_dtype=...)): a policy
// change empties them, and the Python rules fill them again on first use.
void clear_dtype_tables() {
  std::memset(un_rdt, -1, sizeof un_rdt);
  std::memset(un_idt, -1, sizeof un_idt);
  std::memset(bin_rdt, -1, sizeof bin_rdt);
  std::memset(bin_odt, -1, sizeof bin_odt);
  std::memset(bsc_rdt, -1, sizeof bsc_rdt);
  std::memset(bsc_odt, -1, sizeof bsc_odt);
  std::memset(red_odt, -1, sizeof red_odt);
}

PyObject *gate_forget_dtypes(PyObject *, PyObject *) {
  clear_dtype_tables();
  Py_RETURN_NONE;
}

PyObject *gate_clear_kernels(PyObject *, PyObject *) {
  g_kernels.clear();
  Py_RETURN_NONE;
}

PyObject *gate_stats(PyObject *, PyObject *) {
  return Py_BuildValue("{s:K,s:K,s:K,s:K,s:n}", "native_ops", stat_native_ops,
                       "native_materialize", stat_native_mat, "fallbacks", stat_fallback,
                       "native_uploads", stat_uploads, "kernels", (Py_ssize_t)g_kernels.size());
}

PyMethodDef methods[] = {
    {"init", (PyCFunction)gate_init, METH_O, "Bind the Python classes, fallbacks and tables."},
    {"set_library", (PyCFunction)gate_set_library, METH_O,
     "Entry-point addresses of the loaded libmmp_hip.so."},
    {"unary", (PyCFunction)(void (*)(void))gate_unary, METH_FASTCALL,
     "unary(op_name, x): lazy elementwise result (falls back to the Python path)."},
    {"binary", (PyCFunction)(void (*)(void))gate_binary, METH_FASTCALL,
     "binary(op_name, a, b): lazy elementwise result (falls back to the Python path)."},
    {"materialize", (PyCFunction)gate_materialize, METH_O,
     "Evaluate a lazy array in place (falls back to the Python path)."},
    {"run_sum", (PyCFunction)(void (*)(void))gate_run_sum, METH_FASTCALL,
     "run_sum(root, axis_last, out_dtype, out_ptr, mean): fused sum epilogue."},
    {"reduce", (PyCFunction)(void (*)(void))gate_reduce, METH_FASTCALL,
     "reduce(code, x, axis): whole-array or last-axis reduction, or None."},
    {"stats", (PyCFunction)gate_stats, METH_NOARGS, "Counters of the native and fallback paths."},
    {"forget_dtypes", (PyCFunction)gate_forget_dtypes, METH_NOARGS,
     "Empty the result-dtype tables (after a float64 policy change)."},
    {"clear_kernels", (PyCFunction)gate_clear_kernels, METH_NOARGS,
     "Forget the generated kernels known by structure."},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef moddef = {PyModuleDef_HEAD_INIT, "_native",
                      "Native host dispatch of elementwise ops (see native_gate.cpp).", -1,
                      methods};

}  // namespace

PyMODINIT_FUNC PyInit__native(void) {
  DevBufType.tp_name = "macmetalpy_amd._native.DeviceBuffer";
  DevBufType.tp_basicsize = sizeof(DevBuf);
  DevBufType.tp_flags = Py_TPFLAGS_DEFAULT;
  DevBufType.tp_doc =
      "DeviceBuffer(ptr, nbytes, owned=True): handle of one device allocation (the "
      "reference's _Buffer, _metal_backend.py:121-165); an owned one is freed to the "
      "stream-ordered pool (mmp_free) when the last reference goes, a borrowed one "
      "(owned=False) never is.";
  DevBufType.tp_new = PyType_GenericNew;
  DevBufType.tp_init = (initproc)devbuf_init;
  DevBufType.tp_dealloc = (destructor)devbuf_dealloc;
  DevBufType.tp_repr = (reprfunc)devbuf_repr;
  DevBufType.tp_members = devbuf_members;
  DevBufType.tp_getset = devbuf_getset;
  DevBufType.tp_weaklistoffset = offsetof(DevBuf, weakreflist);
  if (PyType_Ready(&DevBufType) < 0) return nullptr;
  PyObject *m = PyModule_Create(&moddef);
  if (!m) return nullptr;
  Py_INCREF(&DevBufType);
  if (PyModule_AddObject(m, "DeviceBuffer", (PyObject *)&DevBufType) < 0) {
    Py_DECREF(&DevBufType);
    Py_DECREF(m);
    return nullptr;
  }
#define INTERN(var, s) var = PyUnicode_InternFromString(s)
  INTERN(s_buffer, "_buffer");
  INTERN(s_np_data, "_np_data");
  INTERN(s_shape, "_shape");
  INTERN(s_dtype, "_dtype");
  INTERN(s_strides, "_strides");
  INTERN(s_offset, "_offset");
  INTERN(s_base, "_base");
  INTERN(s_fnode, "_fusion_node");
  INTERN(s_fusion, "fusion");
  INTERN(s_fast_math, "fast_math");
#undef INTERN
  return m;
}
