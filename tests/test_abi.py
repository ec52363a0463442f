"""C ABI: the library loads without a GPU and exports exactly what
include/mmp_hip.h declares; constants match the Python mirror."""
import ctypes
import os
import re

import numpy as np
import pytest

from macmetalpy_amd import _abi
from macmetalpy_amd._backend import HipError, load_library, lib_path

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mmp_hip.h")


def _header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(mmp_\w+)\(", text, re.M)))


def _header_defines():
    text = open(HEADER).read()
    return {k: int(v) for k, v in re.findall(r"#define (MMP_\w+) (\d+)", text)}


def test_library_exists_and_loads():
    assert os.path.exists(lib_path()), "run __graft_entry__.build() first"
    lib = load_library()
    assert lib is not None


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(lib_path())
    names = _header_functions()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), f"{name} declared in mmp_hip.h but not exported"
    assert sorted(_abi.EXPORTS) == names


def test_dtype_and_op_codes_match_header():
    d = _header_defines()
    names = {np.dtype(np.bool_): "BOOL", np.dtype(np.int16): "I16", np.dtype(np.uint16): "U16",
             np.dtype(np.int32): "I32", np.dtype(np.uint32): "U32", np.dtype(np.int64): "I64",
             np.dtype(np.uint64): "U64", np.dtype(np.float16): "F16",
             np.dtype(np.float32): "F32", np.dtype(np.float64): "F64"}
    for dt, code in _abi.DTYPE_CODES.items():
        assert d["MMP_" + names[dt]] == code
    unary_names = {"neg_op": "NEG", "positive_op": "POSITIVE", "abs_op": "ABS", "sign_op": "SIGN",
                   "square_op": "SQUARE", "reciprocal_op": "RECIPROCAL", "sqrt_op": "SQRT",
                   "cbrt_op": "CBRT", "exp_op": "EXP", "exp2_op": "EXP2", "expm1_op": "EXPM1",
                   "log_op": "LOG", "log2_op": "LOG2", "log10_op": "LOG10", "log1p_op": "LOG1P",
                   "sin_op": "SIN", "cos_op": "COS", "tan_op": "TAN", "asin_op": "ASIN",
                   "acos_op": "ACOS", "atan_op": "ATAN", "sinh_op": "SINH", "cosh_op": "COSH",
                   "tanh_op": "TANH", "asinh_op": "ASINH", "acosh_op": "ACOSH",
                   "atanh_op": "ATANH", "floor_op": "FLOOR", "ceil_op": "CEIL", "rint_op": "RINT",
                   "trunc_op": "TRUNC", "degrees_op": "DEGREES", "radians_op": "RADIANS"}
    for op, hname in unary_names.items():
        assert d["MMP_U_" + hname] == _abi.UNARY_OPS[op][0]
    binary_names = {"add_op": "ADD", "sub_op": "SUB", "mul_op": "MUL", "div_op": "DIV",
                    "floor_divide_op": "FLOOR_DIVIDE", "mod_op": "MOD", "pow_op": "POWER",
                    "max_op": "MAXIMUM", "min_op": "MINIMUM", "fmax_op": "FMAX",
                    "fmin_op": "FMIN", "atan2_op": "ATAN2", "hypot_op": "HYPOT",
                    "fmod_op": "FMOD", "copysign_op": "COPYSIGN", "nextafter_op": "NEXTAFTER",
                    "logaddexp_op": "LOGADDEXP", "logaddexp2_op": "LOGADDEXP2",
                    "heaviside_op": "HEAVISIDE"}
    for op, hname in binary_names.items():
        assert d["MMP_B_" + hname] == _abi.BINARY_OPS[op][0]
    assert d["MMP_R_SUM"] == _abi.REDUCE_SUM and d["MMP_R_MEAN"] == _abi.REDUCE_MEAN
    assert d["MMP_R_ARGMAX"] == _abi.REDUCE_ARGMAX and d["MMP_S_CUMSUM"] == _abi.SCAN_CUMSUM


def test_status_and_message_without_device():
    """Without a GPU every device entry point reports MMP_E_NODEVICE with a
    message; nothing falls back to the CPU."""
    lib = load_library()
    count = ctypes.c_int(-1)
    assert lib.mmp_device_count(ctypes.byref(count)) == 0
    if count.value > 0:
        pytest.skip("a GPU is visible")
    assert lib.mmp_init(0) == _abi.MMP_E_NODEVICE
    assert b"no HIP device" in lib.mmp_last_error()
    p = ctypes.c_void_p()
    assert lib.mmp_alloc(16, ctypes.byref(p)) == _abi.MMP_E_NODEVICE
    import macmetalpy_amd as cp
    with pytest.raises(HipError, match="no HIP device"):
        (cp.arange(4, dtype=np.float32) + 1).get()


def test_rtc_build_without_device():
    from macmetalpy_amd._backend import rtc_build
    code = rtc_build('extern "C" __global__ void k(float* x) { x[threadIdx.x] *= 2.0f; }',
                     "-O3")
    assert code[:4] == b"\x7fELF"
    with pytest.raises(HipError, match="hiprtc compile failed"):
        rtc_build('extern "C" __global__ void k(float* x) { not valid c++ }', "-O3")


def test_error_classes_and_hook_validation():
    """Status codes map to the Python error classes callers catch; the
    test hook rejects unknown kinds without touching a device."""
    from macmetalpy_amd import _abi
    from macmetalpy_amd import _backend as B
    assert B._ERR_CLASSES[_abi.MMP_E_WAIT] is B.HipWaitTimeoutError
    assert issubclass(B.HipWaitTimeoutError, B.HipError)
    assert issubclass(B.HipOutOfMemoryError, MemoryError)
    lib = B.load_library()
    assert lib.mmp_debug_fail_next(5, 1) == _abi.MMP_E_ARG
    assert lib.mmp_debug_fail_next(-1, 1) == _abi.MMP_E_ARG
    assert lib.mmp_debug_fail_next(4, 0) == 0
    import re
    hdr = open(os.path.join(ROOT, "include", "mmp_hip.h")).read()
    codes = dict(re.findall(r"#define (MMP_E_\w+) (\d+)", hdr))
    assert int(codes["MMP_E_WAIT"]) == _abi.MMP_E_WAIT == 8


def test_reduce_noalloc_refuses_before_init():
    """The allocation-free reduction never initialises the library (that
    allocates): before mmp_init it returns MMP_E_ARG without a device."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from macmetalpy_amd._backend import load_library\n"
            "lib = load_library()\n"
            "st = lib.mmp_reduce_noalloc(0, 8, 8, 1, 16, 1, 4096, 8192)\n"
            "print(st, lib.mmp_last_error().decode())\n") % ROOT
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    st, msg = out.stdout.split(" ", 1)
    assert int(st) == _abi.MMP_E_ARG and "mmp_init" in msg
