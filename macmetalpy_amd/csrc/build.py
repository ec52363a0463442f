"""Build libmmp_hip.so (gfx950) from the HIP sources in this directory.

Every ``*.hip`` file is compiled by hipcc into ``_build/<name>.o`` in
parallel and the objects are linked into ``macmetalpy_amd/libmmp_hip.so``
together with hiprtc; ``native_gate.cpp`` is compiled by g++ into the
CPython extension ``macmetalpy_amd/_native*.so``.  Run as a script (the
package cannot be imported before these exist)::

    python macmetalpy_amd/csrc/build.py            # full rebuild
    python macmetalpy_amd/csrc/build.py --incremental
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(PKG, "libmmp_hip.so")
ARCH = os.environ.get("MMP_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: no a*b+c -> fma contraction, so results round op by op
# exactly as NumPy's; the packed-fp32 feature is disabled for all device code.
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{HERE}",
]


def _hipcc() -> str:
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc") or ""):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmmp_hip.so)")


def sources() -> list[str]:
    return sorted(f for f in os.listdir(HERE) if f.endswith(".hip"))


def _newest_header() -> float:
    hs = [os.path.join(HERE, f) for f in os.listdir(HERE) if f.endswith(".h")]
    hs.append(os.path.join(INCLUDE, "mmp_hip.h"))
    return max(os.path.getmtime(h) for h in hs)


def _compile(src: str, incremental: bool, hdr_time: float) -> tuple[str, float, str]:
    obj = os.path.join(BUILD, src[:-4] + ".o")
    path = os.path.join(HERE, src)
    if incremental and os.path.exists(obj):
        ot = os.path.getmtime(obj)
        if ot >= os.path.getmtime(path) and ot >= hdr_time:
            return src, 0.0, ""
    t = time.time()
    cmd = [_hipcc(), *HIPFLAGS, "-c", path, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{p.stdout}\n{p.stderr}")
    warn = "\n".join(
        line for line in (p.stderr or "").splitlines()
        if "packed-fp32-ops" not in line and line.strip()
    )
    return src, time.time() - t, warn


NATIVE_SRC = os.path.join(HERE, "native_gate.cpp")


def native_path() -> str:
    import sysconfig
    return os.path.join(PKG, "_native" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_native(verbose: bool = True) -> str:
    """The CPython extension of the dispatch gate (host code only: g++
    against the Python headers; it reaches libmmp_hip.so through entry-point
    addresses handed over at run time)."""
    import sysconfig
    out = native_path()
    tmp = out + ".tmp"
    cmd = [shutil.which("g++") or "g++", "-O2", "-std=c++17", "-shared", "-fPIC",
           "-fvisibility=hidden", "-Wall", "-Wno-missing-field-initializers",
           "-Wno-cast-function-type", f"-I{sysconfig.get_paths()['include']}", NATIVE_SRC,
           "-o", tmp]
    t = time.time()
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"g++ failed for native_gate.cpp:\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} in {time.time() - t:.1f}s", flush=True)
    return out


def build(incremental: bool = False, jobs: int | None = None, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    hdr = _newest_header()
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    t0 = time.time()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for src, dt, warn in ex.map(lambda s: _compile(s, incremental, hdr), srcs):
            if verbose and dt:
                print(f"  hipcc {src}: {dt:.1f}s", flush=True)
            if verbose and warn:
                print(warn, flush=True)
    objs = [os.path.join(BUILD, s[:-4] + ".o") for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} in {time.time() - t0:.1f}s", flush=True)
    if not (incremental and os.path.exists(native_path())
            and os.path.getmtime(native_path()) >= os.path.getmtime(NATIVE_SRC)):
        build_native(verbose)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--incremental", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    a = ap.parse_args()
    try:
        build(incremental=a.incremental, jobs=a.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
