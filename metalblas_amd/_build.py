"""Ahead-of-time build of libmetalblas_hip.so for gfx950.

The reference compiles Metal kernel variants at first use (metalblas/kernels.py:40-62,
torch.mps.compile_shader).  Here every kernel variant is a C++ template instantiated at
build time: each ``csrc/*.hip`` file is compiled with hipcc for gfx950 in parallel and the
objects are linked into one shared library next to this file.  Python loads it with ctypes
(``metalblas_amd._lib``).
"""
from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libmetalblas_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# object files of the last build (kept for the sanitizer test's link; not shipped)
OBJ_DIR = os.path.join(PKG_DIR, "_build", "obj")
ARCH = os.environ.get("METALBLAS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    # packed-fp32 VALU forms are kept out of generated code on this hardware
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: cannot build libmetalblas_hip.so")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


# The compiled fast path of the Python API (csrc/mb_fast.cpp): a PyTorch C++ extension that
# calls mb_gemm directly for call signatures the Python layer has planned.  Host code only.
FAST_SRC = os.path.join(CSRC, "mb_fast.cpp")


def _fast_target() -> str:
    import sysconfig
    return os.path.join(PKG_DIR, "_fast" + sysconfig.get_config_var("EXT_SUFFIX"))


def _fast_flags():
    import sysconfig
    import torch
    from torch.utils import cpp_extension as ce
    tdir = os.path.dirname(torch.__file__)
    inc = [os.path.join(tdir, "include"), os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
           "/opt/rocm/include", sysconfig.get_paths()["include"]]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_fast",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}"] + [f"-I{d}" for d in inc]
    tlib = os.path.join(tdir, "lib")
    ldflags = [f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
               f"-Wl,-rpath,{tlib}", f"-L{PKG_DIR}", "-lmetalblas_hip", "-Wl,-rpath,$ORIGIN"]
    del ce
    return cflags, ldflags


def _compile_fast(obj):
    cflags, _ = _fast_flags()
    cmd = [os.environ.get("CXX", "g++"), *cflags, "-c", FAST_SRC, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed for mb_fast.cpp:\n{proc.stderr[-6000:]}")
    return obj


def _compile(args):
    hipcc, src, obj = args
    cmd = [hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{proc.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link libmetalblas_hip.so (always rebuilds).

    The core library is linked first.  The optional compiled fast path (``_fast``) is built
    after it; if its compile or link fails (missing torch or Python headers, an ABI mismatch)
    the failure is reported as a warning, any stale ``_fast`` module is removed so it cannot
    bind an older ABI, and the Python path keeps working on the core library alone."""
    hipcc = _hipcc()
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs = [os.path.join(OBJ_DIR, os.path.basename(s) + ".o") for s in srcs]
    fast_obj = os.path.join(OBJ_DIR, "mb_fast.cpp.o")
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        fast = ex.submit(_compile_fast, fast_obj)
        list(ex.map(_compile, [(hipcc, s, o) for s, o in zip(srcs, objs)]))
        fast_err = fast.exception()
    out_tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out_tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(out_tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    target = _fast_target()
    if fast_err is None:
        _, ldflags = _fast_flags()
        cmd = [os.environ.get("CXX", "g++"), "-shared", "-o", target + ".tmp", fast_obj, *ldflags]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            fast_err = RuntimeError(f"link of the fast path failed:\n{proc.stderr[-6000:]}")
        else:
            os.replace(target + ".tmp", target)
            if verbose:
                print(f"built {target}")
    if fast_err is not None:
        for stale in (target, target + ".tmp"):
            if os.path.exists(stale):
                os.remove(stale)
        print(f"warning: metalblas_amd fast path not built ({fast_err}); the Python path runs "
              "on the core library", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
