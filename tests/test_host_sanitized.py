"""The host side of libmetalblas_hip.so (the C planner and its per-signature plan cache,
csrc/mb_api.hip) under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

mb_api.hip is compiled with host-only sanitizers and linked with the other objects of the last
build (metalblas_amd/_build/obj); a Python child process with the sanitizer runtime preloaded
then drives every plan family through mb_gemm (dry runs: plan, relocate, verify, no launch),
mb_plan, mb_gemm_workspace_bytes and mb_tile_candidates, and the host tests of the ABI.  Any
report from either sanitizer aborts the child.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from metalblas_amd import _build  # noqa: E402

pytestmark = pytest.mark.timeout(600)


def _asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def _sanitized_lib(tmp):
    objs = [os.path.join(_build.OBJ_DIR, os.path.basename(s) + ".o") for s in _build.sources()
            if not s.endswith("mb_api.hip")]
    if not all(os.path.exists(o) for o in objs):
        pytest.skip("no objects of a previous build in metalblas_amd/_build/obj (run __graft_entry__.build())")
    hipcc = _build._hipcc()
    api_obj = os.path.join(tmp, "mb_api_san.o")
    flags = [f for f in _build.HIPCC_FLAGS if f != "-O3"]
    cmd = [hipcc, *flags, "-O1", "-g", "-fno-omit-frame-pointer",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined",
           "-c", os.path.join(_build.CSRC, "mb_api.hip"), "-o", api_obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    lib = os.path.join(tmp, "libmetalblas_hip.so")
    cmd = [hipcc, f"--offload-arch={_build.ARCH}", "-shared", "-fPIC", "-shared-libsan",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-o", lib, api_obj, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    return lib


DRIVER = r"""
import ctypes, sys, runpy
sys.path.insert(0, ROOT)
sys.path.insert(0, ROOT + "/tests")
import torch
from metalblas_amd import _lib
assert _lib.LIB_PATH.endswith(LIBNAME), _lib.LIB_PATH
# every plan family through mb_gemm's cache (dry runs, verify mode), as tests/test_launch_cache.py
src = open(ROOT + "/tests/test_launch_cache.py").read()
driver = src.split('DRIVER = r\"\"\"', 1)[1].split('\"\"\"', 1)[0]
exec(compile(driver, "launch_cache_driver", "exec"), {"ROOT": ROOT})
# planner queries on odd shapes, alignments and every dtype
lib = _lib.load()
for dt in _lib.DTYPE_CODE:
    for (M, N, K) in [(1, 1, 1), (3, 5, 7), (513, 257, 129), (4097, 4096, 2048), (128, 128, 65536),
                      (16384, 8, 16384), (8, 16384, 16384), (1, 16384, 16384)]:
        for off in (0, 1, 17):
            a = torch.empty(M * K + off, dtype=dt)[off:].view(M, K)
            b = torch.empty(K, N, dtype=dt)
            c = torch.empty(M, N, dtype=dt)
            d = _lib.make_desc(dt, 1, M, N, K, (a, K, 1, 0), (b, N, 1, 0), (c, N, 1, 0))
            info = _lib.MbPlanInfo()
            assert lib.mb_plan(ctypes.byref(d), ctypes.byref(info)) == 0
            assert lib.mb_gemm_workspace_bytes(ctypes.byref(d)) >= 0
            buf = (ctypes.c_int32 * 128)()
            assert lib.mb_tile_candidates(ctypes.byref(d), buf, 16) >= 0
print("driver ok", flush=True)
"""


def test_planner_under_address_and_undefined_behaviour_sanitizers(tmp_path):
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("clang's AddressSanitizer runtime is not installed")
    lib = _sanitized_lib(str(tmp_path))
    syms = subprocess.run(["nm", "-D", lib], capture_output=True, text=True).stdout
    assert "__asan_" in syms and "__ubsan_handle" in syms, "the planner was not instrumented"
    env = dict(os.environ, LD_PRELOAD=rt, METALBLAS_LIB=lib, METALBLAS_LAUNCH_CACHE="verify",
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    code = f"ROOT = {ROOT!r}\nLIBNAME = {lib!r}\n" + DRIVER
    proc = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=500)
    out = proc.stdout[-3000:] + proc.stderr[-6000:]
    assert proc.returncode == 0, out
    assert "driver ok" in proc.stdout and "all ok" in proc.stdout, out
    assert "runtime error" not in proc.stderr and "AddressSanitizer" not in proc.stderr, out
    # the ABI host tests against the same build
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                           os.path.join(ROOT, "tests", "test_host.py"), "-k", "not sanitized"],
                          env=env, capture_output=True, text=True, timeout=500, cwd=ROOT)
    out = proc.stdout[-3000:] + proc.stderr[-6000:]
    assert proc.returncode == 0, out
    assert "runtime error" not in proc.stderr and "AddressSanitizer" not in proc.stderr, out
