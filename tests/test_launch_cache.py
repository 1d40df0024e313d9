"""mb_gemm's per-signature plan cache (CPU; no GPU needed).

mb_gemm plans a call signature once on sentinel pointers and relocates the cached plan's pointer
fields to each later call's operands.  With METALBLAS_LAUNCH_CACHE=verify the library also replans
every cache hit from the real descriptor and aborts when any relocated pointer or launch choice
differs.  Here every plan family is driven through mb_gemm three times per signature, with the
operands (and workspace) moved to new addresses between calls.  Every call carries
MB_FLAG_DRY_RUN: mb_gemm plans, relocates and verifies, then returns MB_OK without queuing any
work, so the made-up pointers never reach a kernel, with or without a GPU in the machine.
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

DRIVER = r"""
import ctypes, sys
sys.path.insert(0, ROOT)
import torch
from metalblas_amd import _lib
lib = _lib.load()

class Ptr:                       # stands in for a tensor: only data_ptr() is read
    def __init__(self, p): self.p = p
    def data_ptr(self): return self.p

def run(name, dt, batch, M, N, K, a, b, c, bias=None, low=0, ws=True, **kw):
    # a/b/c/bias: (row_stride, col_stride, batch_stride); operand i lives at base + i * 2^40 + low
    codes = set()
    for shift in (0, 0x1000000, 0x2345600):          # moves keep the low 8 bits
        base = 0x7f0000000000 + shift
        ops = [None if m is None else (Ptr(base + i * (1 << 40) + low * (i + 1)),) + tuple(m)
               for i, m in enumerate((a, b, c, bias))]
        d = _lib.make_desc(dt, batch, M, N, K, *ops, flags=_lib.FLAG_DRY_RUN, **kw)
        need = _lib.workspace_bytes(d)
        if need and ws:
            d.workspace, d.workspace_bytes = 0x7e0000000000 + shift, need
        codes.add(lib.mb_gemm(ctypes.byref(d), None))
    assert codes == {_lib.OK}, (name, codes)
    print("ok", name, flush=True)

bf, f16, f32 = torch.bfloat16, torch.float16, torch.float32
rm = lambda r, c: (c, 1, 0)
cm = lambda r, c: (1, r, 0)
ep = (0.5, 2.0, True, True)
run("bf16 8192^3", bf, 1, 8192, 8192, 8192, rm(8192, 8192), rm(8192, 8192), rm(8192, 8192))
for la in (rm, cm):
    for lb in (rm, cm):
        run(f"bf16 2048x4096x2048 {la.__name__}", bf, 1, 2048, 2048, 4096, la(2048, 4096), lb(4096, 2048), rm(2048, 2048))
run("column-major output", f16, 1, 1024, 768, 512, rm(1024, 512), rm(512, 768), cm(1024, 768))
run("offset 17 (operand copy)", bf, 1, 2048, 2048, 4096, rm(2048, 4096), rm(4096, 2048), rm(2048, 2048), low=34)
run("column-sliced", bf, 1, 2048, 2048, 4096, (8192, 2, 0), rm(4096, 2048), rm(2048, 2048))
run("peel M", bf, 1, 4097, 4096, 4096, rm(4097, 4096), rm(4096, 4096), rm(4097, 4096))
run("peel N", bf, 1, 4096, 4100, 4096, rm(4096, 4096), rm(4096, 4100), rm(4096, 4100))
run("peel both + addmm", f16, 1, 4097, 4100, 2048, rm(4097, 2048), rm(2048, 4100), rm(4097, 4100),
    bias=(0, 1, 0), epilogue=ep)
run("packed peel 4097^3", bf, 1, 4097, 4097, 4097, rm(4097, 4097), rm(4097, 4097), rm(4097, 4097))
run("packed peel N + addmm", f16, 1, 4096, 4100, 4100, rm(4096, 4100), rm(4100, 4100), rm(4096, 4100),
    bias=(0, 1, 0), epilogue=ep)
run("addmm bias row", bf, 1, 2048, 2048, 4096, rm(2048, 4096), rm(4096, 2048), rm(2048, 2048),
    bias=(0, 1, 0), epilogue=ep)
run("split-K 128x128x65536", f16, 1, 128, 128, 65536, rm(128, 65536), rm(65536, 128), rm(128, 128))
run("split-K without workspace", f16, 1, 128, 128, 65536, rm(128, 65536), rm(65536, 128), rm(128, 128), ws=False)
run("bmm 8", f16, 8, 512, 512, 256, (256, 1, 512 * 256), (512, 1, 256 * 512), (512, 1, 512 * 512))
run("bmm broadcast B", f16, 8, 512, 512, 256, (256, 1, 512 * 256), (512, 1, 0), (512, 1, 512 * 512))
run("gemv W@x", bf, 1, 16384, 1, 16384, rm(16384, 16384), (1, 1, 0), (1, 1, 0))
run("gemv x@W", bf, 1, 1, 16384, 16384, (16384, 1, 0), rm(16384, 16384), (16384, 1, 0))
run("thin X8@W", bf, 1, 8, 16384, 16384, rm(8, 16384), rm(16384, 16384), rm(8, 16384))
run("thin W@X8", bf, 1, 16384, 8, 16384, rm(16384, 16384), rm(16384, 8), rm(16384, 8))
run("gemv generic strides", f32, 1, 300, 1, 500, (3, 900, 0), (1, 1, 0), (1, 1, 0))
c64 = torch.complex64
run("complex64 2048^3 conj A", c64, 1, 2048, 2048, 2048, rm(2048, 2048), rm(2048, 2048), rm(2048, 2048), conj_a=True)
run("complex64 gemv", c64, 1, 8192, 1, 8192, rm(8192, 8192), (1, 1, 0), (1, 1, 0))
run("complex32 addmm", torch.complex32, 1, 512, 384, 256, rm(512, 256), rm(256, 384), rm(512, 384),
    bias=(0, 1, 0), epilogue=(0.5 + 1j, 2.0, True, True))
run("int8 4096^3", torch.int8, 1, 4096, 4096, 4096, rm(4096, 4096), rm(4096, 4096), rm(4096, 4096))
run("uint8", torch.uint8, 1, 512, 512, 512, rm(512, 512), rm(512, 512), rm(512, 512))
run("int32 256^3", torch.int32, 1, 256, 256, 256, rm(256, 256), rm(256, 256), rm(256, 256))
run("int64 addmm", torch.int64, 1, 64, 96, 80, rm(64, 80), rm(80, 96), rm(64, 96), bias=(96, 1, 0),
    epilogue=(3, -2, True, True))
run("fp32 1000^3", f32, 1, 1000, 1000, 1000, rm(1000, 1000), rm(1000, 1000), rm(1000, 1000))
run("fp32 forced generic", f32, 1, 300, 200, 100, rm(300, 100), rm(100, 200), rm(300, 200),
    backend=_lib.BACKEND_GENERIC)
run("forced tile", bf, 1, 1024, 1024, 1024, rm(1024, 1024), rm(1024, 1024), rm(1024, 1024),
    backend=_lib.BACKEND_MATRIX, tile=(128, 128, 64))
run("K = 0 fill", bf, 1, 64, 64, 0, rm(64, 1), rm(1, 64), rm(64, 64), bias=(0, 1, 0), epilogue=ep)
print("all ok", flush=True)
"""


@pytest.mark.timeout(300)
def test_relocated_plans_match_fresh_plans():
    env = dict(os.environ, METALBLAS_LAUNCH_CACHE="verify")
    proc = subprocess.run([sys.executable, "-c", f"ROOT = {ROOT!r}\n" + DRIVER], env=env,
                          capture_output=True, text=True, timeout=280)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-3000:]
    assert "all ok" in proc.stdout
