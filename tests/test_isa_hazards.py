"""CPU checks of the gfx950 machine code of the LDS-direct kernels.

The matrix-core kernels issue their LDS-direct loads (``buffer_load_* ... lds``) from inline
assembly, which the compiler's hazard recognizer does not look into.  On gfx950 a VMEM
instruction that reads an SGPR written by a VALU instruction (``v_readlane_b32`` SGPR-spill
reloads, ``v_readfirstlane_b32``) needs 5 wait states; the compiler pads its own loads with
``s_nop 4`` (checked below on a probe kernel), the asm must pad itself.  With fewer, the load
can read the SGPR's previous value as its buffer resource or offset, i.e. an arbitrary
address.  These tests compile the kernels to assembly and scan every VMEM instruction for such
a write less than 5 wait states before it."""
import concurrent.futures
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "metalblas_amd", "csrc")
HIPCC = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else None)
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "--offload-device-only", "-S"]
# the sources whose kernels issue LDS-direct loads from inline assembly (one per kernel family)
SOURCES = ["gemm_m16pp_bf16.hip", "gemm_m16_bf16_ktail.hip", "gemm_m16_i8_ktail.hip", "gemm_m16_thin.hip"]
NEEDED = 5

needs_hipcc = pytest.mark.skipif(HIPCC is None, reason="hipcc not available")


def _sregs(text):
    out = set()
    for m in re.finditer(r"\bs\[(\d+):(\d+)\]", text):
        out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"(?<![\w\[])s(\d+)\b", text):
        out.add(int(m.group(1)))
    if re.search(r"\bm0\b", text):
        out.add("m0")
    return out


def scan(asm_text):
    """(function, wait states, VALU write, VMEM instruction) for every VMEM instruction that
    reads an SGPR (or M0, for LDS-direct loads) a VALU instruction wrote fewer than 5 wait
    states earlier in the function's linear instruction order (fall-through across block
    labels, which over-approximates the predecessors)."""
    bad, block, fn = [], [], None
    for line in asm_text.splitlines():
        t = line.split(";")[0].strip()
        if not t or t.startswith("."):
            continue
        if t.endswith(":"):
            fn, block = t[:-1], []
            continue
        block.append(t)
        op = t.split(None, 1)
        if len(op) < 2 or not op[0].startswith(("buffer_", "global_", "scratch_", "flat_")):
            continue
        used = _sregs(op[1])
        if re.search(r"\blds\b", op[1]):
            used.add("m0")
        ws = 0
        for prev in reversed(block[:-1]):
            p = prev.split(None, 1)
            if p[0] == "s_nop":
                ws += int(p[1], 0) + 1 if len(p) > 1 else 1
            else:
                if p[0].startswith("v_") and len(p) > 1 and _sregs(p[1].split(",")[0]) & used:
                    bad.append((fn, ws, prev, t))
                    break
                ws += 1
            if ws >= NEEDED:
                break
    return bad


def _compile(src, out_dir):
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    subprocess.run([HIPCC, *FLAGS, "-o", out, src], check=True, capture_output=True)
    return open(out).read()


PROBE = r"""
#include <hip/hip_runtime.h>
__global__ void probe(const int *a, int *c, int n) {
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)a, (short)0, n * 4, 0x00020000);
    int s = __builtin_amdgcn_readfirstlane(c[threadIdx.x]);
    c[threadIdx.x] = __builtin_amdgcn_raw_buffer_load_b32(r, threadIdx.x * 4, s, 0);
}
"""


@needs_hipcc
def test_compiler_pads_valu_sgpr_to_vmem():
    """The rule the asm follows: the compiler itself puts 5 wait states between a VALU write of
    an SGPR and a buffer load reading it; and the scanner sees no hazard in that code but does
    see one when the padding is removed."""
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "probe.hip")
        open(src, "w").write(PROBE)
        asm = _compile(src, d)
    assert re.search(r"v_readfirstlane_b32 (s\d+).*\n\s*s_nop 4\n\s*buffer_load_dword .*\1 offen", asm), asm
    assert scan(asm) == []
    broken = re.sub(r"\n\s*s_nop 4\n", "\n", asm)
    assert len(scan(broken)) == 1


def test_inline_asm_loads_carry_five_wait_states():
    """Every inline-assembly VMEM instruction in the sources starts with s_nop 4."""
    for name in os.listdir(CSRC):
        if not name.endswith((".hip", ".hpp")):
            continue
        text = open(os.path.join(CSRC, name)).read()
        for m in re.finditer(r'asm\s+volatile\s*\(\s*"([^"]*)"', text):
            body = m.group(1)
            if re.search(r"\b(buffer|global|scratch|flat)_", body):
                assert body.startswith("s_nop 4\\n"), f"{name}: {body!r}"


@needs_hipcc
def test_lds_direct_kernels_have_no_sgpr_hazard():
    with tempfile.TemporaryDirectory() as d:
        with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
            texts = list(ex.map(lambda s: _compile(os.path.join(CSRC, s), d), SOURCES))
    for name, text in zip(SOURCES, texts):
        assert "buffer_load_dwordx4" in text and " lds" in text, name   # the scan sees the loads
        bad = scan(text)
        assert not bad, f"{name}: {bad[:3]}"
