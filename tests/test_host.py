"""CPU tests of the host side: the C ABI's exports and struct layout, the planner's decisions
for the benchmark configurations, error mapping, and the Python layout/scalar logic of
metalblas/dispatch.py that the drop-in keeps.  Nothing here launches a kernel."""
import ctypes
import json
import os
import re
import subprocess
import tempfile

import pytest
import torch

import metalblas_amd as mb
from metalblas_amd import _lib, dispatch, planner

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "metalblas_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^[\w\s\*]+?\b(mb_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    names = _declared_functions()
    assert {"mb_gemm", "mb_plan", "mb_query", "mb_strerror"} <= set(names)
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/metalblas_amd.h but not exported"
    assert set(names) == set(_lib.EXPORTED_SYMBOLS)


def _c_layout():
    """sizeof/offsetof of the ABI structs, as the C compiler lays them out."""
    fields = {
        "mb_matrix": [f for f, _ in _lib.MbMatrix._fields_],
        "mb_gemm_desc": [f for f, _ in _lib.MbGemmDesc._fields_],
        "mb_plan_info": [f for f, _ in _lib.MbPlanInfo._fields_],
    }
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for s, fs in fields.items():
        lines.append(f'printf("{s} size %zu\\n", sizeof({s}));')
        for f in fs:
            lines.append(f'printf("{s} {f} %zu\\n", offsetof({s}, {f}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", "-o", exe, src], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    res = {}
    for ln in out.splitlines():
        s, f, v = ln.split()
        res[(s, f)] = int(v)
    return res


def test_ctypes_layout_matches_header():
    import oracle
    c = _c_layout()
    for s, cls in (("mb_matrix", _lib.MbMatrix), ("mb_gemm_desc", _lib.MbGemmDesc),
                   ("mb_plan_info", _lib.MbPlanInfo)):
        assert ctypes.sizeof(cls) == c[(s, "size")], s
        for f, _ in cls._fields_:
            assert getattr(cls, f).offset == c[(s, f)], f"{s}.{f}"
    # the oracle binds the same descriptor independently
    assert ctypes.sizeof(oracle.Desc) == c[("mb_gemm_desc", "size")]
    for f, _ in oracle.Desc._fields_:
        assert getattr(oracle.Desc, f).offset == c[("mb_gemm_desc", f)]


def test_strerror_and_status_mapping():
    for code in range(0, -9, -1):
        assert _lib.strerror(code) != "unknown status"
    assert _lib.strerror(-99) == "unknown status"
    _lib.check(0)
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_GEMV_SHAPE)
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_BAD_BACKEND)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.ERR_UNSUPPORTED_DTYPE)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_LAUNCH)


def _desc(dtype, a, b, c=None, batch=1, **kw):
    """Descriptor of CPU tensors (for planning only: nothing is launched)."""
    if c is None:
        shape = (a.shape[0], a.shape[1], b.shape[2]) if a.dim() == 3 else (a.shape[0], b.shape[1])
        c = torch.empty(shape, dtype=dtype)
    if a.dim() == 3:
        batch, M, K = a.shape
        N = b.shape[2]
    else:
        M, K = a.shape
        N = b.shape[1]
    return _lib.make_desc(dtype, batch, M, N, K, dispatch._mat(a), dispatch._mat(b), dispatch._mat(c), **kw)


def _plan(dtype, a, b, **kw):
    return _lib.plan(_desc(dtype, a, b, **kw))


def test_abi_rejects_bad_descriptors_before_launch():
    lib = _lib.load()
    a = torch.empty(8, 8, dtype=torch.float32)
    d = _desc(torch.float32, a, a)
    d.dtype = 42
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_UNSUPPORTED_DTYPE
    d = _desc(torch.float32, a, a, backend=_lib.BACKEND_GEMV)
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_GEMV_SHAPE
    d = _desc(torch.float32, a, a)
    d.backend = 17
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_BAD_BACKEND
    d = _desc(torch.float32, a, a)
    d.flags = 2                      # an unknown flag bit
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    # a dry run plans and returns without queuing work (host pointers never reach a kernel)
    d = _desc(torch.float32, a, a)
    d.flags = _lib.FLAG_DRY_RUN
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.OK
    d = _desc(torch.float32, a, a)
    d.M = -1
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    d = _desc(torch.float32, a, a)
    d.c.ptr = None
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    # an epilogue that reads the bias needs one
    d = _desc(torch.float32, a, a, epilogue=(1.0, 1.0, True, True))
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    # empty outputs are a successful no-op
    e = torch.empty(0, 8)
    d = _desc(torch.float32, e, a, c=torch.empty(0, 8))
    assert lib.mb_gemm(ctypes.byref(d), None) == 0
    # the library's internal flag bit (static scratch of mb_gemm_noalloc) is refused by every
    # entry point that takes a descriptor
    d = _desc(torch.float32, a, a)
    d.flags = 1 << 30
    info = _lib.MbPlanInfo()
    tiles = (ctypes.c_int32 * 64)()
    assert lib.mb_gemm(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    assert lib.mb_gemm_noalloc(ctypes.byref(d), None) == _lib.ERR_INVALID_ARG
    assert lib.mb_plan(ctypes.byref(d), ctypes.byref(info)) == _lib.ERR_INVALID_ARG
    assert lib.mb_gemm_workspace_bytes(ctypes.byref(d)) == _lib.ERR_INVALID_ARG
    assert lib.mb_tile_candidates(ctypes.byref(d), tiles, 8) == _lib.ERR_INVALID_ARG


# ---- planner decisions at the benchmark configurations (256 CUs assumed without a GPU) ---------

def test_plan_config3_square_bf16_uses_matrix_cores():
    a = torch.empty(8192, 8192, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, a, a)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and p.split_k == 1 and p.workspace_bytes == 0
    assert p.tile[0] * p.tile[1] >= 128 * 128


@pytest.mark.parametrize("layout", ["rm_rm", "rm_cm", "cm_rm", "cm_cm", "row_sliced"])
def test_plan_config3_layouts_use_matrix_cores(layout):
    M, K, N = 2048, 4096, 2048
    a = torch.empty(K, M, dtype=torch.bfloat16).t() if layout.startswith("cm") else \
        torch.empty(2 * M, K, dtype=torch.bfloat16)[::2] if layout == "row_sliced" else \
        torch.empty(M, K, dtype=torch.bfloat16)
    b = torch.empty(N, K, dtype=torch.bfloat16).t() if layout.endswith("cm") else torch.empty(K, N, dtype=torch.bfloat16)
    assert _lib.FAMILY_NAMES[_plan(torch.bfloat16, a, b).family] == "mfma"


def test_plan_config2_gemv_families():
    n = 16384
    W = torch.empty(n, n, dtype=torch.bfloat16)
    x = torch.empty(n, 1, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, W, x)
    assert _lib.FAMILY_NAMES[p.family] == "gemv_dot" and p.tile[2] == 1   # streaming kernel
    xt = torch.empty(1, n, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, xt, W)
    assert _lib.FAMILY_NAMES[p.family] == "gemv_axpy" and p.tile[2] == 1
    # x @ W streams W along its rows: split over K to fill 256 CUs, partials in the workspace
    assert p.split_k > 1 and p.workspace_bytes == p.split_k * n * 4
    # 8 vectors: the thin matrix-core tile 32 x 128 over K slices, two workgroups per CU
    X8 = torch.empty(8, n, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, X8, W)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and tuple(p.tile[:2]) == (32, 128)
    assert p.split_k * (n // 128) == 256
    # batched vectors with a short K: 32 x 128, no K slices; K = 1024 unsplit: 32 x 256
    p = _plan(torch.bfloat16, torch.empty(64, 8, 512, dtype=torch.bfloat16),
              torch.empty(64, 512, 4096, dtype=torch.bfloat16))
    assert tuple(p.tile[:2]) == (32, 128) and p.split_k == 1 and p.workspace_bytes == 0
    p = _plan(torch.bfloat16, torch.empty(128, 16, 1024, dtype=torch.bfloat16),
              torch.empty(128, 1024, 2048, dtype=torch.bfloat16))
    assert tuple(p.tile[:2]) == (32, 256) and p.split_k == 1
    # W @ X8: k_dotx over the whole K (16 waves x 1024), one 16-quad group per CU, the natural
    # 8-wide vector rows read in place: no copy, no K slices, no workspace
    Xn = torch.empty(n, 8, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, W, Xn)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and tuple(p.tile[:2]) == (4, 8) and p.split_k == 1
    assert p.workspace_bytes == 0 and p.block == 1024 and tuple(p.grid) == (256, 1, 1)
    # K-contiguous vectors stream in place too; 6 natural vectors are copied K-contiguous
    p = _plan(torch.bfloat16, W, torch.empty(8, n, dtype=torch.bfloat16).t())
    assert tuple(p.tile[:2]) == (4, 8) and p.workspace_bytes == 0
    p = _plan(torch.bfloat16, W, torch.empty(n, 6, dtype=torch.bfloat16))
    assert tuple(p.tile[:2]) == (4, 8) and p.workspace_bytes == n * 6 * 2
    # 8192 rows give 128 groups (half the CUs): k_thin_dot4 over K slices, the vector copy and
    # the K-slice planes in the workspace
    p = _plan(torch.bfloat16, torch.empty(8192, n, dtype=torch.bfloat16), Xn)
    assert tuple(p.tile[:2]) == (4, 16) and p.split_k == 4
    assert p.workspace_bytes == n * 8 * 2 + 4 * 8192 * 8 * 4
    # more than 8 vectors, or K past 16 x 1024: k_thin_dot4
    assert tuple(_plan(torch.bfloat16, W, torch.empty(n, 12, dtype=torch.bfloat16)).tile[:2]) == (4, 16)
    assert tuple(_plan(torch.bfloat16, torch.empty(n, 2 * n, dtype=torch.bfloat16),
                       torch.empty(2 * n, 8, dtype=torch.bfloat16)).tile[:2]) == (4, 16)
    # few vectors against a K-contiguous matrix stay on the VALU GEMV kernel
    assert _lib.FAMILY_NAMES[_plan(torch.bfloat16, W, torch.empty(n, 4, dtype=torch.bfloat16)).family] == "gemv_dot"
    # fp32 stays on the VALU kernels
    assert _lib.FAMILY_NAMES[_plan(torch.float32, torch.empty(8, n), torch.empty(n, n)).family] == "gemv_axpy"


def test_plan_narrow_x_at_w_fills_the_cus():
    # x @ W with 4096 columns: the thin matrix-core tile 32 x 128 over 8 K slices (32 tiles x 8
    # = 256 workgroups); a 0.5 GB matrix stays on the VALU stream
    W = torch.empty(4096, 4096, dtype=torch.bfloat16)
    x = torch.empty(1, 4096, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, x, W)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and tuple(p.tile[:2]) == (32, 128) and p.split_k == 8
    big = _plan(torch.bfloat16, torch.empty(1, 16384, dtype=torch.bfloat16), torch.empty(16384, 16384, dtype=torch.bfloat16))
    assert _lib.FAMILY_NAMES[big.family] == "gemv_axpy"
    # the VALU stream on request: two 2048-column bands (no band overhangs the rows), K slices
    # of 32 rows
    p = _plan(torch.bfloat16, x, W, backend=_lib.BACKEND_GEMV)
    assert _lib.FAMILY_NAMES[p.family] == "gemv_axpy"
    assert p.split_k == 128 and p.workspace_bytes == 128 * 4096 * 4


def test_plan_thin_problems_fill_two_workgroups_per_cu():
    def plan(M, N, K):
        p = _plan(torch.bfloat16, torch.empty(M, K, dtype=torch.bfloat16), torch.empty(K, N, dtype=torch.bfloat16))
        return tuple(p.tile[:2]), p.split_k
    assert plan(256, 4096, 4096) == ((64, 128), 4)     # 128 tiles x 4 K slices of 1024
    assert plan(8192, 128, 4096) == ((128, 64), 4)
    assert plan(512, 4096, 4096) == ((64, 128), 1)     # 256 tiles already fill the CUs
    assert plan(128, 4096, 4096) == ((128, 64), 8)     # the cost model's split plan stays
    assert plan(2048, 2048, 2048)[0] == (128, 128)     # not thin


def test_plan_both_operands_copied_pad_k_to_a_stage():
    # 4128 x 4128 x 4097 bf16: both operands are copied (odd leading dimensions, B a column
    # slice with row stride 4129); K is zero-padded to 4160 (a whole 64-deep stage) in both
    # copies: A 4128 x 4160, B 4160 x 4128
    a = torch.empty(4128, 4097, dtype=torch.bfloat16)
    b = torch.empty(4097, 4129, dtype=torch.bfloat16)[:, :4128]
    p = _plan(torch.bfloat16, a, b)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and p.split_k == 1
    assert p.workspace_bytes == 4128 * 4160 * 2 + 4160 * 4128 * 2


def test_plan_packed_peel():
    # 4097^3 bf16: both operands are copied anyway, so they are copied first (A 4097 x 4160, B
    # 4160 x 4104, B's last column K-contiguous 1 x 4160) and the product is peeled on the
    # copies: the plan reports the 4096^2 core on 256 whole 256 x 256 tiles; the workspace holds
    # the copies and then the largest part's own need; the tuner's candidates show that core
    # first (the static plan, run without a request) and whole-product tiles as its rivals (a
    # tile request turns the peeling off)
    a = torch.empty(4097, 4097, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, a, a)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and tuple(p.tile)[:2] == (256, 256)
    assert tuple(p.grid) == (256, 1, 1) and p.split_k == 1
    copies = (4097 * 4160 * 2 + 255) // 256 * 256 + 4160 * 4104 * 2 + (4160 * 2 + 255) // 256 * 256
    assert copies <= p.workspace_bytes <= copies + (8 << 20)
    d = _desc(torch.bfloat16, a, a)
    assert _lib.load().mb_gemm_workspace_bytes(ctypes.byref(d)) == p.workspace_bytes
    cands = _lib.tile_candidates(d, 24)
    assert cands[0][:2] == (256, 256) and len(cands) > 1
    assert all(_plan(torch.bfloat16, a, a, tile=c[:6]).workspace_bytes < p.workspace_bytes for c in cands[1:])
    # an explicit tile keeps the whole product (561 tiles of 256 x 128)
    p = _plan(torch.bfloat16, a, a, tile=(256, 128, 64, 2, 4, 2))
    assert tuple(p.tile)[:2] == (256, 128) and tuple(p.grid) == (561, 1, 1)
    # a core too small for 256 whole tiles stays one product
    a2, b2 = torch.empty(2056, 2051, dtype=torch.bfloat16), torch.empty(2051, 4100, dtype=torch.bfloat16)
    assert tuple(_plan(torch.bfloat16, a2, b2).tile)[:2] != (256, 256)


def test_plan_peels_a_thin_edge_off_whole_tiles():
    # 4097 x 4096 x 4096 bf16: the core 4096^2 runs on 256 whole 256 x 256 tiles (one round)
    # and row 4096 on the streaming GEMV; the plan reports the core, and the workspace is the
    # largest part's (the GEMV's split-K partial planes)
    a = torch.empty(4097, 4096, dtype=torch.bfloat16)
    b = torch.empty(4096, 4096, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, a, b)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and tuple(p.tile)[:2] == (256, 256)
    assert tuple(p.grid) == (256, 1, 1)
    d = _desc(torch.bfloat16, a, b)
    assert _lib.load().mb_gemm_workspace_bytes(ctypes.byref(d)) == p.workspace_bytes > 0
    # not peeled: a remainder above 16 rows, or an explicit tile
    a2 = torch.empty(4128, 4096, dtype=torch.bfloat16)
    assert tuple(_plan(torch.bfloat16, a2, b).grid) != (256, 1, 1)
    p = _plan(torch.bfloat16, a, b, tile=(256, 128, 64, 2, 4, 2))
    assert tuple(p.tile)[:2] == (256, 128)


def test_plan_config4_splitk_and_batches():
    a = torch.empty(1, 128, 65536, dtype=torch.float16)
    b = torch.empty(1, 65536, 128, dtype=torch.float16)
    p = _plan(torch.float16, a, b)
    assert _lib.FAMILY_NAMES[p.family] == "mfma" and p.split_k > 1
    assert p.workspace_bytes == p.split_k * 128 * 128 * 4
    # the deep-K schedule (tile[5] = schedule + 1 = 3) of the 64 x 64 tile: 4 tiles x 64 slices
    # of 1024 on a 1-D grid of 256 workgroups
    assert tuple(p.tile)[:2] == (64, 64) and p.tile[5] == 3 and p.split_k == 64
    assert tuple(p.grid) == (256, 1, 1)
    a = torch.empty(8, 512, 256, dtype=torch.float16)
    b = torch.empty(8, 256, 512, dtype=torch.float16)
    assert _lib.FAMILY_NAMES[_plan(torch.float16, a, b).family] == "mfma"
    bb = torch.empty(256, 512, dtype=torch.float16).expand(8, 256, 512)   # stride-0 batch
    assert _lib.FAMILY_NAMES[_plan(torch.float16, a, bb).family] == "mfma"


@pytest.mark.parametrize("shape", [(128, 128, 65536), (256, 256, 16384), (100, 200, 20000), (64, 64, 65536),
                                   (512, 512, 8192)], ids=str)
def test_plan_deep_k(shape):
    """Deep-K products (at most 64 tiles of 64 x 64, K >= 8192) take the deep-K schedule with
    K slices of >= 1024 and about one workgroup per CU; int8, shallow K, or more tiles do not."""
    M, N, K = shape
    a, b = torch.empty(M, K, dtype=torch.bfloat16), torch.empty(K, N, dtype=torch.bfloat16)
    p = _plan(torch.bfloat16, a, b)
    tiles = -(-M // 64) * -(-N // 64)
    assert p.tile[5] == 3 and tuple(p.tile)[:2] == (64, 64), tuple(p.tile)
    assert 2 <= p.split_k <= 256 // tiles and -(-K // p.split_k) >= 1024 - 63
    assert p.grid[0] == tiles * p.split_k and p.grid[1] == 1
    # the deep-K plan comes first; its rivals are the tile family (with its own K slices) and
    # the deep-K schedule at half and twice the slice count
    cands = _lib.tile_candidates(_desc(torch.bfloat16, a, b), 24)
    assert cands[0][5] == 3
    # (a request is listed only when it plans to exactly that many slices of whole stages)
    deep = sorted(c[6] for c in cands[1:] if c[5] == 3)
    assert deep and set(deep) <= {p.split_k // 2, 2 * p.split_k}, (deep, p.split_k)
    ai, bi = torch.empty(M, K, dtype=torch.int8), torch.empty(K, N, dtype=torch.int8)
    assert _plan(torch.int8, ai, bi).tile[5] != 3
    a2 = torch.empty(M, 4096, dtype=torch.bfloat16)
    assert _plan(torch.bfloat16, a2, torch.empty(4096, N, dtype=torch.bfloat16)).tile[5] != 3


def test_plan_config5_int8_and_complex():
    a = torch.empty(4096, 4096, dtype=torch.int8)
    assert _lib.FAMILY_NAMES[_plan(torch.int8, a, a).family] == "mfma"
    A = torch.empty(8192, 8192, dtype=torch.complex64)
    x = torch.empty(8192, 1, dtype=torch.complex64)
    assert _lib.FAMILY_NAMES[_plan(torch.complex64, A, x).family] == "gemv_dot"


def test_plan_config1_int32_small_generic_tiles():
    """Short-K integer products that 64 x 64 tiles leave underfilled run unsplit on 16 x 16 or
    32 x 32 tiles (one launch, no workspace); deep K keeps the K slices."""
    def gp(M, N, K):
        a, b = torch.empty(M, K, dtype=torch.int32), torch.empty(K, N, dtype=torch.int32)
        p = _plan(torch.int32, a, b)
        return _lib.FAMILY_NAMES[p.family], tuple(p.tile[:3]), p.split_k, p.workspace_bytes
    assert gp(256, 256, 256) == ("generic", (16, 16, 128), 1, 0)
    assert gp(512, 512, 512) == ("generic", (32, 32, 64), 1, 0)
    fam, tile, split, ws = gp(256, 256, 4096)
    assert tile == (64, 64, 16) and split > 1 and ws == split * 256 * 256 * 4
    assert gp(1024, 1024, 1024)[1:3] == ((64, 64, 16), 1)
    assert gp(64, 96, 80)[1:3] == ((64, 64, 16), 1)


def test_plan_complex_gemv_streams_rows():
    """complex64 W @ x with W K-contiguous and even K runs the workgroup-wide row stream (fast
    GEMV, one vector, no workspace); odd K keeps the generic complex dot kernel."""
    for M, K, fast in ((8192, 8192, 1), (3, 512, 1), (4096, 4095, 0)):
        A = torch.empty(M, K, dtype=torch.complex64)
        x = torch.empty(K, 1, dtype=torch.complex64)
        p = _plan(torch.complex64, A, x)
        assert _lib.FAMILY_NAMES[p.family] == "gemv_dot" and p.tile[0] == 1 and p.tile[2] == fast
        assert p.workspace_bytes == 0


def test_plan_k0_fill_and_empty():
    a = torch.empty(4, 0, dtype=torch.bfloat16)
    b = torch.empty(0, 5, dtype=torch.bfloat16)
    assert _lib.FAMILY_NAMES[_plan(torch.bfloat16, a, b).family] == "fill"
    a = torch.empty(0, 3, dtype=torch.bfloat16)
    b = torch.empty(3, 5, dtype=torch.bfloat16)
    assert _lib.FAMILY_NAMES[_plan(torch.bfloat16, a, b).family] == "none"


def test_plan_column_major_output_is_transposed_problem():
    a = torch.empty(256, 512, dtype=torch.bfloat16)
    b = torch.empty(512, 384, dtype=torch.bfloat16)
    c = torch.empty(384, 256, dtype=torch.bfloat16).t()
    p = _lib.plan(_desc(torch.bfloat16, a, b, c=c))
    assert p.transposed == 1


def test_tile_candidates_primary_first():
    a = torch.empty(4096, 4096, dtype=torch.bfloat16)
    d = _desc(torch.bfloat16, a, a)
    p = _lib.plan(d)
    cands = _lib.tile_candidates(d)
    assert len(cands) >= 2 and cands[0][:2] == tuple(p.tile[:2])
    assert len(set(c[:7] for c in cands)) == len(cands)


@pytest.mark.parametrize("shape", [(4096, 16, 4096), (256, 4096, 4096), (8, 16384, 16384), (1, 16384, 16384),
                                   (16384, 1, 16384), (16384, 8, 16384), (2048, 2048, 4096)], ids=str)
def test_tile_candidates_cross_families(shape):
    """The tuner's rivals span the kernel families (the reference times gemv_bt / flipt /
    sgpipe / split-K candidates against its tiles, metalblas/float_dispatch.py:439-481, 516-542):
    entry 0 is the static plan (zeros for a GEMV plan), every rival plans to exactly the tile and
    K slices it names, and no two entries plan alike."""
    M, N, K = shape
    a, b = torch.empty(M, K, dtype=torch.bfloat16), torch.empty(K, N, dtype=torch.bfloat16)
    d = _desc(torch.bfloat16, a, b)
    static = _lib.plan(d)
    cands = _lib.tile_candidates(d, 24)
    assert len(cands) >= 2, cands
    fam = _lib.FAMILY_NAMES[static.family]
    assert cands[0][:2] == (tuple(static.tile[:2]) if fam == "mfma" else (0, 0))
    seen = {(static.family, tuple(static.tile[:6]) if fam == "mfma" else (), static.split_k)}
    thin = {(4, 8), (4, 16), (64, 16), (32, 128), (32, 256)}
    kinds = set()
    for c in cands[1:]:
        p = _plan(torch.bfloat16, a, b, tile=c[:6], split_k=c[6])
        assert _lib.FAMILY_NAMES[p.family] == "mfma" and tuple(p.tile[:2]) == c[:2], (c, tuple(p.tile))
        assert c[6] == 0 or p.split_k == c[6]
        ident = (p.family, tuple(p.tile[:6]), p.split_k)
        assert ident not in seen, c
        seen.add(ident)
        kinds.add("thin" if c[:2] in thin else "split" if c[6] else "tile")
    if min(M, N) <= 32:
        assert "thin" in kinds or fam == "mfma" and tuple(static.tile[:2]) in thin
    if min(M, N) > 1 and max(M, N) > 32:
        assert "tile" in kinds


def test_tile_candidates_skip_small_tiles_on_large_products():
    # 8192^3: the static 256 x 256 tile gives every CU four tiles, so tiles of less than a
    # quarter of its area (128 x 64 and smaller, the register-staged 32 x 32) are not timed;
    # 2048 x 2048 x 4096 (one 128 x 128 tile per CU) keeps the whole family
    a = torch.empty(8192, 8192, dtype=torch.bfloat16)
    cands = _lib.tile_candidates(_desc(torch.bfloat16, a, a), 24)
    assert all(c[0] * c[1] * 4 >= 256 * 256 for c in cands) and len(cands) >= 5, cands
    a2, b2 = torch.empty(2048, 4096, dtype=torch.bfloat16), torch.empty(4096, 2048, dtype=torch.bfloat16)
    cands = _lib.tile_candidates(_desc(torch.bfloat16, a2, b2), 24)
    assert any(c[:2] == (64, 64) for c in cands) and any(c[:2] == (32, 32) for c in cands), cands
    # a short K keeps the small tiles (chained batch entries on them can win): bmm 192 x 512 x
    # 512 x 64
    a3, b3 = torch.empty(192, 512, 64, dtype=torch.bfloat16), torch.empty(192, 64, 512, dtype=torch.bfloat16)
    cands = _lib.tile_candidates(_desc(torch.bfloat16, a3, b3), 24)
    assert any(c[:2] == (64, 128) for c in cands), cands


# ---- Python layer: layouts, scalars, errors (metalblas/dispatch.py) ---------------------------

@pytest.mark.parametrize("dt", [torch.int8, torch.uint8, torch.bfloat16, torch.float16, torch.float32], ids=str)
def test_tile_candidates_are_compiled_tiles(dt):
    """Every autotune candidate names a tile compiled for the dtype: the 8-bit ping-pong
    schedule exists at 256 x 256 only (a 256 x 128 ping-pong candidate cannot launch)."""
    a = torch.empty(4096, 4096, dtype=dt)
    cands = _lib.tile_candidates(_desc(dt, a, a))
    assert len(cands) > 1
    for t in cands:
        if dt in (torch.int8, torch.uint8) and t[5] == 2:
            assert t[:2] == (256, 256), t
    # a forced 256 x 128 ping-pong tile snaps to a compiled 8-bit tile
    if dt in (torch.int8, torch.uint8):
        info = _plan(dt, a, a, backend=_lib.BACKEND_TILED, tile=(256, 128, 128, 2, 4, 2))
        assert not (info.tile[5] == 2 and info.tile[1] != 256), tuple(info.tile)


def test_unit_lead_classification():
    """metalblas/dispatch.py:23-35 on the benchmark's config-3 layouts."""
    M, K = 64, 96
    rm = torch.empty(M, K)
    assert dispatch._unit_lead(rm, M, K) == (False, K)
    cm = torch.empty(K, M).t()
    assert dispatch._unit_lead(cm, M, K) == (True, M)
    rows = torch.empty(2 * M, K)[::2]
    assert dispatch._unit_lead(rows, M, K) == (False, 2 * K)
    cols = torch.empty(M, 2 * K)[:, ::2]
    assert dispatch._unit_lead(cols, M, K) is None
    assert dispatch._matrix_view(cols, M, K).is_contiguous()
    off = torch.empty(M * K + 17)[17:].view(M, K)
    assert dispatch._unit_lead(off, M, K) == (False, K) and off.storage_offset() == 17
    assert dispatch._matrix_view(off, M, K).data_ptr() == off.data_ptr()   # no copy


def test_scalars_cast_like_reference():
    """metalblas/dispatch.py:127-131."""
    assert dispatch._scalars(torch.int32, 2.7, -1.2) == (2, -1, True, True)
    assert dispatch._scalars(torch.int8, 0.4, 1) == (0, 1, False, True)
    assert dispatch._scalars(torch.bfloat16, 1, 0) == (1.0, 0.0, True, False)
    beta, alpha, bnz, anz = dispatch._scalars(torch.complex64, 1j, 0)
    assert beta == 1j and alpha == 0 and bnz and not anz


def test_make_desc_fields():
    a = torch.empty(4 * 6 + 17)[17:].view(4, 6)
    b = torch.empty(5, 6).t()
    c = torch.empty(4, 5)
    d = _lib.make_desc(torch.float32, 1, 4, 5, 6, dispatch._mat(a), dispatch._mat(b), dispatch._mat(c),
                       epilogue=(0.5, -2, True, True), swizzle_log=2)
    assert d.a.ptr == a.data_ptr() and (d.a.row_stride, d.a.col_stride) == (6, 1)
    assert (d.b.row_stride, d.b.col_stride) == (1, 6)
    assert d.epilogue == 1 and d.beta_re == 0.5 and d.alpha_re == -2.0 and d.alpha_int == -2
    assert d.swizzle_log == 2
    assert _lib._wrap64(2 ** 64 - 1) == -1 and _lib._wrap64(-5) == -5


@pytest.mark.parametrize("op", ["matmul", "bmm", "addmm"])
def test_cpu_tensors_are_rejected(op):
    """The reference asserts its device (metalblas/dispatch.py:118,191); so does the drop-in:
    no silent CPU fallback."""
    a = torch.randn(4, 4)
    with pytest.raises(AssertionError):
        if op == "matmul":
            mb.matmul(a, a)
        elif op == "bmm":
            mb.bmm(a[None], a[None])
        else:
            mb.addmm(a, a, a)


def test_api_surface_matches_reference():
    """metalblas/__init__.py exports these names."""
    for name in ("matmul", "gemm", "addmm", "bmm", "baddbmm", "addbmm", "dot", "vdot", "outer",
                 "ger", "mv", "kernels"):
        assert hasattr(mb, name)
    assert mb.gemm is mb.matmul and mb.ger is mb.outer
    assert callable(mb.kernels.has_metal4)
    for bk in ("gemv", "mpp_tensor", "mpp", "simd", "auto", None):
        assert bk in dispatch.BACKENDS


def test_import_name_matches_reference():
    """``import metalblas`` (the reference's package name, /root/reference/pyproject.toml:6) exports
    the reference's names (metalblas/__init__.py:1-19), bound to this library."""
    import metalblas
    from metalblas.kernels import has_metal4
    assert sorted(metalblas.__all__) == sorted(mb.__all__)
    for name in metalblas.__all__:
        if name != "kernels":
            assert getattr(metalblas, name) is getattr(mb, name), name
    assert has_metal4 is mb.kernels.has_metal4


def test_autotune_probe_params_and_cache(tmp_path, monkeypatch):
    w0 = planner.probe_params(256, 256, 256)
    w2 = planner.probe_params(8192, 8192, 8192)
    assert w0[1] >= w2[1] and w0[0] >= w2[0]
    path = tmp_path / "plans.json"
    monkeypatch.setenv("METALBLAS_PLAN_CACHE", str(path))
    planner.clear()
    planner._PLANS["k1"] = (256, 256, 64, 2, 4, 0, 0, 0)
    planner._PLANS["k2"] = None
    planner._save_cache()
    saved = json.loads(path.read_text())
    assert saved["k1"][:2] == [256, 256] and saved["k2"] is None
    planner.clear()
    planner._load_cache()
    assert planner.cached()["k1"][:2] == (256, 256) and planner.cached()["k2"] is None
    # a second file is merged in when the variable names it; plans already held win
    other = tmp_path / "other.json"
    other.write_text(json.dumps({"k1": [64, 64, 64, 2, 2, 0, 0, 0], "k3": [128, 128, 64, 2, 2, 0, 0, 0]}))
    monkeypatch.setenv("METALBLAS_PLAN_CACHE", str(other))
    planner._load_cache()
    assert planner.cached()["k1"][:2] == (256, 256) and planner.cached()["k3"][:2] == (128, 128)
    planner.clear()


def test_autotune_switch(monkeypatch):
    """As the reference (metalblas/float_dispatch.py:156): on unless METALBLAS_AUTOTUNE=0."""
    monkeypatch.delenv("METALBLAS_AUTOTUNE", raising=False)
    assert planner.enabled()
    monkeypatch.setenv("METALBLAS_AUTOTUNE", "0")
    assert not planner.enabled()
    monkeypatch.setenv("METALBLAS_AUTOTUNE", "1")
    assert planner.enabled()
    monkeypatch.setenv("METALBLAS_AUTOTUNE", "yes")
    assert planner.enabled()


def test_tuner_skips_under_graph_capture(monkeypatch):
    """Timing candidates synchronises, which a HIP graph capture forbids: under capture the
    tuner leaves the descriptor's request alone and records nothing."""
    monkeypatch.delenv("METALBLAS_AUTOTUNE", raising=False)
    monkeypatch.setattr(torch._C, "_cuda_isCurrentStreamCapturing", lambda: True)
    planner.clear()
    d = _lib.make_desc(torch.bfloat16, 1, 4096, 4096, 4096, (None, 4096, 1, 0), (None, 4096, 1, 0),
                       (None, 4096, 1, 0))
    before = bytes(d)

    class Unused:
        def __getattr__(self, name):
            raise AssertionError(f"the tuner touched its output ({name}) under capture")
    planner.tune(d, None, None, Unused())
    assert bytes(d) == before and planner.cached() == {}


def test_tuner_scratch_keeps_output_layout():
    """Candidates are timed into scratch with the real output's strides and pointer alignment."""
    base = torch.empty(40 * 33 + 17, dtype=torch.bfloat16)
    out = base[17:].as_strided((33, 40), (1, 33))          # column-major at a 34-byte offset
    s = planner._like_out(out)
    assert s.shape == out.shape and s.stride() == out.stride()
    assert s.data_ptr() % 256 == out.data_ptr() % 256
    out3 = torch.empty(3, 64, 48, dtype=torch.complex64)[:, :, ::1]
    s3 = planner._like_out(out3)
    assert s3.stride() == out3.stride() and s3.data_ptr() % 256 == out3.data_ptr() % 256


def test_product_never_touches_the_oracle():
    """The oracle is test infrastructure: the package must not import, load or run it."""
    pkg = os.path.join(ROOT, "metalblas_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "from oracle" not in text, f
                assert "mb_oracle" not in text and "libmb_oracle" not in text, f


def test_trace_summary_keeps_the_last_dispatches(tmp_path):
    """perf.trace_summary: per-kernel statistics of a rocprofv3 CSV kernel trace, optionally over
    each kernel's last N dispatches (the timed steps after planning and warmup calls)."""
    from metalblas_amd import perf
    f = tmp_path / "t_kernel_trace.csv"
    f.write_text("Kernel_Name,Start_Timestamp,End_Timestamp\nk_a,100,1100\nk_a,2000,4000\n"
                 "k_b,5000,5500\nk_a,6000,7000\n")
    full = perf.trace_summary(str(f))
    assert "| `k_a` | 3 | 1.33 | 1.00 | 2.00 |" in full and "| `k_b` | 1 | 0.50 |" in full
    last = perf.trace_summary(str(f), last=2, names=["k_a"])
    assert "| `k_a` | 2 | 1.50 | 1.00 | 2.00 |" in last and "k_b" not in last


def test_pmc_summary_averages_the_last_dispatches(tmp_path):
    """perf.pmc_summary: per-counter means of a rocprofv3 --pmc CSV over a kernel's last N
    dispatches."""
    from metalblas_amd import perf
    f = tmp_path / "p_counter_collection.csv"
    rows = ["Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value"]
    for d, (a, b) in enumerate([(10, 1), (20, 2), (30, 3)], start=1):
        rows += [f"{d},k_gemm,SQ_A,{a}", f"{d},k_gemm,SQ_B,{b}", f"{d},other,SQ_A,999"]
    f.write_text("\n".join(rows) + "\n")
    s = perf.pmc_summary(str(f), "k_gemm", last=2)
    assert s["dispatches"] == 2 and s["SQ_A"] == 25 and s["SQ_B"] == 2.5
    assert perf.pmc_summary(str(f), "k_gemm")["SQ_A"] == 20


def test_counter_report_derives_clock_busy_and_traffic(tmp_path):
    """perf.counter_report: duration from the trace, clock from one counter run's own cycles and
    timestamps, matrix-core busy, conflicts per LDS instruction and the scaled HBM traffic, over
    the kernel's last N dispatches."""
    from metalblas_amd import perf
    tr = tmp_path / "run_kernel_trace.csv"
    tr.write_text("Kernel_Name,Start_Timestamp,End_Timestamp\n"
                  "k_x,0,5000\nk_x,10000,12000\nk_x,20000,22000\nother,0,9\n")
    sq = tmp_path / "sq.csv"
    rows = ["Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value,Start_Timestamp,End_Timestamp"]
    for d in (1, 2, 3):   # 2 us dispatches; 256 CUs x 4000 cycles -> 2 GHz; busy 1024 x 1000 / (1024 x 4000)
        rows += [f"{d},k_x,SQ_BUSY_CU_CYCLES,{256 * 4000},0,2000", f"{d},k_x,SQ_VALU_MFMA_BUSY_CYCLES,{1024 * 1000},0,2000",
                 f"{d},k_x,SQ_INSTS_LDS,100,0,2000", f"{d},k_x,SQ_LDS_BANK_CONFLICT,50,0,2000"]
    sq.write_text("\n".join(rows) + "\n")
    fe = tmp_path / "fetch.csv"
    fe.write_text("Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value\n1,k_x,FETCH_SIZE,1\n2,k_x,FETCH_SIZE,3\n3,k_x,FETCH_SIZE,3\n")
    wr = tmp_path / "write.csv"
    wr.write_text("Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value\n1,k_x,WRITE_SIZE,2\n2,k_x,WRITE_SIZE,2\n3,k_x,WRITE_SIZE,2\n")
    r = perf.counter_report(str(tr), [str(sq), str(fe), str(wr)], "k_x", 2, alg_bytes=8192)
    assert r["dispatches"] == 2 and r["us"] == 2.0
    assert abs(r["ghz"] - 2.0) < 1e-9 and abs(r["mfma_busy"] - 0.25) < 1e-12
    assert r["lds_conflict_per_inst"] == 0.5
    assert r["fetch_bytes"] == 3 * 1024 * 2 and r["write_bytes"] == 2 * 1024 and r["traffic_x_alg"] == 1.0


def test_chained_batch_plans():
    """Short-K batched products on small matrix-core tiles run on fewer z-blocks than batch
    entries (each workgroup streams the stages of several entries); more than four stages, a
    tile whose staged output does not fit one stage, an 8-bit tile, or too few tiles keep one
    z-block per entry."""
    def z(B, M, N, K, tile, dtype=torch.bfloat16):
        a = torch.empty(1, dtype=dtype)
        d = _lib.make_desc(dtype, B, M, N, K, (a, K, 1, M * K), (a, N, 1, K * N), (a, N, 1, M * N), tile=tile)
        p = _lib.plan(d)
        assert tuple(p.tile[:2]) == tile
        return p.grid[2]
    assert z(96, 512, 512, 64, (64, 128)) == 32           # 3072 tiles: 3 entries per workgroup
    assert z(48, 2048, 2048, 64, (128, 64)) == 3          # at most 16 entries per workgroup
    assert z(96, 512, 512, 128, (64, 128)) == 32          # two stages
    assert z(96, 512, 512, 320, (64, 128)) == 96          # five stages
    assert z(96, 512, 512, 64, (128, 128)) == 96          # staged 128 x 128 output > one stage
    assert z(8, 512, 512, 64, (64, 128)) == 8             # too few tiles
    assert z(192, 512, 512, 128, (128, 128), torch.int8) == 192   # 16-bit tiles only
