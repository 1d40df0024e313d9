"""mb_gemm_noalloc: the allocation-free entry point (static per-device scratch) against mb_gemm.

Every case is a product that needs scratch (split-K partial planes, GEMV partial planes, an
operand copy, the complex expansion, the thin-product vector copy and reduction).  Each runs
through the C ABI twice in a row, the second time with a smaller input, and each output must
equal bit for bit what mb_gemm gives for the same descriptor with a torch-allocated workspace
(the same plan and kernels run).  A product that needs more than the static buffer is refused
before anything is queued.
"""
import ctypes

import pytest
import torch

from metalblas_amd import _lib
from helpers import gen, rand

pytestmark = pytest.mark.gpu


def _mat(t):
    if t.dim() == 3:
        return (t, t.stride(1), t.stride(2), t.stride(0))
    return (t, t.stride(0), t.stride(1), 0)


def _desc(a, b, out, *, bias=None, epilogue=None, conj_a=False):
    batch = a.shape[0] if a.dim() == 3 else 1
    M, K = a.shape[-2:]
    N = b.shape[-1]
    return _lib.make_desc(out.dtype, batch, M, N, K, _mat(a), _mat(b), _mat(out),
                          _mat(bias) if bias is not None else None, epilogue=epilogue, conj_a=conj_a)


def _stream():
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device())


def _noalloc(d):
    return _lib.load().mb_gemm_noalloc(ctypes.byref(d), _stream())


def _split_k(dev, g, big):
    K = 65536 if big else 16384
    a = rand((128, K), torch.float16, g).to(dev)
    b = rand((K, 128), torch.float16, g).to(dev)
    return a, b, {}


def _split_k_addmm(dev, g, big):
    a, b, _ = _split_k(dev, g, big)
    bias = rand((128,), torch.float16, g).to(dev).expand(128, 128)
    return a, b, {"bias": bias, "epilogue": (0.5, 2.0, True, True)}


def _gemv_xw(dev, g, big):
    n = 16384 if big else 4096
    x = rand((1, n), torch.bfloat16, g).to(dev)
    W = rand((n, n), torch.bfloat16, g).to(dev)
    return x, W, {}


def _col_sliced(dev, g, big):
    M, K, N = (2048, 4096, 2048) if big else (1024, 2048, 768)
    a = rand((M, 2 * K + 3), torch.bfloat16, g).to(dev)[:, 3:][:, :K]     # odd leading dimension
    b = rand((K, N), torch.bfloat16, g).to(dev)
    return a, b, {}


def _complex(dev, g, big):
    n = 2048 if big else 512
    a = rand((n, n), torch.complex64, g).to(dev)
    b = rand((n, n), torch.complex64, g).to(dev)
    return a, b, {"conj_a": True}


def _thin(dev, g, big):
    # matrices of 8192 / 4096 rows: k_thin_dot4 over K slices (the vector copy and the K-slice
    # planes in scratch); at 16384 rows the whole-K kernel needs no scratch
    m, n = (8192, 16384) if big else (4096, 4096)
    W = rand((m, n), torch.bfloat16, g).to(dev)
    X = rand((n, 8), torch.bfloat16, g).to(dev)
    return W, X, {}


def _packed_peel(dev, g, big):
    # odd leading dimensions copy both operands; with N = 4097 the product is peeled after the
    # copies (the core on whole 256 x 256 tiles, the last column on the dot GEMV), and copies
    # plus parts fit the static buffer (34.6 MB), so noalloc runs the same peeled plan.  The
    # second call (2049^3, 17 MB of copies) is unpeeled.
    M, N, K = (4096, 4097, 2049) if big else (2049, 2049, 2049)
    a = rand((M, K), torch.bfloat16, g).to(dev)
    b = rand((K, N), torch.bfloat16, g).to(dev)
    return a, b, {}


CASES = {"split_k": _split_k, "split_k_addmm": _split_k_addmm, "gemv_x@W": _gemv_xw,
         "operand_copy": _col_sliced, "complex64_conj": _complex, "thin_W@X8": _thin,
         "packed_peel": _packed_peel}


@pytest.mark.parametrize("case", list(CASES))
def test_noalloc_matches_mb_gemm(dev, case):
    g = gen(hash(case) % 1000)
    limit = _lib.load().mb_gemm_noalloc_scratch_bytes()
    assert limit == 64 << 20
    for big in (True, False):          # two calls in a row, the second one smaller
        a, b, kw = CASES[case](dev, g, big)
        M, N = a.shape[-2], b.shape[-1]
        out = torch.empty(M, N, dtype=a.dtype, device=dev)
        d = _desc(a, b, out, **kw)
        need = _lib.workspace_bytes(d)
        assert 0 < need <= limit, (case, big, need)
        print(f"noalloc {case} {'big' if big else 'small'} {tuple(a.shape)} @ {tuple(b.shape)} "
              f"scratch {need} B", flush=True)
        assert _noalloc(d) == _lib.OK
        want = torch.empty_like(out)
        d2 = _desc(a, b, want, **kw)
        _lib.run(d2, dev)              # mb_gemm with a torch-allocated workspace
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"{case}: mb_gemm_noalloc differs from mb_gemm"


def test_noalloc_refuses_beyond_its_buffer(dev):
    """complex64 4096^3 needs a 256 MiB expansion of B: refused, nothing queued."""
    g = gen(5)
    a = rand((4096, 4096), torch.complex64, g).to(dev)
    b = rand((4096, 4096), torch.complex64, g).to(dev)
    out = torch.full((4096, 4096), 7 + 7j, dtype=torch.complex64, device=dev)
    d = _desc(a, b, out)
    assert _lib.workspace_bytes(d) > _lib.load().mb_gemm_noalloc_scratch_bytes()
    assert _noalloc(d) == _lib.ERR_SCRATCH_LIMIT
    torch.cuda.synchronize()
    assert bool((out == (7 + 7j)).all())
    assert "static buffer" in _lib.strerror(_lib.ERR_SCRATCH_LIMIT)


def test_noalloc_flags(dev):
    g = gen(6)
    a = rand((128, 65536), torch.float16, g).to(dev)
    b = rand((65536, 128), torch.float16, g).to(dev)
    out = torch.empty(128, 128, dtype=torch.float16, device=dev)
    d = _desc(a, b, out)
    d.flags = _lib.FLAG_DRY_RUN
    assert _noalloc(d) == _lib.OK
    d.flags = 2
    assert _noalloc(d) == _lib.ERR_INVALID_ARG
    d.flags = 1 << 30                   # the library's internal bit is not accepted from callers
    assert _lib.load().mb_gemm(ctypes.byref(d), _stream()) == _lib.ERR_INVALID_ARG
    assert _noalloc(d) == _lib.ERR_INVALID_ARG
