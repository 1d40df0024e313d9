"""HIP graph capture (torch.cuda.graph) of the library's products.

A product planned and tuned eagerly is captured and replayed several times, with eager work of
the program between the replays (other products on the same stream, which reuse the kept
scratch, and new input values), and every replay must equal the eager result bit for bit (the
same plan and kernels run).  The cases cover products with scratch: split-K planes, GEMV K-slice
planes and their reduction, the complex expansion and operand copies, whose workspace under
capture comes from the graph's private pool.  A signature first seen under capture runs its
static plan (the tuner synchronises and does not run then) and is not cached, so a later eager
call still tunes it.  The graphs hold only the library's launches and torch allocations, no
memset nodes.
"""
import pytest
import torch

import metalblas_amd as mb
from metalblas_amd import dispatch
from helpers import assert_parity, gen, rand

pytestmark = pytest.mark.gpu


def _gemm(dev, g):
    a = rand((1024, 1024), torch.bfloat16, g).to(dev)
    b = rand((1024, 1024), torch.bfloat16, g).to(dev)
    return [a, b], lambda: mb.matmul(a, b)


def _split_k(dev, g):
    a = rand((128, 65536), torch.float16, g).to(dev)
    b = rand((65536, 128), torch.float16, g).to(dev)
    return [a, b], lambda: mb.matmul(a, b)


def _gemv_xw(dev, g):
    x = rand((1, 8192), torch.bfloat16, g).to(dev)
    W = rand((8192, 8192), torch.bfloat16, g).to(dev)
    return [x, W], lambda: mb.matmul(x, W)


def _thin_x8w(dev, g):
    X = rand((8, 8192), torch.bfloat16, g).to(dev)
    W = rand((8192, 8192), torch.bfloat16, g).to(dev)
    return [X, W], lambda: mb.matmul(X, W)


def _addmm(dev, g):
    bias = rand((768,), torch.bfloat16, g).to(dev)
    a = rand((512, 2048), torch.bfloat16, g).to(dev)
    b = rand((2048, 768), torch.bfloat16, g).to(dev)
    return [bias, a, b], lambda: mb.addmm(bias, a, b, beta=0.5, alpha=2.0)


def _bmm(dev, g):
    a = rand((8, 512, 256), torch.float16, g).to(dev)
    b = rand((8, 256, 512), torch.float16, g).to(dev)
    return [a, b], lambda: mb.bmm(a, b)


def _complex_conj(dev, g):
    a = rand((512, 512), torch.complex64, g).to(dev)
    b = rand((512, 512), torch.complex64, g).to(dev)
    return [a, b], lambda: mb.matmul(a.conj(), b)


def _offset_copies(dev, g):
    # a [1:, 1:] view: misaligned rows, both operands copied into the workspace
    a = rand((1025, 1025), torch.bfloat16, g).to(dev)
    b = rand((1025, 1025), torch.bfloat16, g).to(dev)
    return [a, b], lambda: mb.matmul(a[1:, 1:], b[1:, 1:])


def _int8(dev, g):
    a = rand((512, 512), torch.int8, g).to(dev)
    b = rand((512, 512), torch.int8, g).to(dev)
    return [a, b], lambda: mb.matmul(a, b)


CASES = {"gemm_bf16": _gemm, "split_k_f16": _split_k, "gemv_x@W": _gemv_xw, "thin_X8@W": _thin_x8w,
         "addmm_bf16": _addmm, "bmm_f16": _bmm, "complex64_conj": _complex_conj,
         "offset_copies": _offset_copies, "int8": _int8}


@pytest.fixture(scope="module")
def other_work(dev):
    """Eager products to run between replays: a split-K product and a 16384^2 GEMV whose K-slice
    planes (8 MiB) outgrow any case's scratch, so the kept scratch of the stream is replaced
    (and the old block freed) while the graphs live."""
    a = torch.randn(128, 65536, device=dev, dtype=torch.float16)
    b = torch.randn(65536, 128, device=dev, dtype=torch.float16)
    x = torch.randn(1, 16384, device=dev, dtype=torch.bfloat16)
    W = torch.randn(16384, 16384, device=dev, dtype=torch.bfloat16)

    def run():
        mb.matmul(a, b)
        mb.matmul(x, W)
    return run


@pytest.mark.parametrize("case", list(CASES))
def test_graph_replays_match_eager(dev, case, other_work):
    g = gen(list(CASES).index(case))
    inputs, fn = CASES[case](dev, g)
    print(f"graph case {case}", flush=True)
    fn()                                   # plans and tunes the signature eagerly
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):          # warm-up on a side stream, as torch.cuda.graph asks
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    torch.cuda.synchronize()
    for rep in range(3):
        if rep:                            # new input values, copied in place
            for t in inputs:
                t.copy_(rand(tuple(t.shape), t.dtype, g).to(dev))
        other_work()
        torch.cuda.synchronize()
        want = fn().clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"{case}: replay {rep} differs from the eager call"
    del graph


def test_signature_first_seen_under_capture(dev):
    """A product first called during capture runs its static plan, stays out of the descriptor
    cache, and replays to within the parity bar of the oracle; the next eager call tunes it."""
    g = gen(7)
    a = rand((1000, 1536), torch.bfloat16, g)
    b = rand((1536, 1100), torch.bfloat16, g)
    ad, bd = a.to(dev), b.to(dev)
    mb.matmul(rand((64, 64), torch.bfloat16, g).to(dev), rand((64, 64), torch.bfloat16, g).to(dev))
    torch.cuda.synchronize()
    n_cached = len(dispatch._DESC_CACHE)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = mb.matmul(ad, bd)
    assert len(dispatch._DESC_CACHE) == n_cached
    for _ in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(out, a, b, tag="captured first call")
    eager = mb.matmul(ad, bd)              # tunes and caches now
    torch.cuda.synchronize()
    assert len(dispatch._DESC_CACHE) in (n_cached + 1, 1)   # 1: the insert cleared a full cache
    assert_parity(eager, a, b, tag="eager after capture")
    del graph
