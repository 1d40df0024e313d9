"""GPU parity at every benchmark workload, through the exact calls bench.py times.

Each case builds bench.py's workload group (the same seeds, shapes, operand layouts, ``out=``
buffers and API entry points), runs the benched call once, and checks the output with
``assert_parity_full``: the CPU oracle on spread sampled rows (the first and last batch of a
batched product), a float64 / complex128 GPU product pinned to the oracle on those rows, and
every element of the output against that product to the parity bar (integers bit-exact).
The check semantics follow the reference's tests/test_basic.py:53-69 at the north star's
tolerances (tests/helpers.py).

Extra cases beyond the benched calls: the 8192^3 product in the other three operand orders,
addmm in every config-3 layout, the config-4 split-K shape as a 2-D product, and config 1 at its
stated value range.
"""
import functools

import pytest
import torch

import bench
import metalblas_amd as mb
from helpers import assert_parity_full, gen

pytestmark = pytest.mark.gpu

NAMES = [n for g in bench.WORKLOADS for n in bench.WORKLOADS[g]]
GROUP_OF = {n: g for g in bench.WORKLOADS for n in bench.WORKLOADS[g]}

# oracle rows per workload: more where a row is cheap, fewer on the 8192-wide headline
ROWS = {"bf16_gemm_8192": 8, "gemv_x@W": 1, "gemv_Wt@x": 48, "gemv_X8@W": 3, "c64_gemm_2048_conjA": 24,
        "i8_gemm_4096": 24}


@functools.lru_cache(maxsize=1)
def _group(name):
    """bench.py's workload group, built once and kept while its cases run (parametrised cases
    run in order, so one group is alive at a time)."""
    torch.cuda.empty_cache()
    return {w.name: w for w in bench.GROUPS[name](torch, mb)}


@pytest.mark.parametrize("name", NAMES)
def test_config(dev, name):
    w = _group(GROUP_OF[name])[name]
    out = w.call()
    torch.cuda.synchronize()
    view, a, b, kw = w.check
    got = view(out).clone()      # benched calls reuse one out= buffer
    print(f"config {w.cfg} {name}: output {tuple(got.shape)} {got.dtype}", flush=True)
    assert_parity_full(got, a, b, rows=ROWS.get(name, 32), tag=name, **kw)
    # a second call through the cached launch plan gives the same bits
    again = view(w.call()).clone()
    torch.cuda.synchronize()
    assert torch.equal(again, got), f"{name}: a repeated call differs"


@pytest.mark.parametrize("layout", ["rm_cm", "cm_rm", "cm_cm"])
def test_headline_other_layouts(dev, layout):
    """bf16 8192^3 with the operands in the other three orders (both K-contiguous, A M-contiguous,
    both M/N-contiguous): each runs its own loader variant of the 256 x 256 schedule."""
    _group.cache_clear()
    torch.cuda.empty_cache()
    n = 8192
    g = gen(0)
    a = torch.randn(n, n, generator=g).to(torch.bfloat16).cuda()
    b = torch.randn(n, n, generator=g).to(torch.bfloat16).cuda()
    if layout[:2] == "cm":
        a = a.t()
    if layout[3:] == "cm":
        b = b.t()
    got = mb.matmul(a, b)
    assert_parity_full(got, a, b, rows=6, tag=f"8192^3 {layout}")


@pytest.mark.parametrize("layout", ["rm_cm", "cm_rm", "cm_cm", "row_sliced", "col_sliced", "offset17"])
def test_config3_addmm_layouts(dev, layout):
    """Config 3's addmm (bias 2048, beta 0.5, alpha 2) on every operand layout."""
    _group.cache_clear()
    views, (_, bias) = bench.layout_views(torch)
    (_, _), (a, b) = views[layout]
    got = mb.addmm(bias, a, b, beta=0.5, alpha=2.0)
    assert_parity_full(got, a, b, bias=bias, beta=0.5, alpha=2.0, rows=24, tag=f"addmm {layout}")


def test_config4_splitk_2d(dev):
    """The split-K shape as a plain 2-D product (M = N = 128, K = 65536), matmul and addmm."""
    g = gen(4)
    a = torch.randn(128, 65536, generator=g).to(torch.float16).cuda()
    b = torch.randn(65536, 128, generator=g).to(torch.float16).cuda()
    assert_parity_full(mb.matmul(a, b), a, b, rows=16, tag="split-K 2-D")
    bias = torch.randn(128, generator=g).to(torch.float16).cuda()
    got = mb.addmm(bias, a, b, beta=0.5, alpha=2.0)
    assert_parity_full(got, a, b, bias=bias, beta=0.5, alpha=2.0, rows=16, tag="split-K addmm")


def test_config1_value_range(dev):
    """Config 1 as stated: int32 256 x 256 @ 256 x 256, entries uniform in [-8, 8], and the
    extreme case of every entry at +/-8 (bit-exact)."""
    g = gen(1)
    a = torch.randint(-8, 9, (256, 256), generator=g, dtype=torch.int32).cuda()
    b = torch.randint(-8, 9, (256, 256), generator=g, dtype=torch.int32).cuda()
    assert_parity_full(mb.matmul(a, b), a, b, rows=256, tag="cfg1")
    s = torch.full((256, 256), 8, dtype=torch.int32, device=dev)
    s[::2] = -8
    assert_parity_full(mb.matmul(s, s), s, s, rows=256, tag="cfg1 extremes")
