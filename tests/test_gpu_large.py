"""Products past 32-bit element counts and past the LDS-direct loaders' 31-bit operand offsets.

Every kernel family addresses operands and outputs with 64-bit element offsets; the LDS-direct
and thin kernels address each operand tile through 31-bit byte offsets and hand larger spans to
the register-staged and VALU kernels.  These cases reach those limits:
  * an output of 2^31 elements (the last rows sit past 2^31 elements from the base);
  * leading dimensions of 2^21 + 64 elements (a 256-row tile spans more than 2^30 bytes) in
    both orientations, and of 2^24 + 64 (every tile does), and a batch stride past 2^31
    elements;
  * GEMV and thin products on a matrix of 2^31 elements.
The GEMM cases are checked against the oracle on sampled rows (first and last included).  The
GEMV cases use integer-valued bf16 inputs whose fp32 sums are exact (|sum| < 2^24), so the
result must equal the exact product rounded once to bf16, bit for bit; the exact product is a
float64 product on the GPU, taken in row chunks.
"""
import pytest
import torch

import metalblas_amd as mb
import oracle
from helpers import assert_parity, check_values, gen, rand, sample_rows

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _need(dev, gib):
    free, _ = torch.cuda.mem_get_info(dev)
    if free < gib * (1 << 30):
        pytest.skip(f"needs {gib} GiB of free device memory")


def _rows_vs_oracle(got, a, b, tag):
    rows = sample_rows(a.shape[0], 24)
    ref, exact = oracle.gemm(a, b, rows=rows)
    sel = got[torch.tensor(rows, device=got.device)].cpu()
    check_values(sel, ref, exact, got.dtype, a.shape[1], tag=tag)


def test_output_past_2g_elements(dev):
    _need(dev, 8)
    g = gen(1)
    M, N, K = 65536, 32768, 64                       # C: 2^31 elements (4 GiB of bf16)
    a, b = rand((M, K), BF, g), rand((K, N), BF, g)
    print(f"large: output {M} x {N}, K {K}", flush=True)
    c = mb.matmul(a.to(dev), b.to(dev))
    torch.cuda.synchronize()
    _rows_vs_oracle(c, a, b, "2^31-element output")
    del c
    torch.cuda.empty_cache()


def _strided_copy(src, ld, dev, transpose):
    """src (r x c) on the GPU as a view with leading dimension ld: row-major rows of ld
    elements, or (transpose) the transposed view of a row-major (c x ld) buffer."""
    r, c = src.shape
    if transpose:
        buf = torch.empty(c, ld, dtype=src.dtype, device=dev)
        buf[:, :r] = src.t().to(dev)
        return buf[:, :r].t()
    buf = torch.empty(r, ld, dtype=src.dtype, device=dev)
    buf[:, :c] = src.to(dev)
    return buf[:, :c]


# ld 2^21 + 64: a 256-row tile spans more than 2^30 bytes (smaller tiles still fit);
# ld 2^24 + 64: every tile does (32 rows of 32 MiB)
@pytest.mark.parametrize("dtype,layout,ld", [(BF, "rm_rm", (1 << 21) + 64), (BF, "cm_cm", (1 << 21) + 64),
                                             (torch.float16, "rm_cm", (1 << 21) + 64),
                                             (torch.int8, "rm_rm", (1 << 21) + 64), (BF, "rm_rm", (1 << 24) + 64)])
def test_leading_dimension_past_loader_offsets(dev, dtype, layout, ld):
    M, N, K = (512, 768, 1024) if ld < (1 << 24) else (256, 256, 512)
    _need(dev, 2 + (M + K) * ld * dtype.itemsize / (1 << 30))
    g = gen(2)
    a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    print(f"large: {dtype} {layout} ld {ld}", flush=True)
    ad = _strided_copy(a, ld, dev, layout[0] == "c")
    bd = _strided_copy(b, ld, dev, layout[3] == "c")
    assert max(ad.stride()) == ld and max(bd.stride()) == ld
    got = mb.matmul(ad, bd)
    torch.cuda.synchronize()
    assert_parity(got, a, b, tag=f"ld {ld} {layout}")
    del ad, bd, got
    torch.cuda.empty_cache()


def test_batch_stride_past_2g_elements(dev):
    _need(dev, 14)
    g = gen(3)
    B, M, N, K = 3, 256, 512, 768
    S = (1 << 31) + 4096                             # batch stride of A, in elements
    a, b = rand((B, M, K), BF, g), rand((B, K, N), BF, g)
    print(f"large: bmm with batch stride {S}", flush=True)
    buf = torch.empty(B * S, dtype=BF, device=dev)
    ad = buf.as_strided((B, M, K), (S, K, 1))
    ad.copy_(a.to(dev))
    got = mb.bmm(ad, b.to(dev))
    torch.cuda.synchronize()
    assert_parity(got, a, b, tag="batch stride past 2^31")
    del buf, ad, got
    torch.cuda.empty_cache()


def _exact_rows(W, X, chunk=8192):
    """W @ X in float64, in row chunks of W, rounded once to bf16."""
    return torch.cat([W[i:i + chunk].double() @ X.double() for i in range(0, W.shape[0], chunk)]).to(BF)


def _exact_cols(Y, W, chunk=8192):
    """Y @ W in float64, summed over row chunks of W, rounded once to bf16."""
    acc = None
    for i in range(0, W.shape[0], chunk):
        p = Y[..., i:i + chunk].double() @ W[i:i + chunk].double()
        acc = p if acc is None else acc + p
    return acc.to(BF)


def test_gemv_and_thin_on_a_2g_element_matrix(dev):
    _need(dev, 16)
    gd = torch.Generator(device=dev).manual_seed(4)
    R, C = 65536, 32768                               # W: 2^31 elements (4 GiB of bf16)

    def ints(*shape):
        return torch.randint(-4, 4, shape, generator=gd, device=dev, dtype=torch.int8).to(BF)

    W = ints(R, C)
    cases = [("W @ x", lambda: mb.matmul(W, xc), lambda: _exact_rows(W, xc)),
             ("x @ W", lambda: mb.matmul(xr, W), lambda: _exact_cols(xr, W)),
             ("W @ X8", lambda: mb.matmul(W, X8c), lambda: _exact_rows(W, X8c)),
             ("X8 @ W", lambda: mb.matmul(X8r, W), lambda: _exact_cols(X8r, W))]
    xc, xr = ints(C), ints(R)
    X8c, X8r = ints(C, 8), ints(8, R)
    for name, run, exact in cases:
        print(f"large: {name} on {R} x {C}", flush=True)
        got = run()
        torch.cuda.synchronize()
        want = exact()
        assert got.shape == want.shape, name
        assert torch.equal(got, want), f"{name}: {(got != want).sum().item()} outputs differ from the exact product"
    del W
    torch.cuda.empty_cache()
