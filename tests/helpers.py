"""Shared test helpers: seeded inputs, oracle products and the parity bar.

The bar (north star of this build, on top of the reference's own checks in
tests/test_basic.py:45-69):
  * integers: bit-exact against the oracle (which wraps like tests/test_basic.py:27-34);
  * bf16 / fp16: |got - exact| <= scale * 1e-2 * sqrt(K / 1024) + 1e-2 * |exact| elementwise,
    exact = fp64 product; and the reference's own limit max|got - round(exact)| <=
    scale * _atol(dtype, K) (tests/test_basic.py:45-50, 65-68);
  * fp32: |got - exact| <= scale * max(1e-3, 1e-5 * K) + 1e-5 * |exact| (the reference's
    strict fp32 limit, tests/test_basic.py:47, plus a relative term for large outputs);
  * complex64: elementwise |got - exact| <= 1e-4 * (|exact| + rms(exact)) (the north star's
    rtol 1e-4; the absolute term, 1e-4 of the output's RMS magnitude, keeps near-zero outputs
    of a long fp32 sum from being held to a pure relative limit: the fp32 accumulation error
    of an element grows with the magnitude of the partial sums, i.e. with the output scale,
    not with the element), and max|got - exact| / max|exact| <= 1e-4 (the reference's
    normalised form, tests/test_basic.py:62, at the north star's limit); complex32: the
    normalised form <= 3e-2 (tests/test_basic.py:63).
``scale`` is |alpha| + |beta| for fused ops (tests/test_basic.py:137).
"""
from __future__ import annotations

import math

import torch

import oracle

INTS = (torch.int8, torch.uint8, torch.int16, torch.int32, torch.int64)
FLOATS = (torch.float32, torch.float16, torch.bfloat16)
COMPLEX = (torch.complex64, torch.complex32)
ALL = FLOATS + COMPLEX + INTS

# oracle work above which rows / batches are sampled
FULL_LIMIT = 1 << 23


def gen(seed=0):
    return torch.Generator().manual_seed(seed)


def rand(shape, dtype, g):
    """CPU tensor like tests/test_basic.py:20-24 (ints in [-4, 4), uint8 in [0, 4))."""
    if dtype in INTS:
        lo = 0 if dtype is torch.uint8 else -4
        return torch.randint(lo, 4, shape, dtype=dtype, generator=g)
    if dtype is torch.complex32:
        return torch.randn(shape, dtype=torch.complex64, generator=g).to(torch.complex32)
    return torch.randn(shape, dtype=dtype, generator=g)


def ref_limit_atol(dtype, k, strict=False):
    """tests/test_basic.py:45-50."""
    if dtype is torch.float32:
        return max(1e-3, 1e-5 * k) if strict else max(0.1, 5e-3 * k ** 0.5)
    if dtype is torch.bfloat16:
        return max(0.5, 3e-2 * k ** 0.5)
    return max(5e-2, 1e-2 * k ** 0.5)


def sample_rows(M, count=24):
    if M <= count:
        return list(range(M))
    step = M / count
    rows = sorted({0, M - 1, *[int(i * step) for i in range(count)]})
    return rows


def oracle_product(a, b, *, bias=None, beta=None, alpha=None, force_full=False):
    """Oracle on CPU copies; samples rows (2-D) or batches (3-D) above FULL_LIMIT.

    Returns (index, c, exact): index selects the compared part of the full output
    (None = everything)."""
    a, b = a.cpu(), b.cpu()
    bias = bias.cpu() if bias is not None else None
    if a.dim() == 3:
        Bb, M, K = a.shape
        N = b.shape[2]
        work = Bb * M * N * K
        if force_full or work <= FULL_LIMIT:
            c, e = oracle.gemm(a, b, bias=bias, beta=beta, alpha=alpha)
            return None, c, e
        per = M * N * K
        nb = max(1, min(Bb, FULL_LIMIT // max(per, 1)))
        idx = sorted({0, Bb - 1, *range(0, Bb, max(1, Bb // nb))})[:max(2, nb)]
        idx_t = torch.tensor(idx)
        bx = None
        if bias is not None:
            bx = bias.expand(Bb, M, N)[idx_t]
        if per > FULL_LIMIT:
            # sample rows inside each sampled batch
            rows = sample_rows(M, max(1, FULL_LIMIT // (N * K)))
            cs, es = [], []
            for i in idx:
                bi = bx[idx.index(i)] if bx is not None else None
                c, e = oracle.gemm(a[i], b[i], bias=bi, beta=beta, alpha=alpha, rows=rows)
                cs.append(c)
                es.append(e)
            return (idx_t, torch.tensor(rows)), torch.stack(cs), torch.stack(es)
        c, e = oracle.gemm(a[idx_t], b[idx_t], bias=bx, beta=beta, alpha=alpha)
        return (idx_t,), c, e
    M, K = a.shape
    N = b.shape[1]
    if force_full or M * N * K <= FULL_LIMIT:
        c, e = oracle.gemm(a, b, bias=bias, beta=beta, alpha=alpha)
        return None, c, e
    rows = sample_rows(M, max(2, FULL_LIMIT // max(N * K, 1)))
    bx = bias.expand(M, N) if bias is not None else None
    c, e = oracle.gemm(a, b, bias=bx, beta=beta, alpha=alpha, rows=rows)
    return (torch.tensor(rows),), c, e


def _select(t, index):
    if index is None:
        return t
    if len(index) == 2:     # (batches, rows)
        return t[index[0]][:, index[1]]
    return t[index[0]]


def assert_parity(got, a, b, *, bias=None, beta=None, alpha=None, k=None, tag="", strict=False):
    """Compare a GPU result with the oracle on the same inputs to the parity bar."""
    dtype = got.dtype
    index, c_ref, exact = oracle_product(a, b, bias=bias, beta=beta, alpha=alpha)
    got_c = _select(got.cpu(), index)
    assert got_c.shape == c_ref.shape, f"{tag}: shape {tuple(got_c.shape)} vs {tuple(c_ref.shape)}"
    K = k if k is not None else a.shape[-1]
    scale = 1.0
    if beta is not None or alpha is not None:
        scale = abs(complex(alpha or 0)) + abs(complex(beta or 0))
        scale = max(scale, 1e-12)
    check_values(got_c, c_ref, exact, dtype, K, scale=scale, tag=tag, strict=strict)


def check_values(got, c_ref, exact, dtype, K, scale=1.0, tag="", strict=False):
    if dtype in INTS:
        if not torch.equal(got, c_ref):
            bad = (got != c_ref).nonzero()[:5].tolist()
            raise AssertionError(f"{tag}: integer mismatch at {bad}")
        return
    if dtype in COMPLEX:
        g = got.to(torch.complex128)
        err = (g - exact).abs()
        denom = exact.abs().max().item() + 1e-9
        rel = err.max().item() / denom
        limit = 3e-2 if dtype is torch.complex32 else 1e-4
        assert rel <= limit, f"{tag}: relative error {rel:.3e} > {limit:.1e}"
        if dtype is torch.complex64:
            rms = exact.abs().pow(2).mean().sqrt().item()
            lim = 1e-4 * (exact.abs() + rms)
            if not bool((err <= lim).all()):
                i = int(torch.argmax(err - lim))
                raise AssertionError(f"{tag}: |got-exact| {err.flatten()[i].item():.3e} > "
                                     f"{lim.flatten()[i].item():.3e} (exact {exact.flatten()[i].item()})")
        return
    g = got.double()
    assert not torch.isnan(g).any() or torch.isnan(exact).any(), f"{tag}: NaN in output"
    err = (g - exact).abs()
    if dtype is torch.float32:
        lim = scale * max(1e-3, 1e-5 * K) + 1e-5 * exact.abs()
    else:
        lim = scale * 1e-2 * math.sqrt(max(K, 1) / 1024) + 1e-2 * exact.abs()
    if not bool((err <= lim).all()):
        i = int(torch.argmax(err - lim))
        raise AssertionError(f"{tag}: |got-exact| {err.flatten()[i].item():.3e} > "
                             f"{lim.flatten()[i].item() if torch.is_tensor(lim) else lim:.3e} "
                             f"(got {g.flatten()[i].item():.6g}, exact {exact.flatten()[i].item():.6g})")
    # the reference's own limit against the exact value rounded to the output dtype
    ref_err = (g - exact.to(dtype).double()).abs().max().item()
    ref_lim = scale * ref_limit_atol(dtype, K, strict)
    assert ref_err <= ref_lim, f"{tag}: reference limit {ref_err:.3e} > {ref_lim:.3e}"


# ---- whole outputs of the benchmark workloads ---------------------------------------------------

def spread_rows(M, count, salt=53):
    """``count`` rows spread over [0, M): the first and last rows plus one row per equal band,
    each at a different offset inside its band (so the sample lands on different lanes of the
    row tiles, not always on a tile's first row)."""
    if M <= count:
        return list(range(M))
    band = M // count
    rows = {0, M - 1}
    for i in range(count):
        rows.add(min(M - 1, i * band + (i * salt) % max(band, 1)))
    return sorted(rows)


def _wrap_int(x, dtype):
    """int64 values wrapped to ``dtype``'s range (two's complement), as tests/test_basic.py:27-34."""
    if dtype is torch.int64:
        return x
    bits = torch.iinfo(dtype).bits
    mod = 1 << bits
    x = torch.remainder(x, mod)
    if dtype is not torch.uint8:
        x = torch.where(x >= mod // 2, x - mod, x)
    return x.to(dtype)


def gpu_exact(a, b, *, bias=None, beta=None, alpha=None):
    """The unrounded product of device tensors a @ b (2-D or 3-D), computed on the GPU in
    float64 / complex128, with the epilogue beta * bias + alpha * P applied in that type (a
    zero beta drops the bias term, a zero alpha the product).  Integers come back as exact int64
    (the float64 sums are exact while K * max|a| * max|b| < 2^53, which is asserted)."""
    dtype = a.dtype
    if dtype in COMPLEX:
        wide = torch.complex128
    else:
        wide = torch.float64
    A = a.resolve_conj().to(wide)
    B = b.resolve_conj().to(wide)
    if dtype in INTS:
        bound = a.shape[-1] * A.abs().max().item() * B.abs().max().item()
        assert bound < 2.0 ** 53, "integer product too large for an exact float64 sum"
    P = torch.matmul(A, B.contiguous())
    if dtype in INTS:
        P = P.round().to(torch.int64)
    if beta is None and alpha is None:
        return P
    beta = 0 if beta is None else beta
    alpha = 0 if alpha is None else alpha
    out = alpha * P if alpha != 0 else torch.zeros_like(P)
    if beta != 0:
        bw = bias.resolve_conj().to(torch.int64 if dtype in INTS else wide).expand(P.shape)
        out = out + beta * bw
    return out


def assert_parity_full(got, a, b, *, bias=None, beta=None, alpha=None, rows=16, tag="", k=None):
    """Parity of a whole output too large for the CPU oracle at full size.

    1. The oracle (CPU) on ``rows`` spread rows of every batch (2-D) or of the first and last
       batch (3-D), checked to the parity bar, exactly as ``assert_parity``.
    2. A float64 / complex128 product of the same operands computed on the GPU (``gpu_exact``)
       must equal the oracle's exact values on those rows (within 1e-9 relative; integers
       bit-exact), which pins it.
    3. Every element of ``got`` is then checked against it to the same bar (integers: wrapped to
       the output width and compared bit-exactly)."""
    dtype = got.dtype
    K = k if k is not None else a.shape[-1]
    scale = 1.0
    if beta is not None or alpha is not None:
        scale = max(abs(complex(alpha or 0)) + abs(complex(beta or 0)), 1e-12)
    exact_all = gpu_exact(a, b, bias=bias, beta=beta, alpha=alpha)
    a_c, b_c = a.cpu(), b.cpu()
    bias_c = bias.cpu() if bias is not None else None
    if a.dim() == 3:
        Bb, M = a.shape[0], a.shape[1]
        batches = sorted({0, Bb - 1})
    else:
        Bb, M = 1, a.shape[0]
        batches = [None]
    sel = spread_rows(M, rows)
    sel_t = torch.tensor(sel)
    for bi in batches:
        a_i = a_c if bi is None else a_c[bi]
        b_i = b_c if bi is None else b_c[bi]
        g_i = got if bi is None else got[bi]
        e_i = exact_all if bi is None else exact_all[bi]
        bias_i = None
        if bias_c is not None:   # the oracle reads bias row m for output row m
            full = bias_c.expand(*got.shape)
            bias_i = full if bi is None else full[bi]
        c_ref, ex = oracle.gemm(a_i, b_i, bias=bias_i, beta=beta, alpha=alpha, rows=sel)
        check_values(g_i.cpu()[sel_t], c_ref, ex, dtype, K, scale=scale, tag=f"{tag} oracle rows")
        e_rows = e_i.cpu()[sel_t]
        if dtype in INTS:
            assert torch.equal(e_rows.to(torch.int64), ex.to(torch.int64)), f"{tag}: GPU exact != oracle"
        else:
            d = (e_rows - ex).abs().max().item()
            assert d <= 1e-9 * (1.0 + ex.abs().max().item()), f"{tag}: GPU float64 product off the oracle by {d:.3e}"
    if dtype in INTS:
        want = _wrap_int(exact_all, dtype)
        if not torch.equal(got, want):
            bad = (got != want).nonzero()[:5].tolist()
            raise AssertionError(f"{tag}: integer mismatch at {bad}")
        return
    check_values(got, None, exact_all, dtype, K, scale=scale, tag=f"{tag} all elements")
