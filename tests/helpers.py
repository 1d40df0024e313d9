"""Shared test helpers: seeded inputs, oracle products and the parity bar.

The bar (north star of this build, on top of the reference's own checks in
tests/test_basic.py:45-69):
  * integers: bit-exact against the oracle (which wraps like tests/test_basic.py:27-34);
  * bf16 / fp16: |got - exact| <= scale * 1e-2 * sqrt(K / 1024) + 1e-2 * |exact| elementwise,
    exact = fp64 product; and the reference's own limit max|got - round(exact)| <=
    scale * _atol(dtype, K) (tests/test_basic.py:45-50, 65-68);
  * fp32: |got - exact| <= scale * max(1e-3, 1e-5 * K) + 1e-5 * |exact| (the reference's
    strict fp32 limit, tests/test_basic.py:47, plus a relative term for large outputs);
  * complex64: max|got - exact| / max|exact| <= 1e-4 (normalised by the largest output, as
    tests/test_basic.py:62 does, because a plain elementwise rtol fails on near-zero
    outputs); complex32: <= 3e-2 (tests/test_basic.py:63).
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
        denom = exact.abs().max().item() + 1e-9
        rel = (g - exact).abs().max().item() / denom
        limit = 3e-2 if dtype is torch.complex32 else 1e-4
        assert rel <= limit, f"{tag}: relative error {rel:.3e} > {limit:.1e}"
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
