"""CPU tests that pin the oracle (oracle/mb_oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own code:
  * golden vectors written by exact rational / big-integer brute force
    (tests/golden/make_golden.py): bit-exact outputs and exact fp64 values;
  * torch's CPU matmul, which wraps integers exactly like the reference's own oracle
    (tests/test_basic.py:27-39), for every integer dtype at full value range;
  * numpy float64 / complex128 matmul for the unrounded value;
  * torch's float32 -> bfloat16 / float16 conversions for the rounding helpers;
  * layout invariance (strided, transposed, offset, stride-0 batch views);
  * the parity checker itself rejects planted mistakes (transposed operand, dropped bias
    term, off-by-one integer, wrong sign of the imaginary part).
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import check_values, gen, rand

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "oracle_golden.json")) as _f:
    CASES = json.load(_f)["cases"]
_NPZ = np.load(os.path.join(GOLDEN, "oracle_golden.npz"), allow_pickle=False)

INT_T = {"i8": torch.int8, "u8": torch.uint8, "i16": torch.int16, "i32": torch.int32, "i64": torch.int64}
FLOAT_T = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _bits_tensor(arr, fmt):
    """Storage bits (uint16 / uint32 numpy) -> torch tensor of the float format."""
    if fmt == "f32":
        return torch.from_numpy(arr.astype(np.uint32).view(np.int32)).view(torch.float32)
    t = torch.from_numpy(arr.astype(np.uint16).view(np.int16))
    return t.view(torch.bfloat16 if fmt == "bf16" else torch.float16)


def _tensor(arr, case):
    dt = case["dtype"]
    if dt in INT_T:
        return torch.from_numpy(np.ascontiguousarray(arr))
    if dt in FLOAT_T:
        return _bits_tensor(np.ascontiguousarray(arr), dt)
    part = "f32" if dt == "c64" else "f16"
    return torch.view_as_complex(_bits_tensor(np.ascontiguousarray(arr), part))


def _bits(t):
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16)
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    if t.dtype == torch.complex64:
        return torch.view_as_real(t).view(torch.int32)
    if t.dtype == torch.complex32:
        return torch.view_as_real(t).view(torch.int16)
    return t


def _operands(case):
    name = case["name"]
    a = _tensor(_NPZ[f"{name}.a"], case)
    b = _tensor(_NPZ[f"{name}.b"], case)
    if case.get("a_layout") == "t":
        a = a.transpose(-2, -1)
    if case.get("b_layout") == "t":
        b = b.transpose(-2, -1)
    if case.get("b_bcast"):
        b = b.expand(case["batch"], *b.shape)
    if case.get("conj_a"):
        a = a.conj()
    if case.get("conj_b"):
        b = b.conj()
    bias = beta = alpha = None
    if f"{name}.bias" in _NPZ:
        bias = _tensor(_NPZ[f"{name}.bias"], case)
        beta, alpha = case["beta"], case["alpha"]
        if isinstance(beta, list):
            beta, alpha = complex(*beta), complex(*alpha)
    return a, b, bias, beta, alpha


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden(case):
    """The oracle reproduces every golden vector bit for bit."""
    name = case["name"]
    a, b, bias, beta, alpha = _operands(case)
    c, exact = oracle.gemm(a, b, bias=bias, beta=beta, alpha=alpha)
    want = _tensor(_NPZ[f"{name}.c"], case)
    assert c.shape == want.shape and c.dtype == want.dtype
    assert torch.equal(_bits(c), _bits(want)), f"{name}: rounded output differs"
    if f"{name}.exact" in _NPZ:
        ex = torch.from_numpy(_NPZ[f"{name}.exact"])
        if exact.is_complex():
            exact = torch.view_as_real(exact)
        assert torch.equal(exact, ex), f"{name}: exact value differs"


def test_golden_covers_edges():
    """The fixtures include the edge cases the parity bar depends on."""
    names = {c["name"] for c in CASES}
    for need in ("bf16_ties", "f16_ties", "f16_subnormal", "f16_overflow", "bf16_beta0_nan",
                 "bf16_k0_bias", "u8_k0", "i8_127", "i32_cross", "i64_full", "c64_conj_a"):
        assert need in names
    # 127*127*13 mod 256 as int8 (closed form)
    v = (127 * 127 * 13) % 256
    assert int(_NPZ["i8_127.c"][0, 0]) == (v - 256 if v >= 128 else v)
    # the f16 overflow case really overflows, the subnormal case really is subnormal
    c = _bits_tensor(_NPZ["f16_overflow.c"], "f16").float()
    assert torch.isinf(c).any() and torch.isfinite(c).any()
    s = _bits_tensor(_NPZ["f16_subnormal.c"], "f16").float().abs()
    assert ((s > 0) & (s < 2.0 ** -14)).any()
    # round half to even: 1 + 2^-8 -> 1, 1 + 2^-7 + 2^-8 -> 1 + 2^-6
    t = _bits_tensor(_NPZ["bf16_ties.c"], "bf16").float().flatten().tolist()
    assert t == [1.0, 1.0 + 2.0 ** -6, -1.0]


# ---- integers against torch's CPU matmul (same dtype, wraps mod 2^bits) ------------------------

@pytest.mark.parametrize("dtype", list(INT_T.values()), ids=str)
@pytest.mark.parametrize("layout", ["rm", "ta", "tb"])
def test_int_vs_torch(dtype, layout):
    g = gen(3)
    info = torch.iinfo(dtype)
    M, N, K = 37, 29, 301
    lo, hi = max(info.min, -(2 ** 62)), min(info.max, 2 ** 62)
    a = torch.randint(lo, hi, (K, M) if layout == "ta" else (M, K), generator=g, dtype=torch.int64).to(dtype)
    b = torch.randint(lo, hi, (N, K) if layout == "tb" else (K, N), generator=g, dtype=torch.int64).to(dtype)
    if layout == "ta":
        a = a.t()
    if layout == "tb":
        b = b.t()
    c, exact = oracle.gemm(a, b)
    ref = torch.matmul(a.contiguous(), b.contiguous())
    assert torch.equal(c, ref)
    if dtype in (torch.int8, torch.uint8, torch.int16):
        # the fp64 'exact' channel carries the unwrapped sum (exact below 2^53)
        assert torch.equal(exact, torch.matmul(a.to(torch.int64), b.to(torch.int64)))


@pytest.mark.parametrize("dtype", list(INT_T.values()), ids=str)
def test_int_epilogue_vs_torch(dtype):
    """alpha*P + beta*bias with wraparound equals torch's addmm in the same dtype."""
    g = gen(4)
    a, b = rand((20, 33), dtype, g), rand((33, 17), dtype, g)
    bias = rand((17,), dtype, g)
    for beta, alpha in ((2, 3), (0, 1), (1, 0), (0, 0), (-3, 5)):
        c, _ = oracle.gemm(a, b, bias=bias, beta=beta, alpha=alpha)
        ref = torch.addmm(bias.expand(20, 17), a, b, beta=beta, alpha=alpha)
        assert torch.equal(c, ref), (beta, alpha)


# ---- floats and complex against numpy fp64 -----------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
def test_float_exact_vs_numpy(dtype):
    g = gen(5)
    a, b = rand((48, 200), dtype, g), rand((200, 40), dtype, g)
    c, exact = oracle.gemm(a, b)
    ref = a.double().numpy() @ b.double().numpy()
    np.testing.assert_allclose(exact.numpy(), ref, rtol=1e-12, atol=1e-12)
    # the rounded output is the exact value rounded once to the output format
    assert torch.equal(_bits(c), _bits(exact.float().to(dtype))) or dtype == torch.float32
    if dtype == torch.float32:
        assert torch.equal(c, exact.float())


def test_float_epilogue_closed_form():
    g = gen(6)
    a, b = rand((16, 64), torch.bfloat16, g), rand((64, 24), torch.bfloat16, g)
    bias = rand((16, 1), torch.bfloat16, g)
    _, p = oracle.gemm(a, b)
    for beta, alpha in ((0.5, 2.0), (0.0, 1.0), (1.0, 0.0), (0.0, 0.0), (-1.25, 3.0)):
        _, e = oracle.gemm(a, b, bias=bias, beta=beta, alpha=alpha)
        want = alpha * p + beta * bias.double().expand(16, 24)
        assert torch.equal(e, want), (beta, alpha)
    nan_bias = torch.full((16, 24), float("nan"), dtype=torch.bfloat16)
    c, _ = oracle.gemm(a, b, bias=nan_bias, beta=0.0, alpha=1.0)
    assert not torch.isnan(c).any()


@pytest.mark.parametrize("dtype", [torch.complex64, torch.complex32], ids=str)
@pytest.mark.parametrize("conj", ["none", "a", "b", "ab"])
def test_complex_vs_numpy(dtype, conj):
    g = gen(7)
    a, b = rand((12, 40), dtype, g), rand((40, 9), dtype, g)
    an, bn = a.to(torch.complex128).numpy(), b.to(torch.complex128).numpy()
    if "a" in conj:
        a, an = a.conj(), np.conj(an)
    if "b" in conj:
        b, bn = b.conj(), np.conj(bn)
    _, exact = oracle.gemm(a, b)
    np.testing.assert_allclose(exact.numpy(), an @ bn, rtol=1e-12, atol=1e-12)


def test_complex_epilogue_closed_form():
    g = gen(8)
    a, b = rand((6, 10), torch.complex64, g), rand((10, 5), torch.complex64, g)
    bias = rand((5,), torch.complex64, g)
    beta, alpha = complex(0.5, -1.0), complex(2.0, 0.25)
    _, p = oracle.gemm(a, b)
    _, e = oracle.gemm(a, b, bias=bias, beta=beta, alpha=alpha)
    want = alpha * p.numpy() + beta * bias.to(torch.complex128).numpy()[None, :]
    np.testing.assert_allclose(e.numpy(), want, rtol=1e-13, atol=1e-13)


# ---- rounding helpers against torch's conversions ---------------------------------------------

def _float32_samples():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(20000, generator=g) * torch.exp2(torch.randint(-140, 130, (20000,), generator=g).float())
    special = torch.tensor([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 2.0 ** -24,
                            2.0 ** -25, 3.0 * 2.0 ** -26, 2.0 ** -14, 3.3895e38, 3.4e38,
                            float("inf"), -float("inf"), 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,
                            1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 9.18e-41, 1e-45])
    return torch.cat([x, special])


def test_bf16_rounding_vs_torch():
    x = _float32_samples()
    want = x.to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF
    got = torch.tensor([oracle.bf16_bits(v) for v in x.tolist()])
    assert torch.equal(got, want)
    # decoding is exact
    vals = [oracle.bf16_value(int(bits)) for bits in want[:2000].tolist()]
    assert torch.equal(torch.tensor(vals, dtype=torch.float64), x[:2000].to(torch.bfloat16).double())
    assert oracle.bf16_bits(float("nan")) & 0x7F80 == 0x7F80


def test_f16_rounding_vs_torch():
    x = _float32_samples()
    want = x.to(torch.float16).view(torch.int16).to(torch.int64) & 0xFFFF
    got = torch.tensor([oracle.f16_bits(v) for v in x.tolist()])
    assert torch.equal(got, want)
    vals = [oracle.f16_value(int(bits)) for bits in want[:2000].tolist()]
    assert torch.equal(torch.tensor(vals, dtype=torch.float64), x[:2000].to(torch.float16).double())


# ---- layout invariance and row sampling --------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.int8, torch.complex64], ids=str)
def test_layout_invariance(dtype):
    g = gen(10)
    M, N, K = 24, 20, 36
    a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    c0, e0 = oracle.gemm(a, b)
    views = {
        "ta": (rand((K, M), dtype, g).t(), None),
        "row_sliced": (rand((2 * M, K), dtype, g)[::2], None),
        "col_sliced": (rand((M, 2 * K), dtype, g)[:, ::2], None),
    }
    for name, (v, _) in views.items():
        c1, _ = oracle.gemm(v, b)
        c2, _ = oracle.gemm(v.contiguous(), b)
        assert torch.equal(_bits(c1), _bits(c2)), name
    flat = torch.cat([rand((17,), dtype, g), a.reshape(-1)])
    off = flat[17:].view(M, K)
    assert off.storage_offset() == 17
    c3, e3 = oracle.gemm(off, b)
    assert torch.equal(_bits(c3), _bits(c0)) and torch.equal(e3, e0)
    # stride-0 batch (broadcast B) equals per-batch products
    a3 = rand((3, M, K), dtype, g)
    cb, _ = oracle.gemm(a3, b.expand(3, K, N))
    for i in range(3):
        ci, _ = oracle.gemm(a3[i], b)
        assert torch.equal(_bits(cb[i]), _bits(ci))
    # sampled rows equal the full result's rows
    cr, er = oracle.gemm(a, b, rows=[0, 5, M - 1])
    assert torch.equal(_bits(cr), _bits(c0[[0, 5, M - 1]])) and torch.equal(er, e0[[0, 5, M - 1]])


# ---- the checker rejects planted mistakes -------------------------------------------------------

def test_checker_catches_planted_mistakes():
    g = gen(11)
    n = 64
    a, b = rand((n, n), torch.bfloat16, g), rand((n, n), torch.bfloat16, g)
    c, exact = oracle.gemm(a, b)
    check_values(c, c, exact, torch.bfloat16, n)            # the true result passes
    ct, _ = oracle.gemm(a, b.t())                            # transposed operand
    with pytest.raises(AssertionError):
        check_values(ct, c, exact, torch.bfloat16, n)
    bias = rand((n,), torch.bfloat16, g)
    cbias, ebias = oracle.gemm(a, b, bias=bias, beta=0.5, alpha=2.0)
    cdrop, _ = oracle.gemm(a, b, bias=bias, beta=0.0, alpha=2.0)  # dropped bias term
    with pytest.raises(AssertionError):
        check_values(cdrop, cbias, ebias, torch.bfloat16, n, scale=2.5)
    ai, bi = rand((n, n), torch.int32, g), rand((n, n), torch.int32, g)
    ci, ei = oracle.gemm(ai, bi)
    bad = ci.clone()
    bad[3, 7] += 1                                           # off by one
    with pytest.raises(AssertionError):
        check_values(bad, ci, ei, torch.int32, n)
    ac, bc = rand((16, 32), torch.complex64, g), rand((32, 16), torch.complex64, g)
    cc, ec = oracle.gemm(ac, bc)
    cconj, _ = oracle.gemm(ac.conj(), bc)                    # wrong sign of imag(A)
    with pytest.raises(AssertionError):
        check_values(cconj, cc, ec, torch.complex64, 32)
    # fp32: a result rounded through bf16 is too coarse for the fp32 bar
    af, bf = rand((32, 256), torch.float32, g), rand((256, 32), torch.float32, g)
    cf, ef = oracle.gemm(af, bf)
    with pytest.raises(AssertionError):
        check_values(cf.to(torch.bfloat16).float(), cf, ef, torch.float32, 256)
    assert math.isfinite(float(ef.abs().max()))
