"""Generate the golden vectors that pin the CPU oracle (tests/golden/oracle_golden.npz + .json).

The reference (Isalia20/metalBLAS) stores no golden vectors: its tests draw inputs from the
MPS RNG and compare against torch (tests/test_basic.py:20-69).  These fixtures are written
by brute force that shares no code with oracle/mb_oracle.c:

  * integers: exact Python-int dot products, then the modular wrap of
    tests/test_basic.py:27-34 (``_wrap``) applied as ``v mod 2**bits`` (two's complement);
    the epilogue alpha*P + beta*bias is taken in the same exact arithmetic before the wrap,
    which equals the reference's 32-bit (64-bit for int64) wraparound accumulate and
    truncating store (metalblas/integer_dispatch.py:13-19, shaders/int_gemm.h:147-150);
  * floats / complex: exact rational (fractions.Fraction) sums, the fused epilogue in exact
    arithmetic (shaders/mb_epi.h:16-26, shaders/complex_pack.h:41-58), then ONE rounding to
    the output format with round-half-to-even done by Python's exact ``round`` on
    Fractions.  Inputs are drawn so every exact result is also a float64 (checked here), so
    the oracle's fp64 accumulation must reproduce them bit for bit.

Run ``python tests/golden/make_golden.py`` to rewrite the fixtures (deterministic).
"""
from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
NPZ = os.path.join(HERE, "oracle_golden.npz")
META = os.path.join(HERE, "oracle_golden.json")

# (significand bits incl. the implicit one, minimum normal exponent, largest finite value)
FORMATS = {
    "bf16": (8, -126, Fraction(2 ** 8 - 1, 2 ** 7) * 2 ** 127),
    "f16": (11, -14, Fraction(65504)),
    "f32": (24, -126, Fraction(2 ** 24 - 1, 2 ** 23) * 2 ** 127),
}
INT_BITS = {"i8": (8, True), "u8": (8, False), "i16": (16, True), "i32": (32, True), "i64": (64, True)}
NP_INT = {"i8": np.int8, "u8": np.uint8, "i16": np.int16, "i32": np.int32, "i64": np.int64}
INF = "inf"


def _floor_log2(a: Fraction) -> int:
    e = a.numerator.bit_length() - a.denominator.bit_length()
    # fix up so that 2**e <= a < 2**(e+1)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    return e


def round_to(x: Fraction, fmt: str):
    """Round an exact rational to format ``fmt``, ties to even; returns a Fraction or +-INF."""
    p, emin, maxv = FORMATS[fmt]
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = max(_floor_log2(a), emin)
    q = Fraction(2) ** (e - (p - 1))
    y = round(a / q) * q          # round() on a Fraction rounds half to even
    if y > maxv:
        return sign * float("inf")
    return sign * y


def encode(v, fmt: str) -> int:
    """Bit pattern of an (already representable) value."""
    f = float(v)
    if fmt == "bf16":
        return int(np.array([f], dtype=np.float32).view(np.uint32)[0] >> 16)
    if fmt == "f16":
        return int(np.array([f], dtype=np.float16).view(np.uint16)[0])
    return int(np.array([f], dtype=np.float32).view(np.uint32)[0])


def decode(bits: int, fmt: str) -> Fraction:
    if fmt == "bf16":
        f = np.array([bits << 16], dtype=np.uint32).view(np.float32)[0]
    elif fmt == "f16":
        f = np.array([bits], dtype=np.uint16).view(np.float16)[0]
    else:
        f = np.array([bits], dtype=np.uint32).view(np.float32)[0]
    return Fraction(float(f))


def storage_dtype(fmt):
    return np.uint32 if fmt == "f32" else np.uint16


def rand_float_bits(rng, shape, fmt, scale=1.0, mant_bits=None):
    """N(0,1)*scale values rounded to ``fmt`` (optionally to fewer significand bits)."""
    vals = rng.standard_normal(size=shape) * scale
    out = np.zeros(shape, dtype=storage_dtype(fmt))
    for idx in np.ndindex(*shape):
        x = Fraction(float(vals[idx]))
        if mant_bits is not None and x != 0:
            e = _floor_log2(abs(x))
            q = Fraction(2) ** (e - (mant_bits - 1))
            x = round(x / q) * q
        out[idx] = encode(round_to(x, fmt), fmt)
    return out


def exact_check(v: Fraction):
    assert Fraction(float(v)) == v, "exact value is not a float64; pick other inputs"
    return float(v)


CASES = []
ARRAYS = {}


def add_case(name, meta, arrays):
    meta = dict(meta, name=name)
    CASES.append(meta)
    for k, v in arrays.items():
        ARRAYS[f"{name}.{k}"] = v


def view(arr, layout):
    """Logical operand of a stored array: 'rm' as stored, 't' transposed."""
    return arr.T if layout == "t" else arr


# ------------------------------------------------------------------------------------------
# integers
# ------------------------------------------------------------------------------------------

def wrap(v: int, key: str) -> int:
    bits, signed = INT_BITS[key]
    v &= (1 << bits) - 1
    if signed and v >= 1 << (bits - 1):
        v -= 1 << bits
    return v


def int_case(name, key, rng, M, N, K, lo, hi, a_layout="rm", b_layout="rm", epi=None, batch=0,
             fixed=None):
    shp_a = (K, M) if a_layout == "t" else (M, K)
    shp_b = (N, K) if b_layout == "t" else (K, N)
    if batch:
        shp_a, shp_b = (batch,) + shp_a, (batch,) + shp_b
    if fixed is not None:
        a = np.full(shp_a, fixed[0], dtype=NP_INT[key])
        b = np.full(shp_b, fixed[1], dtype=NP_INT[key])
    else:
        a = rng.integers(lo, hi, size=shp_a, endpoint=True, dtype=np.int64).astype(NP_INT[key])
        b = rng.integers(lo, hi, size=shp_b, endpoint=True, dtype=np.int64).astype(NP_INT[key])
    nb = batch or 1
    A = [view(a[i] if batch else a, "t" if a_layout == "t" else "rm") for i in range(nb)]
    B = [view(b[i] if batch else b, "t" if b_layout == "t" else "rm") for i in range(nb)]
    bias = None
    arrays = {"a": a, "b": b}
    meta = {"dtype": key, "M": M, "N": N, "K": K, "a_layout": a_layout, "b_layout": b_layout,
            "batch": batch}
    if epi is not None:
        beta, alpha, bshape = epi
        bias = rng.integers(lo, hi, size=bshape, endpoint=True, dtype=np.int64).astype(NP_INT[key])
        arrays["bias"] = bias
        meta.update(beta=beta, alpha=alpha, bias_shape=list(bshape))
    c = np.zeros((nb, M, N), dtype=NP_INT[key])
    for z in range(nb):
        bz = np.broadcast_to(bias, (M, N)) if bias is not None else None
        for m in range(M):
            for n in range(N):
                p = sum(int(A[z][m, k]) * int(B[z][k, n]) for k in range(K))
                if epi is not None:
                    v = (alpha * p if alpha != 0 else 0) + (beta * int(bz[m, n]) if beta != 0 else 0)
                else:
                    v = p
                c[z, m, n] = wrap(v, key)
    arrays["c"] = c if batch else c[0]
    add_case(name, meta, arrays)


# ------------------------------------------------------------------------------------------
# real floating point
# ------------------------------------------------------------------------------------------

def float_case(name, fmt, rng, M, N, K, a_layout="rm", b_layout="rm", epi=None, scale=1.0,
               mant_bits=None, a_bits=None, b_bits=None, nan_bias=False, batch=0, b_bcast=False):
    shp_a = (K, M) if a_layout == "t" else (M, K)
    shp_b = (N, K) if b_layout == "t" else (K, N)
    if batch:
        shp_a = (batch,) + shp_a
        if not b_bcast:
            shp_b = (batch,) + shp_b
    a = a_bits if a_bits is not None else rand_float_bits(rng, shp_a, fmt, scale, mant_bits)
    b = b_bits if b_bits is not None else rand_float_bits(rng, shp_b, fmt, scale, mant_bits)
    nb = batch or 1
    arrays = {"a": a, "b": b}
    meta = {"dtype": fmt, "M": M, "N": N, "K": K, "a_layout": a_layout, "b_layout": b_layout,
            "batch": batch, "b_bcast": b_bcast}
    bias = None
    if epi is not None:
        beta, alpha, bshape = epi
        if nan_bias:
            bias = np.full(bshape, encode(float("nan"), fmt) if fmt != "bf16" else 0x7FC0,
                           dtype=storage_dtype(fmt))
        else:
            bias = rand_float_bits(rng, bshape, fmt, 1.0, mant_bits)
        arrays["bias"] = bias
        meta.update(beta=beta, alpha=alpha, bias_shape=list(bshape))
    c = np.zeros((nb, M, N), dtype=storage_dtype(fmt))
    ex = np.zeros((nb, M, N), dtype=np.float64)
    for z in range(nb):
        az = a[z] if batch else a
        bzz = b[z] if (batch and not b_bcast) else b
        Aop, Bop = view(az, a_layout), view(bzz, b_layout)
        bb = np.broadcast_to(bias, (M, N)) if bias is not None else None
        for m in range(M):
            for n in range(N):
                p = sum((decode(int(Aop[m, k]), fmt) * decode(int(Bop[k, n]), fmt) for k in range(K)),
                        Fraction(0))
                if epi is not None:
                    v = Fraction(0)
                    if alpha != 0:
                        v += Fraction(alpha) * p
                    if beta != 0:
                        v += Fraction(beta) * decode(int(bb[m, n]), fmt)
                else:
                    v = p
                ex[z, m, n] = exact_check(v)
                r = round_to(v, fmt)
                c[z, m, n] = encode(r, fmt)
    arrays["c"] = c if batch else c[0]
    arrays["exact"] = ex if batch else ex[0]
    add_case(name, meta, arrays)


# ------------------------------------------------------------------------------------------
# complex (interleaved re/im of fp32 or fp16 parts)
# ------------------------------------------------------------------------------------------

def complex_case(name, fmt, rng, M, N, K, conj_a=False, conj_b=False, epi=None, a_layout="rm"):
    key = "c64" if fmt == "f32" else "c32"
    shp_a = (K, M) if a_layout == "t" else (M, K)
    a = rand_float_bits(rng, shp_a + (2,), fmt, 1.0, 12 if fmt == "f32" else None)
    b = rand_float_bits(rng, (K, N, 2), fmt, 1.0, 12 if fmt == "f32" else None)
    arrays = {"a": a, "b": b}
    meta = {"dtype": key, "M": M, "N": N, "K": K, "conj_a": conj_a, "conj_b": conj_b,
            "a_layout": a_layout, "b_layout": "rm", "batch": 0}
    bias = None
    if epi is not None:
        beta, alpha, bshape = epi
        bias = rand_float_bits(rng, tuple(bshape) + (2,), fmt, 1.0, 12 if fmt == "f32" else None)
        arrays["bias"] = bias
        meta.update(beta=[beta.real, beta.imag], alpha=[alpha.real, alpha.imag],
                    bias_shape=list(bshape))

    def cval(arr, idx):
        re = decode(int(arr[idx + (0,)]), fmt)
        im = decode(int(arr[idx + (1,)]), fmt)
        return re, im

    c = np.zeros((M, N, 2), dtype=storage_dtype(fmt))
    ex = np.zeros((M, N, 2), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            sr = si = Fraction(0)
            for k in range(K):
                ar, ai = cval(a, (k, m) if a_layout == "t" else (m, k))
                br, bi = cval(b, (k, n))
                if conj_a:
                    ai = -ai
                if conj_b:
                    bi = -bi
                sr += ar * br - ai * bi
                si += ar * bi + ai * br
            vr, vi = sr, si
            if epi is not None:
                beta, alpha, bshape = epi
                assert len(bshape) == 1, "complex fixtures use a row-vector bias"
                xr, xi = cval(bias, (n,))
                ar_, ai_ = Fraction(alpha.real), Fraction(alpha.imag)
                br_, bi_ = Fraction(beta.real), Fraction(beta.imag)
                vr = ar_ * sr - ai_ * si + br_ * xr - bi_ * xi
                vi = ar_ * si + ai_ * sr + br_ * xi + bi_ * xr
            ex[m, n, 0] = exact_check(vr)
            ex[m, n, 1] = exact_check(vi)
            c[m, n, 0] = encode(round_to(vr, fmt), fmt)
            c[m, n, 1] = encode(round_to(vi, fmt), fmt)
    arrays["c"] = c
    arrays["exact"] = ex
    add_case(name, meta, arrays)


def main():
    rng = np.random.default_rng(20260101)
    # integers: full-range values so the accumulators wrap
    int_case("i8_full", "i8", rng, 5, 6, 7, -128, 127)
    int_case("u8_full", "u8", rng, 5, 6, 7, 0, 255)
    int_case("i16_full", "i16", rng, 4, 5, 9, -32768, 32767)
    int_case("i32_full", "i32", rng, 4, 5, 9, -(2 ** 31), 2 ** 31 - 1)
    int_case("i64_full", "i64", rng, 3, 4, 5, -(2 ** 63), 2 ** 63 - 1)
    int_case("i8_127", "i8", rng, 2, 3, 13, 0, 0, fixed=(127, 127))          # 127^2*13 mod 256
    int_case("u8_255", "u8", rng, 2, 3, 11, 0, 0, fixed=(255, 255))
    int_case("i32_cross", "i32", rng, 2, 2, 3, 0, 0, fixed=(2 ** 30, 3))    # crosses 2^31
    int_case("i32_small_ta", "i32", rng, 6, 5, 8, -8, 8, a_layout="t")
    int_case("i32_epi", "i32", rng, 4, 5, 6, -(2 ** 31), 2 ** 31 - 1, epi=(-2, 3, (5,)))
    int_case("i8_epi_col", "i8", rng, 4, 5, 6, -128, 127, epi=(5, -7, (4, 1)))
    int_case("i64_epi", "i64", rng, 3, 3, 4, -(2 ** 62), 2 ** 62, epi=(3, -5, (3, 3)))
    int_case("i16_bmm", "i16", rng, 3, 4, 5, -32768, 32767, batch=3)
    int_case("u8_k0", "u8", rng, 3, 4, 0, 0, 255, epi=(3, 2, (4,)))
    # bf16 / fp16 / fp32
    float_case("bf16_rand", "bf16", rng, 6, 5, 16)
    float_case("bf16_tt", "bf16", rng, 5, 6, 12, a_layout="t", b_layout="t")
    float_case("f16_rand", "f16", rng, 6, 5, 16)
    float_case("f32_rand", "f32", rng, 4, 5, 8, mant_bits=12)
    float_case("bf16_addmm", "bf16", rng, 4, 6, 10, epi=(0.5, 2.0, (6,)))
    float_case("f16_addmm_col", "f16", rng, 4, 6, 10, epi=(-1.5, 3.0, (4, 1)))
    float_case("f32_addmm_full", "f32", rng, 3, 4, 6, epi=(2.0, -0.25, (3, 4)), mant_bits=12)
    float_case("bf16_beta0_nan", "bf16", rng, 3, 4, 8, epi=(0.0, 1.0, (3, 4)), nan_bias=True)
    float_case("f16_alpha0", "f16", rng, 3, 4, 8, epi=(2.0, 0.0, (4,)))
    float_case("bf16_k0_bias", "bf16", rng, 3, 4, 0, epi=(0.5, 1.0, (4,)))
    float_case("f16_subnormal", "f16", rng, 3, 3, 4, scale=2.0 ** -9)
    float_case("f16_overflow", "f16", rng, 3, 4, 6, scale=2.0 ** 8)
    float_case("bf16_overflow", "bf16", rng, 3, 4, 6, scale=2.0 ** 64)
    float_case("bf16_bmm_bcast", "bf16", rng, 3, 4, 8, batch=3, b_bcast=True)
    # round-half-to-even ties: [1, 2^-8] . [1, 1] = 1 + 2^-8 (tie -> 1), and
    # [1 + 2^-7, 2^-8] . [1, 1] = 1 + 2^-7 + 2^-8 (tie -> 1 + 2^-6)
    tie_a = np.array([[encode(Fraction(1), "bf16"), encode(Fraction(1, 256), "bf16")],
                      [encode(Fraction(129, 128), "bf16"), encode(Fraction(1, 256), "bf16")],
                      [encode(Fraction(-1), "bf16"), encode(Fraction(-1, 256), "bf16")]], dtype=np.uint16)
    tie_b = np.array([[encode(Fraction(1), "bf16")], [encode(Fraction(1), "bf16")]], dtype=np.uint16)
    float_case("bf16_ties", "bf16", rng, 3, 1, 2, a_bits=tie_a, b_bits=tie_b)
    ftie_a = np.array([[encode(Fraction(1), "f16"), encode(Fraction(1, 2048), "f16")],
                       [encode(Fraction(1025, 1024), "f16"), encode(Fraction(1, 2048), "f16")]], dtype=np.uint16)
    ftie_b = np.array([[encode(Fraction(1), "f16")], [encode(Fraction(1), "f16")]], dtype=np.uint16)
    float_case("f16_ties", "f16", rng, 2, 1, 2, a_bits=ftie_a, b_bits=ftie_b)
    # complex
    complex_case("c64_rand", "f32", rng, 4, 3, 6)
    complex_case("c64_conj_a", "f32", rng, 3, 4, 5, conj_a=True)
    complex_case("c64_conj_b_ta", "f32", rng, 3, 4, 5, conj_b=True, a_layout="t")
    complex_case("c64_addmm", "f32", rng, 3, 4, 5, epi=(complex(0.5, -1.0), complex(2.0, 0.25), (4,)))
    complex_case("c32_rand", "f16", rng, 3, 4, 6)
    complex_case("c32_conj", "f16", rng, 3, 3, 4, conj_a=True, conj_b=True)

    np.savez_compressed(NPZ, **ARRAYS)
    with open(META, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py", "cases": CASES}, f, indent=1)
    print(f"wrote {len(CASES)} cases to {NPZ}")


if __name__ == "__main__":
    main()
