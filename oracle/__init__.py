"""Python handle of the CPU oracle (oracle/mb_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the metalblas_amd package.

``gemm(a, b, ...)`` runs the C restatement on CPU tensors of any strides and returns
``(c, exact)``: ``c`` in the input dtype (rounded / wrapped exactly as the reference
specifies) and ``exact`` as float64 / complex128 / int64 (the value before the final rounding; for
integers the 64-bit wraparound accumulator before truncation to the output width, carried
through a double and so exact only below 2^53).  The descriptor layout mirrors include/metalblas_amd.h and is defined
here independently of the product's own binding.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libmb_oracle.so")

DTYPE_CODE = {
    torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.complex64: 3,
    torch.complex32: 4, torch.int8: 5, torch.uint8: 6, torch.int16: 7, torch.int32: 8,
    torch.int64: 9,
}
INTS = (torch.int8, torch.uint8, torch.int16, torch.int32, torch.int64)
COMPLEX = (torch.complex64, torch.complex32)


class Matrix(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("row_stride", ctypes.c_int64),
                ("col_stride", ctypes.c_int64), ("batch_stride", ctypes.c_int64)]


class Desc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("backend", ctypes.c_int32),
        ("batch", ctypes.c_int64), ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("a", Matrix), ("b", Matrix), ("c", Matrix), ("bias", Matrix),
        ("conj_a", ctypes.c_int32), ("conj_b", ctypes.c_int32),
        ("epilogue", ctypes.c_int32), ("beta_nz", ctypes.c_int32), ("alpha_nz", ctypes.c_int32),
        ("swizzle_log", ctypes.c_int32),
        ("alpha_re", ctypes.c_double), ("alpha_im", ctypes.c_double),
        ("beta_re", ctypes.c_double), ("beta_im", ctypes.c_double),
        ("alpha_int", ctypes.c_int64), ("beta_int", ctypes.c_int64),
        ("tile", ctypes.c_int32 * 8),
        ("split_k", ctypes.c_int32), ("flags", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
    ]


_LIBH = None


def load():
    global _LIBH
    if _LIBH is None:
        if not os.path.exists(LIB):
            from . import build_oracle
            build_oracle.build()
        lib = ctypes.CDLL(LIB)
        lib.mbo_gemm.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_double)]
        lib.mbo_gemm.restype = ctypes.c_int
        for name in ("mbo_bf16_to_double", "mbo_f16_to_double"):
            getattr(lib, name).argtypes = [ctypes.c_uint16]
            getattr(lib, name).restype = ctypes.c_double
        for name in ("mbo_double_to_bf16", "mbo_double_to_f16"):
            getattr(lib, name).argtypes = [ctypes.c_double]
            getattr(lib, name).restype = ctypes.c_uint16
        _LIBH = lib
    return _LIBH


def _wrap64(v) -> int:
    iv = int(v.real) if isinstance(v, complex) else int(v)
    iv &= (1 << 64) - 1
    return iv - (1 << 64) if iv >= (1 << 63) else iv


def _mat(t, elem_offset=0):
    if t is None:
        return Matrix(None, 0, 0, 0)
    es = t.element_size()
    ptr = t.data_ptr() + elem_offset * es
    if t.dim() == 3:
        return Matrix(ptr, t.stride(1), t.stride(2), t.stride(0))
    return Matrix(ptr, t.stride(0), t.stride(1), 0)


def _conj(t):
    if t is not None and t.is_conj():
        return t.conj(), True
    return t, False


def gemm(a, b, *, bias=None, beta=None, alpha=None, rows=None):
    """Oracle product of CPU tensors a (M x K or B x M x K) and b (K x N or B x K x N).

    bias: tensor broadcastable to the output (expanded here); beta/alpha: the epilogue
    scalars (already cast as metalblas/dispatch.py:127-131 casts them), both None = plain
    product.  rows: optional list of output rows to compute (2-D only).
    Returns (c, exact).
    """
    assert a.device.type == "cpu" and b.device.type == "cpu"
    a, ca = _conj(a)
    b, cb = _conj(b)
    dtype = a.dtype
    assert b.dtype == dtype
    batched = a.dim() == 3
    if batched:
        Bb, M, K = a.shape
        N = b.shape[2]
    else:
        Bb = 1
        M, K = a.shape
        N = b.shape[1]
    epi = beta is not None or alpha is not None
    if epi:
        beta = 0 if beta is None else beta
        alpha = 0 if alpha is None else alpha
    row_list = list(range(M)) if rows is None else [int(r) for r in rows]
    assert rows is None or not batched
    Mo = len(row_list)
    shape = (Bb, Mo, N) if batched else (Mo, N)
    c = torch.zeros(shape, dtype=dtype)
    complex_ = dtype in COMPLEX
    exact = torch.zeros(shape + ((2,) if complex_ else ()), dtype=torch.float64)
    biasx = None
    if epi and bias is not None:
        biasx = bias.to(dtype).expand(*((Bb, M, N) if batched else (M, N)))
    lib = load()
    if rows is None:
        d = _desc(dtype, Bb, M, N, K, a, b, c, biasx, ca, cb, epi, beta, alpha)
        st = lib.mbo_gemm(ctypes.byref(d), ctypes.cast(exact.data_ptr(), ctypes.POINTER(ctypes.c_double)))
        assert st == 0, st
    else:
        for i, m in enumerate(row_list):
            d = _desc(dtype, 1, 1, N, K, a, b, c, biasx, ca, cb, epi, beta, alpha,
                      a_row=m, c_row=i, bias_row=m)
            ptr = exact.data_ptr() + i * N * exact.element_size() * (2 if complex_ else 1)
            st = lib.mbo_gemm(ctypes.byref(d), ctypes.cast(ptr, ctypes.POINTER(ctypes.c_double)))
            assert st == 0, st
    if complex_:
        exact = torch.view_as_complex(exact)
    elif dtype in INTS:
        exact = exact.to(torch.int64)
    return c, exact


def _desc(dtype, Bb, M, N, K, a, b, c, bias, ca, cb, epi, beta, alpha, a_row=0, c_row=0, bias_row=0):
    d = Desc()
    d.dtype = DTYPE_CODE[dtype]
    d.batch, d.M, d.N, d.K = Bb, M, N, K
    d.a = _mat(a, a_row * (a.stride(-2)))
    d.b = _mat(b)
    d.c = _mat(c, c_row * (c.stride(-2)))
    d.bias = _mat(bias, bias_row * bias.stride(-2)) if bias is not None else Matrix(None, 0, 0, 0)
    d.conj_a, d.conj_b = int(ca), int(cb)
    if epi:
        d.epilogue = 1
        d.beta_nz = int(beta != 0)
        d.alpha_nz = int(alpha != 0)
        cbeta, calpha = complex(beta), complex(alpha)
        d.beta_re, d.beta_im = cbeta.real, cbeta.imag
        d.alpha_re, d.alpha_im = calpha.real, calpha.imag
        d.beta_int, d.alpha_int = _wrap64(beta), _wrap64(alpha)
    return d


def bf16_bits(x: float) -> int:
    return int(load().mbo_double_to_bf16(float(x)))


def f16_bits(x: float) -> int:
    return int(load().mbo_double_to_f16(float(x)))


def bf16_value(bits: int) -> float:
    return float(load().mbo_bf16_to_double(int(bits)))


def f16_value(bits: int) -> float:
    return float(load().mbo_f16_to_double(int(bits)))
