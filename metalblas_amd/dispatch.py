"""Public PyTorch API of metalblas on MI355X (gfx950), with the reference's semantics.

Every function keeps the name, arguments, result dtype/shape and error behaviour of
metalblas/dispatch.py (Isalia20/metalBLAS); only the device changes from ``mps`` to a
PyTorch-ROCm tensor (``device.type == "cuda"``).  The arithmetic runs in the hand-written
HIP kernels of libmetalblas_hip.so, reached through the C ABI (``_lib``).

Routing follows metalblas/dispatch.py:174-185: complex if either operand is complex,
integer if ``a`` is an integer tensor, floating point otherwise.  Differences from the
reference that change no result:
  * conjugated operands are passed as a conj flag instead of being materialised
    (metalblas/complex_dispatch.py:25-30 resolves them by copying);
  * batched integer/complex products run as one batched kernel instead of a Python loop
    (metalblas/dispatch.py:134-145, integer_dispatch.py:125-127);
  * outputs are freshly allocated (the reference's pooled outputs can alias a returned view,
    metalblas/dispatch.py:78-93 with :167-170);
  * ``out=`` tensors of any stride are written in place.
"""
from __future__ import annotations

import ctypes
import os
import threading
from math import prod

import torch

from . import _lib
from . import planner as _planner

# The compiled fast path (csrc/mb_fast.cpp): matmul / bmm calls whose signature this module has
# already planned skip the Python checks and ctypes.  Not loaded when METALBLAS_LIB names
# another build of the library.
_FAST = None
if not os.environ.get("METALBLAS_LIB"):
    try:
        from . import _fast as _FAST
    except ImportError:
        _FAST = None

INTS = (torch.int8, torch.uint8, torch.int16, torch.int32, torch.int64)
FLOATS = (torch.float32, torch.float16, torch.bfloat16)
COMPLEX = (torch.complex64, torch.complex32)
INT_DTYPES = frozenset(INTS)
FLOAT_DTYPES = frozenset(FLOATS)
COMPLEX_DTYPES = frozenset(COMPLEX)

# backend= names accepted by matmul (metalblas/float_dispatch.py:802-852); "generic" is this
# build's element-gather kernel (works on any layout).
BACKENDS = {
    None: _lib.BACKEND_AUTO,
    "auto": _lib.BACKEND_AUTO,
    "gemv": _lib.BACKEND_GEMV,
    "mpp_tensor": _lib.BACKEND_MATRIX,
    "mpp": _lib.BACKEND_TILED,
    "simd": _lib.BACKEND_TILED,
    "generic": _lib.BACKEND_GENERIC,
}


def _on_device(t) -> bool:
    return t.device.type == "cuda"


def _unit_lead(t, rows, cols):
    """``(is_column_major, leading_stride)`` for a simple matrix view, else None
    (metalblas/dispatch.py:23-30)."""
    s0, s1 = map(int, t.stride()[-2:])
    if s1 == 1 and s0 >= cols:
        return False, s0
    if s0 == 1 and s1 >= rows:
        return True, s1
    return None


def _matrix_view(t, rows, cols):
    """Keep row/column-major views, copy anything else (metalblas/dispatch.py:33-35)."""
    return t if _unit_lead(t, rows, cols) else t.contiguous()


def _mat(t):
    """(tensor, row_stride, col_stride, batch_stride) of a 2-D or 3-D tensor."""
    if t.dim() == 3:
        return (t, t.stride(1), t.stride(2), t.stride(0))
    return (t, t.stride(0), t.stride(1), 0)


def _scalars(dtype, beta, alpha):
    """Cast beta/alpha like metalblas/dispatch.py:127-131 and report which terms are live."""
    if dtype in INT_DTYPES:
        beta, alpha = int(beta), int(alpha)
    elif dtype not in COMPLEX_DTYPES:
        beta, alpha = float(beta), float(alpha)
    return beta, alpha, beta != 0, alpha != 0


def _conj_split(t):
    """(tensor whose memory holds the values, conj flag) — a conj view is read through the
    flag rather than copied."""
    if t.is_conj():
        return t.conj(), True
    return t, False


# Descriptors already planned (and tuned) for a call signature: the dtype, sizes, strides,
# pointer alignment classes, flags and scalars.  A hit skips descriptor construction and the
# tuner; only the data pointers (and the workspace) change between calls.  Each thread patches
# its own copy of a descriptor (the C call runs without the GIL), through a view of its 64-bit
# words.
_DESC_CACHE: dict = {}
_DESC_CACHE_CAP = 4096
_DESC_GEN = [0]   # bumped when _DESC_CACHE is cleared: the threads' copies are dropped too
_TLS = threading.local()
_W = ctypes.c_uint64 * _lib.DESC_WORDS


def clear_descriptors() -> None:
    """Forget every cached call signature (the next call of each plans it again)."""
    _DESC_CACHE.clear()
    _DESC_GEN[0] += 1
    if _FAST is not None:
        _FAST.clear()


def _thread_desc(key, template):
    """(descriptor, its word view, byref) of this thread for a cached call signature."""
    mine = getattr(_TLS, "descs", None)
    if mine is None or mine[0] != _DESC_GEN[0]:
        mine = _TLS.descs = (_DESC_GEN[0], {})
    ent = mine[1].get(key)
    if ent is None:
        d = _lib.MbGemmDesc.from_buffer_copy(template)
        ent = mine[1][key] = (d, _W.from_buffer(d), ctypes.byref(d))
    return ent


def _launch(dtype, batch, M, N, K, a, b, out, *, bias=None, epilogue=None, conj_a=False,
            conj_b=False, backend=_lib.BACKEND_AUTO, tile=None, swizzle_log=None):
    """Describe and queue one (batched) product; a/b/out/bias are 2-D or 3-D tensors."""
    idx = out.get_device()
    pa, pb, pc = a.data_ptr(), b.data_ptr(), out.data_ptr()
    pbias = bias.data_ptr() if bias is not None else 0
    key = (dtype, batch, M, N, K, a.stride(), pa & 255, b.stride(), pb & 255, out.stride(), pc & 255,
           bias.stride() if bias is not None else None, pbias & 255, conj_a, conj_b, epilogue, backend,
           tile if tile is None else tuple(tile), swizzle_log, idx, _planner.enabled())
    hit = _DESC_CACHE.get(key)
    keep = True
    if hit is None:
        desc = _lib.make_desc(dtype, batch, M, N, K, _mat(a), _mat(b), _mat(out),
                              _mat(bias) if bias is not None else None,
                              conj_a=conj_a, conj_b=conj_b, epilogue=epilogue, backend=backend,
                              tile=tile, swizzle_log=swizzle_log)
        # under HIP graph capture the tuner cannot time candidates (it synchronises): the static
        # plan is captured and not kept, so the first eager call of the signature still tunes
        keep = not torch._C._cuda_isCurrentStreamCapturing()
        if backend == _lib.BACKEND_AUTO and tile is None and keep:
            with torch.cuda.device(idx):
                _planner.tune(desc, a, b, out, bias)
        hit = (desc, _lib.workspace_bytes(desc))
        if keep:
            if len(_DESC_CACHE) >= _DESC_CACHE_CAP:
                clear_descriptors()
            _DESC_CACHE[key] = hit
    template, ws_bytes = hit
    if (keep and _FAST is not None and bias is None and epilogue is None and not conj_a and not conj_b
            and backend == _lib.BACKEND_AUTO and tile is None and swizzle_log is None):
        _FAST.register(a, b, out, bytes(template), ws_bytes)   # later calls take the fast path
    desc, w, ref = _thread_desc(key, template)
    w[_lib.W_A] = pa
    w[_lib.W_B] = pb
    w[_lib.W_C] = pc
    w[_lib.W_BIAS] = pbias
    if idx != torch._C._cuda_getDevice():
        with torch.cuda.device(idx):
            _lib.launch(desc, ws_bytes, idx)
        return out
    stream = torch._C._cuda_getCurrentRawStream(idx)
    ws, lock = None, _lib._NO_LOCK   # ws is held until mb_gemm has queued the kernels using it
    if ws_bytes > 0:
        if ws_bytes <= _lib._WS_KEEP:
            ws, lock = _lib.workspace(idx, stream, ws_bytes)
        else:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=out.device)
        w[_lib.W_WS] = ws.data_ptr()
        w[_lib.W_WS_BYTES] = ws_bytes
    with lock:
        status = (_lib._LIB or _lib.load()).mb_gemm(ref, stream)
    if status:
        _lib.check(status)
    del ws
    return out


# ---------------------------------------------------------------------------------------
# 2-D products by dtype family
# ---------------------------------------------------------------------------------------

def _check_out(out, shape, dtype):
    assert out.shape == tuple(shape) and out.dtype == dtype and _on_device(out), \
        f"out must be {tuple(shape)} {dtype} on cuda"


def _float_matmul(a, b, backend, tile, swizzle_log, out, epilogue=None):
    """metalblas/float_dispatch.py:745-852 (matmul) and :897-956 (addmm)."""
    assert _on_device(a) and _on_device(b)
    assert a.dtype == b.dtype
    dtype = a.dtype
    if dtype not in FLOAT_DTYPES:
        raise NotImplementedError(f"dtype {dtype} not supported")
    assert a.dim() == 2 and b.dim() == 2, "matmul currently expects 2-D inputs"
    M, K = a.shape
    K2, N = b.shape
    assert K == K2, f"shape mismatch: A is {a.shape}, B is {b.shape}"
    if backend not in BACKENDS:
        raise ValueError(f"unknown backend {backend}")
    code = BACKENDS[backend]
    if code == _lib.BACKEND_GEMV and M != 1 and N != 1:
        raise ValueError("gemv backend requires M==1 or N==1")
    if code == _lib.BACKEND_MATRIX and tile is not None:
        assert len(tile) >= 3
    if out is None:
        out = a.new_empty(M, N)
    else:
        _check_out(out, (M, N), dtype)
    A, B = _matrix_view(a, M, K), _matrix_view(b, K, N)
    if M == 0 or N == 0:
        return out
    bias = ep = None
    if epilogue is not None:
        bias, beta, alpha, bnz, anz = epilogue
        ep = (beta, alpha, bnz, anz)
    return _launch(dtype, 1, M, N, K, A, B, out, bias=bias, epilogue=ep, backend=code,
                   tile=tile, swizzle_log=swizzle_log)


def _int_matmul(a, b, out=None, epilogue=None):
    """metalblas/integer_dispatch.py:92-117."""
    assert _on_device(a) and _on_device(b)
    assert a.dtype == b.dtype, "integer matmul requires both operands the same dtype"
    assert a.dim() == 2 and b.dim() == 2, "matmul currently expects 2-D inputs"
    dtype = a.dtype
    M, K = a.shape
    K2, N = b.shape
    assert K == K2, f"shape mismatch: A is {a.shape}, B is {b.shape}"
    if out is None:
        out = a.new_empty(M, N)
    else:
        _check_out(out, (M, N), dtype)
    A, B = _matrix_view(a, M, K), _matrix_view(b, K, N)
    if M == 0 or N == 0:
        return out
    bias = ep = None
    if epilogue is not None:
        bias, beta, alpha, bnz, anz = epilogue
        ep = (beta, alpha, bnz, anz)
    return _launch(dtype, 1, M, N, K, A, B, out, bias=bias, epilogue=ep)


def _complex_inputs(a, b):
    """Promote the real operand to the complex dtype (metalblas/complex_dispatch.py:25-30);
    conjugation stays a flag."""
    dtype = a.dtype if a.dtype in COMPLEX_DTYPES else b.dtype
    a = a.to(dtype) if a.dtype != dtype else a
    b = b.to(dtype) if b.dtype != dtype else b
    a, ca = _conj_split(a)
    b, cb = _conj_split(b)
    return a, b, ca, cb, dtype


def _complex_matmul(a, b, out=None, epilogue=None):
    """metalblas/complex_dispatch.py:84-115."""
    a, b, ca, cb, dtype = _complex_inputs(a, b)
    assert _on_device(a) and _on_device(b)
    assert a.dim() == 2 and b.dim() == 2, "complex matmul currently expects 2-D inputs"
    M, K = a.shape
    K2, N = b.shape
    assert K == K2, f"shape mismatch: A is {a.shape}, B is {b.shape}"
    if out is not None:
        _check_out(out, (M, N), dtype)
    else:
        out = torch.empty(M, N, dtype=dtype, device=a.device)
    A, B = _matrix_view(a, M, K), _matrix_view(b, K, N)
    if M == 0 or N == 0:
        return out
    bias = ep = None
    if epilogue is not None:
        bias, beta, alpha, bnz, anz = epilogue
        ep = (beta, alpha, bnz, anz)
    return _launch(dtype, 1, M, N, K, A, B, out, bias=bias, epilogue=ep, conj_a=ca, conj_b=cb)


# ---------------------------------------------------------------------------------------
# Public API (metalblas/dispatch.py:148-302)
# ---------------------------------------------------------------------------------------

def _matmul_nd(a, b, out=None):
    """Vector promotion and broadcast batches around the 2-D/3-D kernels
    (metalblas/dispatch.py:148-171)."""
    assert a.ndim and b.ndim, "matmul operands must be at least 1-D"
    a_vec, b_vec = a.ndim == 1, b.ndim == 1
    if a_vec:
        a = a.unsqueeze(0)
    if b_vec:
        b = b.unsqueeze(-1)
    M, K = a.shape[-2:]
    K2, N = b.shape[-2:]
    assert K == K2, f"shape mismatch: A is {a.shape}, B is {b.shape}"
    if a.ndim >= 3 and b.ndim == 2 and not b_vec and out is None and a.numel() and K:
        # (..., M, K) @ (K, N) with the leading dims of A foldable into its rows: one 2-D
        # product of (batch*M) x K, the same sums as the broadcast batches below, one launch
        try:
            a2 = a.view(-1, K)   # raises when the leading dims do not fold without a copy
        except RuntimeError:
            a2 = None
        if a2 is not None:
            return matmul(a2, b).view(*a.shape[:-1], N)
    batch = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    if batch:
        size = prod(batch)
        a3 = a.expand(*batch, M, K).reshape(size, M, K)
        b3 = b.expand(*batch, K, N).reshape(size, K, N)
        result = bmm(a3, b3).reshape(*batch, M, N)
    else:
        if (out is not None and (a_vec or b_vec) and out.dtype == a.dtype == b.dtype
                and out.device == a.device):
            # a 1-D result: write straight into out's (M, N) view, no temporary + copy
            o2 = out.unsqueeze(0) if a_vec and not b_vec else out.unsqueeze(-1) if b_vec and not a_vec \
                else out.reshape(1, 1)
            if o2.shape == (M, N) and o2.data_ptr() == out.data_ptr():
                matmul(a, b, out=o2)
                return out
        result = matmul(a, b)
    if a_vec:
        result = result.squeeze(-2)
    if b_vec:
        result = result.squeeze(-1)
    return out.copy_(result) if out is not None else result


def matmul(a: torch.Tensor, b: torch.Tensor, *, backend: str | None = None,
           tile: tuple | None = None, swizzle_log: int | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """Compute ``a @ b`` on the GPU (metalblas/dispatch.py:174-185)."""
    if _FAST is not None and out is None and backend is None and tile is None and swizzle_log is None:
        r = _FAST.matmul(a, b)
        if r is not None:
            return r
    if a.ndim != 2 or b.ndim != 2:
        return _matmul_nd(a, b, out)
    if _on_device(a) and (a.dtype in COMPLEX_DTYPES or b.dtype in COMPLEX_DTYPES):
        return _complex_matmul(a, b, out)
    if _on_device(a) and a.dtype in INT_DTYPES:
        return _int_matmul(a, b, out)
    return _float_matmul(a, b, backend, tile, swizzle_log, out)


def addmm(input: torch.Tensor, mat1: torch.Tensor, mat2: torch.Tensor, *,
          beta=1, alpha=1, out: torch.Tensor | None = None) -> torch.Tensor:
    """Compute ``beta * input + alpha * (mat1 @ mat2)`` with one final rounding
    (metalblas/dispatch.py:188-208)."""
    assert _on_device(mat1) and _on_device(mat2)
    assert mat1.dim() == 2 and mat2.dim() == 2, "addmm expects 2-D mat1, mat2"
    M, K = mat1.shape
    K2, N = mat2.shape
    assert K == K2, f"shape mismatch: mat1 is {mat1.shape}, mat2 is {mat2.shape}"
    dtype = mat1.dtype
    assert mat2.dtype == dtype, "addmm requires mat1.dtype == mat2.dtype"
    if out is not None:
        assert out.shape == (M, N) and out.dtype == dtype and _on_device(out)
    beta, alpha, bnz, anz = _scalars(dtype, beta, alpha)
    bias = input if (input.dtype == dtype and input.device == mat1.device) else \
        input.to(device=mat1.device, dtype=dtype)
    bias2 = bias.expand(M, N)
    epilogue = bias2, beta, alpha, bnz, anz
    if dtype in COMPLEX_DTYPES:
        return _complex_matmul(mat1, mat2, out, epilogue)
    if dtype in INT_DTYPES:
        return _int_matmul(mat1, mat2, out, epilogue)
    return _float_matmul(mat1, mat2, None, None, None, out, epilogue)


def _bmm_shape(a, b, op):
    """metalblas/dispatch.py:117-124."""
    assert _on_device(a) and _on_device(b), f"{op} expects cuda tensors"
    assert a.dim() == 3 and b.dim() == 3, f"{op} expects 3-D inputs"
    assert a.dtype == b.dtype, f"{op} requires both operands the same dtype"
    Bb, M, K = a.shape
    Bb2, K2, N = b.shape
    assert Bb == Bb2 and K == K2, f"{op} shape mismatch: {a.shape} @ {b.shape}"
    return Bb, M, N, K, a.dtype


def _bmm_out(a, out, Bb, M, N, dtype):
    if out is None:
        return a.new_empty(Bb, M, N)
    _check_out(out, (Bb, M, N), dtype)
    return out


def _batched(a, b, out, Bb, M, N, K, dtype, bias=None, epilogue=None):
    if dtype not in INT_DTYPES and dtype not in FLOAT_DTYPES and dtype not in COMPLEX_DTYPES:
        raise NotImplementedError(f"dtype {dtype} not supported")
    ca = cb = False
    if dtype in COMPLEX_DTYPES:
        a, ca = _conj_split(a)
        b, cb = _conj_split(b)
    A, B = _matrix_view(a, M, K), _matrix_view(b, K, N)
    return _launch(dtype, Bb, M, N, K, A, B, out, bias=bias, epilogue=epilogue,
                   conj_a=ca, conj_b=cb)


def bmm(a: torch.Tensor, b: torch.Tensor, *,
        out: torch.Tensor | None = None) -> torch.Tensor:
    """Batched 3-D matrix multiplication (metalblas/dispatch.py:211-225)."""
    if _FAST is not None and out is None:
        r = _FAST.bmm(a, b)
        if r is not None:
            return r
    Bb, M, N, K, dtype = _bmm_shape(a, b, "bmm")
    if Bb == 0 or M == 0 or N == 0:
        return out if out is not None else a.new_empty(Bb, M, N)
    if K == 0:
        return (out if out is not None else a.new_empty(Bb, M, N)).zero_()
    o = _bmm_out(a, out, Bb, M, N, dtype)
    return _batched(a, b, o, Bb, M, N, K, dtype)


def baddbmm(input: torch.Tensor, batch1: torch.Tensor, batch2: torch.Tensor, *,
            beta=1, alpha=1, out: torch.Tensor | None = None) -> torch.Tensor:
    """``beta * input + alpha * (batch1 @ batch2)`` (metalblas/dispatch.py:228-242)."""
    Bb, M, N, K, dtype = _bmm_shape(batch1, batch2, "baddbmm")
    beta, alpha, bnz, anz = _scalars(dtype, beta, alpha)
    o = _bmm_out(batch1, out, Bb, M, N, dtype)
    if Bb == 0 or M == 0 or N == 0:
        return o
    bias = input if (input.dtype == dtype and input.device == batch1.device) else \
        input.to(device=batch1.device, dtype=dtype)
    bias3 = bias.expand(Bb, M, N)
    return _batched(batch1, batch2, o, Bb, M, N, K, dtype, bias=bias3,
                    epilogue=(beta, alpha, bnz, anz))


def addbmm(input: torch.Tensor, batch1: torch.Tensor, batch2: torch.Tensor, *,
           beta=1, alpha=1, out: torch.Tensor | None = None) -> torch.Tensor:
    """``beta * input + alpha * sum_b(batch1[b] @ batch2[b])`` as one addmm with K' = Bb*K
    (metalblas/dispatch.py:245-260)."""
    Bb, M, N, K, dtype = _bmm_shape(batch1, batch2, "addbmm")
    if Bb == 0 or K == 0:
        # beta * input broadcast to (M, N): a K == 0 product with the fused epilogue
        empty_a = batch1.new_empty(M, 0)
        empty_b = batch1.new_empty(0, N)
        return addmm(input, empty_a, empty_b, beta=beta, alpha=alpha, out=out)
    A = batch1.permute(1, 0, 2).reshape(M, Bb * K)
    B = batch2.reshape(Bb * K, N)
    return addmm(input, A, B, beta=beta, alpha=alpha, out=out)


def dot(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """1-D inner product, matching ``torch.dot`` (metalblas/dispatch.py:263-271)."""
    assert a.dim() == 1 and b.dim() == 1, \
        f"1D tensors expected, but got {a.dim()}D and {b.dim()}D tensors"
    assert a.shape[0] == b.shape[0], \
        f"inconsistent tensor size, expected [{a.shape[0]}] and [{b.shape[0]}]"
    assert a.dtype == b.dtype, \
        f"dot : expected both vectors to have same dtype, got {a.dtype} and {b.dtype}"
    return matmul(a, b)


def vdot(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Inner product conjugating the first argument (metalblas/dispatch.py:274-276)."""
    return dot(a.conj() if a.is_complex() else a, b)


def outer(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Outer product of two vectors (metalblas/dispatch.py:279-283), computed as the K == 1
    product ``a[:, None] @ b[None, :]``; mixed dtypes promote as torch's ``*`` does."""
    assert a.dim() == 1, f"outer: Expected 1-D argument self, but got {a.dim()}-D"
    assert b.dim() == 1, f"outer: Expected 1-D argument vec2, but got {b.dim()}-D"
    if a.dtype != b.dtype:
        dt = torch.result_type(a, b)
        a, b = a.to(dt), b.to(dt)
    return matmul(a.unsqueeze(1), b.unsqueeze(0))


def mv(mat: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
    """Matrix-vector product (metalblas/dispatch.py:286-292)."""
    assert mat.dim() == 2 and vec.dim() == 1, \
        f"vector + matrix @ vector expected, got {mat.dim()}, {mat.dim()}, {vec.dim()}"
    assert mat.shape[1] == vec.shape[0], \
        f"size mismatch, got mat ({mat.shape[0]}x{mat.shape[1]}), vec ({vec.shape[0]})"
    return matmul(mat, vec)


gemm = matmul
ger = outer
