"""ctypes binding of libmetalblas_hip.so (the C ABI declared in include/metalblas_amd.h).

This replaces the reference's kernel-handle boundary: ``torch.mps.compile_shader(src)`` and
``lib.<kernel>(*buffers, threads=, group_size=)`` (metalblas/kernels.py:55-62 and every
``fn(...)`` call in metalblas/float_dispatch.py, integer_dispatch.py, complex_dispatch.py).
Tensors cross the boundary as raw device pointers (``data_ptr()``, storage offset included)
plus element strides; scalars as doubles / int64; the stream is torch's current HIP stream.
Split-K scratch is allocated here through torch's stream-ordered caching allocator.

There is no CPU fallback: if the library is missing the call raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# METALBLAS_LIB names another build of the same library (e.g. a sanitizer build for host tests)
LIB_PATH = os.environ.get("METALBLAS_LIB") or os.path.join(PKG_DIR, "libmetalblas_hip.so")

# mb_dtype codes
DTYPE_CODE = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.complex64: 3,
    torch.complex32: 4,
    torch.int8: 5,
    torch.uint8: 6,
    torch.int16: 7,
    torch.int32: 8,
    torch.int64: 9,
}

# mb_backend codes
BACKEND_AUTO, BACKEND_GEMV, BACKEND_MATRIX, BACKEND_TILED, BACKEND_GENERIC = range(5)

# mb_family codes
FAMILY_NAMES = {0: "none", 1: "fill", 2: "generic", 3: "mfma", 4: "gemv_dot", 5: "gemv_axpy"}

# mb_status codes
OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED_DTYPE = -2
ERR_UNSUPPORTED_LAYOUT = -3
ERR_WORKSPACE = -4
ERR_LAUNCH = -5
ERR_NO_DEVICE = -6
ERR_GEMV_SHAPE = -7
ERR_BAD_BACKEND = -8
ERR_SCRATCH_LIMIT = -9

# mb_gemm_desc.flags bits
FLAG_DRY_RUN = 1

# mb_query codes
QUERY_ABI_VERSION, QUERY_HAS_MATRIX_CORES, QUERY_CU_COUNT, QUERY_GFX_ARCH, QUERY_LDS_BYTES = range(5)

ABI_VERSION = 1

EXPORTED_SYMBOLS = ("mb_gemm", "mb_gemm_noalloc", "mb_gemm_noalloc_scratch_bytes",
                    "mb_gemm_workspace_bytes", "mb_plan", "mb_tile_candidates", "mb_query",
                    "mb_strerror")


class MbMatrix(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("row_stride", ctypes.c_int64),
                ("col_stride", ctypes.c_int64), ("batch_stride", ctypes.c_int64)]


class MbGemmDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32), ("backend", ctypes.c_int32),
        ("batch", ctypes.c_int64), ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("a", MbMatrix), ("b", MbMatrix), ("c", MbMatrix), ("bias", MbMatrix),
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


class MbPlanInfo(ctypes.Structure):
    _fields_ = [
        ("family", ctypes.c_int32), ("tile", ctypes.c_int32 * 8), ("split_k", ctypes.c_int32),
        ("swizzle_log", ctypes.c_int32), ("transposed", ctypes.c_int32),
        ("grid", ctypes.c_int32 * 3), ("block", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_int64),
    ]


_LIB = None


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes handle of libmetalblas_hip.so."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{os.path.basename(path)} is not built; run `python -m metalblas_amd._build` "
            "(or __graft_entry__.build()) first")
    lib = ctypes.CDLL(path)
    lib.mb_gemm.argtypes = [ctypes.POINTER(MbGemmDesc), ctypes.c_void_p]
    lib.mb_gemm.restype = ctypes.c_int
    lib.mb_gemm_noalloc.argtypes = [ctypes.POINTER(MbGemmDesc), ctypes.c_void_p]
    lib.mb_gemm_noalloc.restype = ctypes.c_int
    lib.mb_gemm_noalloc_scratch_bytes.argtypes = []
    lib.mb_gemm_noalloc_scratch_bytes.restype = ctypes.c_int64
    lib.mb_gemm_workspace_bytes.argtypes = [ctypes.POINTER(MbGemmDesc)]
    lib.mb_gemm_workspace_bytes.restype = ctypes.c_int64
    lib.mb_plan.argtypes = [ctypes.POINTER(MbGemmDesc), ctypes.POINTER(MbPlanInfo)]
    lib.mb_plan.restype = ctypes.c_int
    lib.mb_tile_candidates.argtypes = [ctypes.POINTER(MbGemmDesc), ctypes.POINTER(ctypes.c_int32),
                                       ctypes.c_int]
    lib.mb_tile_candidates.restype = ctypes.c_int
    lib.mb_query.argtypes = [ctypes.c_int32]
    lib.mb_query.restype = ctypes.c_int64
    lib.mb_strerror.argtypes = [ctypes.c_int32]
    lib.mb_strerror.restype = ctypes.c_char_p
    _LIB = lib
    return lib


def strerror(status: int) -> str:
    return load().mb_strerror(int(status)).decode()


def check(status: int) -> None:
    """Map an mb_status to the exception types the reference raises."""
    if status == OK:
        return
    msg = strerror(status)
    if status in (ERR_GEMV_SHAPE, ERR_BAD_BACKEND):
        raise ValueError(msg)
    if status == ERR_UNSUPPORTED_DTYPE:
        raise NotImplementedError(msg)
    raise RuntimeError(f"metalblas_amd: {msg} (status {status})")


def query(what: int) -> int:
    return int(load().mb_query(int(what)))


def matrix(t, rs=None, cs=None, bs=0) -> MbMatrix:
    """Describe tensor ``t`` as a strided matrix (element strides)."""
    if t is None:
        return MbMatrix(None, 0, 0, 0)
    return MbMatrix(ctypes.c_void_p(t.data_ptr()), int(rs), int(cs), int(bs))


def make_desc(dtype, batch, M, N, K, a, b, c, bias=None, *, conj_a=False, conj_b=False,
              epilogue=None, backend=BACKEND_AUTO, tile=None, swizzle_log=None,
              split_k=0, flags=0) -> MbGemmDesc:
    """Build a descriptor.  a/b/c/bias are (tensor, row_stride, col_stride, batch_stride).

    epilogue: None or (beta, alpha, beta_nz, alpha_nz) with beta/alpha already cast the way
    metalblas/dispatch.py:127-131 (_scalars) casts them.
    """
    d = MbGemmDesc()
    d.dtype = DTYPE_CODE[dtype]
    d.backend = backend
    d.batch, d.M, d.N, d.K = int(batch), int(M), int(N), int(K)
    d.a = matrix(*a)
    d.b = matrix(*b)
    d.c = matrix(*c)
    d.bias = matrix(*bias) if bias is not None else MbMatrix(None, 0, 0, 0)
    d.conj_a = int(bool(conj_a))
    d.conj_b = int(bool(conj_b))
    if epilogue is not None:
        beta, alpha, bnz, anz = epilogue
        d.epilogue = 1
        d.beta_nz = int(bool(bnz))
        d.alpha_nz = int(bool(anz))
        cb, ca = complex(beta), complex(alpha)
        d.beta_re, d.beta_im = cb.real, cb.imag
        d.alpha_re, d.alpha_im = ca.real, ca.imag
        d.beta_int = _wrap64(beta)
        d.alpha_int = _wrap64(alpha)
    d.swizzle_log = -1 if swizzle_log is None else int(swizzle_log)
    if tile is not None:
        vals = [int(v) for v in tile][:8]
        for i, v in enumerate(vals):
            d.tile[i] = v
    d.split_k = int(split_k)
    d.flags = int(flags)
    return d


def _wrap64(v) -> int:
    """Two's-complement int64 bits of an integer scalar (non-integers: truncated)."""
    try:
        iv = int(v.real) if isinstance(v, complex) else int(v)
    except (TypeError, ValueError, OverflowError):
        return 0
    iv &= (1 << 64) - 1
    return iv - (1 << 64) if iv >= (1 << 63) else iv


def plan(desc: MbGemmDesc) -> MbPlanInfo:
    info = MbPlanInfo()
    check(load().mb_plan(ctypes.byref(desc), ctypes.byref(info)))
    return info


def tile_candidates(desc: MbGemmDesc, cap: int = 16) -> list[tuple]:
    buf = (ctypes.c_int32 * (8 * cap))()
    n = load().mb_tile_candidates(ctypes.byref(desc), buf, cap)
    if n < 0:
        check(n)
    return [tuple(buf[8 * i: 8 * i + 8]) for i in range(n)]


def workspace_bytes(desc: MbGemmDesc) -> int:
    """Device scratch mb_gemm() needs for this descriptor."""
    n = int(load().mb_gemm_workspace_bytes(ctypes.byref(desc)))
    if n < 0:
        check(n)
    return n


def _device_index(device) -> int:
    if isinstance(device, int):
        return device
    return device.index if device.index is not None else torch.cuda.current_device()


def _current_stream(device) -> int:
    """Raw handle of torch's current HIP stream on ``device`` (a torch.device or an index; the
    same stream ``torch.cuda.current_stream(device).cuda_stream`` names, without building a
    Stream object: a few microseconds per call on small products)."""
    return torch._C._cuda_getCurrentRawStream(_device_index(device))


# Split-K workspace kept per (device, stream): the kernels of one stream run in order, so a
# call's scratch is free again for the next call queued on the same stream -- provided the
# calls' launch sequences do not interleave.  A call queues up to several kernels (a split-K
# product and its reduction) without the GIL, so two host threads on one stream could queue
# k1(A), k1(B), reduce(A), reduce(B) and A's reduction would read B's planes.  Each kept
# workspace therefore has a lock that its user holds while its kernels are queued.
# Workspaces above _WS_KEEP bytes are taken from the caching allocator per call instead.
_WS: dict = {}
_WS_KEEP = 64 << 20
_WS_LOCK = threading.Lock()


def workspace(idx: int, stream: int, nbytes: int):
    """(tensor, lock): a device tensor of at least ``nbytes`` of scratch for work queued on
    ``stream`` (torch's current stream), and the lock to hold while queuing the kernels that use
    it.

    The caller keeps the tensor referenced until its launch is queued: another host thread that
    needs more scratch on the same stream replaces the kept tensor, and the reference keeps the
    old block out of the caching allocator until then (stream order protects it after).

    While the stream is being captured into a HIP graph, the scratch is a new tensor instead:
    torch allocates it from the graph's private pool, which the graph holds for its replays.  A
    kept tensor could be replaced and freed by a later call while the graph still uses it."""
    if torch._C._cuda_isCurrentStreamCapturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=torch.device("cuda", idx)), _NO_LOCK
    key = (idx, stream)
    with _WS_LOCK:
        ent = _WS.get(key)
        if ent is None or ent[0].numel() < nbytes:
            t = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=torch.device("cuda", idx))
            ent = _WS[key] = (t, ent[1] if ent is not None else threading.Lock())
    return ent


_NO_LOCK = contextlib.nullcontext()


# 64-bit word indices of the pointer fields in MbGemmDesc (checked at import below)
W_A, W_B, W_C, W_BIAS, W_WS, W_WS_BYTES = 5, 9, 13, 17, 35, 36
DESC_WORDS = ctypes.sizeof(MbGemmDesc) // 8
assert ctypes.sizeof(MbGemmDesc) % 8 == 0 and (MbGemmDesc.a.offset, MbGemmDesc.b.offset, MbGemmDesc.c.offset,
        MbGemmDesc.bias.offset, MbGemmDesc.workspace.offset, MbGemmDesc.workspace_bytes.offset) == \
    tuple(8 * w for w in (W_A, W_B, W_C, W_BIAS, W_WS, W_WS_BYTES))


def launch(desc: MbGemmDesc, nbytes: int, device) -> None:
    """Queue the product on torch's current stream of ``device`` (the current device; a
    torch.device or an index) with ``nbytes`` of workspace."""
    idx = _device_index(device)
    stream = torch._C._cuda_getCurrentRawStream(idx)
    ws, lock = None, _NO_LOCK   # ws is held until mb_gemm has queued the kernels that use it
    if nbytes > 0:
        if nbytes <= _WS_KEEP:
            ws, lock = workspace(idx, stream, nbytes)
        else:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=torch.device("cuda", idx))
        desc.workspace = ws.data_ptr()
        desc.workspace_bytes = nbytes
    with lock:
        status = (_LIB or load()).mb_gemm(ctypes.byref(desc), stream)
    if status:
        check(status)
    # ws returns to torch's caching allocator (or stays kept); reuse is ordered on the stream
    del ws


def run(desc: MbGemmDesc, device) -> None:
    """Queue the product on torch's current stream of ``device``."""
    launch(desc, workspace_bytes(desc), device)
