"""Kernel-library facts (the reference's ``metalblas.kernels`` module, metalblas/kernels.py).

The reference assembles Metal kernel variants at first use and exposes ``has_metal4()``
(metalblas/kernels.py:65-73), which its tests use to decide whether the matrix-unit
backends exist.  Here all kernel variants are compiled ahead of time into
libmetalblas_hip.so; ``has_metal4()`` keeps its meaning ("the matrix-unit GEMM path is
available") and is true on gfx950.
"""
from __future__ import annotations

from functools import lru_cache

import torch

from . import _lib


@lru_cache(maxsize=1)
def has_metal4() -> bool:
    """True when the current device runs the matrix-core (MFMA) GEMM family."""
    return has_matrix_cores()


def has_matrix_cores() -> bool:
    if not torch.cuda.is_available():
        return False
    return _lib.query(_lib.QUERY_HAS_MATRIX_CORES) == 1


def library_path() -> str:
    return _lib.LIB_PATH


def device_info() -> dict:
    """Architecture, CU count and LDS size as the library sees the current device."""
    return {
        "abi": _lib.query(_lib.QUERY_ABI_VERSION),
        "gfx": _lib.query(_lib.QUERY_GFX_ARCH),
        "cus": _lib.query(_lib.QUERY_CU_COUNT),
        "lds_bytes": _lib.query(_lib.QUERY_LDS_BYTES),
        "matrix_cores": bool(_lib.query(_lib.QUERY_HAS_MATRIX_CORES)),
    }


def plan(a, b, *, batch=None, backend=None, tile=None, out_dtype=None, out=None, tuned=False) -> dict:
    """The plan libmetalblas_hip.so would run for ``a @ b`` (2-D or 3-D tensors): kernel
    family, tile, split-K and workspace.  For tests and reports.  With ``tuned=True`` the plan
    the one-shot autotuner already chose for this call signature (``out``'s layout included)
    replaces the static one; nothing is timed here.  ``tile`` is a tile request as matmul's."""
    from . import planner
    from .dispatch import BACKENDS, _mat
    dtype = a.dtype
    if a.dim() == 3:
        Bb, M, K = a.shape
        N = b.shape[2]
        c = out if out is not None else torch.empty(Bb, M, N, dtype=out_dtype or dtype, device=a.device)
    else:
        Bb = 1
        M, K = a.shape
        N = b.shape[1]
        c = out if out is not None else torch.empty(M, N, dtype=out_dtype or dtype, device=a.device)
    desc = _lib.make_desc(dtype, Bb, M, N, K, _mat(a), _mat(b), _mat(c), backend=BACKENDS[backend], tile=tile)
    if tuned:
        choice = planner.cached().get(planner._key(desc, c.device))
        if choice is not None:
            planner.apply(desc, choice)
    info = _lib.plan(desc)
    return {
        "family": _lib.FAMILY_NAMES.get(info.family, str(info.family)),
        "tile": tuple(info.tile),
        "split_k": info.split_k,
        "swizzle_log": info.swizzle_log,
        "transposed": bool(info.transposed),
        "grid": tuple(info.grid),
        "block": info.block,
        "workspace_bytes": info.workspace_bytes,
    }
