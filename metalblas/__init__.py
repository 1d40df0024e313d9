"""``import metalblas`` for PyTorch-ROCm tensors on MI355X.

The reference package's import name and public API (metalblas/__init__.py:1-19 of
Isalia20/metalBLAS): the same functions and the ``kernels`` module, implemented by
``metalblas_amd`` on hand-written gfx950 HIP kernels.  A caller of the reference changes only the
tensors' device (``"mps"`` -> ``"cuda"``).
"""
from metalblas_amd import (
    addbmm,
    addmm,
    baddbmm,
    bmm,
    dot,
    gemm,
    ger,
    matmul,
    mv,
    outer,
    vdot,
)

from . import kernels

__all__ = [
    "matmul", "gemm", "addmm", "bmm", "baddbmm", "addbmm",
    "dot", "vdot", "outer", "ger", "mv", "kernels",
]
