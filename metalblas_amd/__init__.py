"""metalblas for MI355X: the metalblas matmul API on hand-written gfx950 HIP kernels.

Drop-in for Isalia20/metalBLAS (``import metalblas_amd as metalblas``): same functions,
keyword arguments, result dtypes and error behaviour (metalblas/__init__.py:1-19), on
PyTorch-ROCm tensors instead of ``mps`` tensors.
"""
from . import kernels
from .dispatch import (
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

__all__ = [
    "matmul", "gemm", "addmm", "bmm", "baddbmm", "addbmm",
    "dot", "vdot", "outer", "ger", "mv", "kernels",
]
