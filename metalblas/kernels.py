"""``metalblas.kernels`` (metalblas/kernels.py of the reference): ``has_metal4()`` keeps its
meaning, "the matrix-unit GEMM path is available", which on gfx950 is the MFMA family."""
from metalblas_amd.kernels import device_info, has_matrix_cores, has_metal4, library_path, plan

__all__ = ["has_metal4", "has_matrix_cores", "device_info", "library_path", "plan"]
