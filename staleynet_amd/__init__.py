"""MI355X (gfx950) implementation of StaleyNET's GEMM hot path.

The product is ``libstaleynet_gemm.so`` (C ABI: ``include/staleynet_gemm.h``),
hand-written HIP kernels behind the reference's ``Gpu::matmul`` boundary.
This package holds its sources (``csrc/``), the build (``build.py``), the
C++ host mirror (``host/``) and the Python mirror of the reference API
(``gemm.py``).
"""
from .gemm import (BatchStrides, Gpu, GpuError, Mask, MatmulKernel, MatmulPanic, MatmulSpec, Precision, Shape,
                   Storage, Tensor, WriteMode, library, status_string, validate)

__all__ = ["BatchStrides", "Gpu", "GpuError", "Mask", "MatmulKernel", "MatmulPanic", "MatmulSpec", "Precision",
           "Shape", "Storage", "Tensor", "WriteMode", "library", "status_string", "validate"]
