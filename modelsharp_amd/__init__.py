"""MI355X-native MatMulNBits (INT4 block-quantized matmul) for ModelSharp.

Layout:
  csrc/          HIP kernels for gfx950 and the C ABI (include/ms_hip_kernels.h)
  lib/           the built libms_hip_nbits.so
  native.py      ctypes binding of the C ABI
  graph.py       the reference's operator interface (IKernel, KernelRegistry, ...)
  hip_kernel.py  HipMatMulNBitsKernel, the drop-in operator
  workloads.py   seeded synthetic workloads and their algorithmic cost
"""
from . import native  # noqa: F401

__all__ = ["native"]
