"""opennpu_amd: OpenNPU's int4 weight-only quantized matmul hot path on one AMD Instinct MI355X.

The product is libonpu_hip.so (opennpu_amd/csrc, C ABI in include/onpu.h): hand-written HIP
kernels for gfx950 behind the reference's libonpu entry points. Python modules:
  _lib       loads the library and declares its ABI
  device     torch-tensor wrappers over the device-pointer entry points
  synthetic  seeded inputs with the benchmark distributions
  build      hipcc build of the library
"""
from ._lib import FMT_G128S, FMT_NAMES, FMT_Q4_0, FMT_Q4NX, FMT_Q4S, LibraryMissing, lib, require_gpu  # noqa: F401
