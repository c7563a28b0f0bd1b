"""jules_amd: the Jules fused-kernel path (fused GEMM + bias + activation,
flash-attention forward, W8A16 decode GEMM, int8 GEMM) as hand-written HIP for
MI355X (gfx950), behind the C ABI of include/jules_hip.h.

The kernels live in libjules_hip.so (built from jules_amd/csrc by
jules_amd/build.py).  `jules_amd.ops` calls them on torch GPU tensors;
`jules_amd._lib` is the raw ctypes binding.
"""
from ._lib import LIB_PATH, JulesHipError, kernel_names, lib, lookup  # noqa: F401

__all__ = ["LIB_PATH", "JulesHipError", "kernel_names", "lib", "lookup"]
