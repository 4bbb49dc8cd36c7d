"""MI355X-native hybrid fp16 SpMM / SDDMM (TR-SpMM "online" path), gfx950.

Layers
  graphs     seeded synthetic graphs (the benchmark configurations) as canonical CSR
  _native    ctypes binding of the C ABI (include/trspmm.h, libtrspmm.so) and the torch extension
  ops        Format (builder output, cache files), Plan (device plan), spmm / sddmm on torch
             device tensors
  reorder    TCA row reorder (clusters rows with similar column sets into windows)
Drop-in module names live next to this package: Libra5BlockOnline, Libra6SpMMOnline.
"""
from .ops import Format, Plan, build_format, build_format_cached, spmm, sddmm  # noqa: F401
