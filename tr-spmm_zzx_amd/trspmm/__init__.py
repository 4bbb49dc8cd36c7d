"""MI355X-native hybrid fp16 SpMM / SDDMM (TR-SpMM "online" path), gfx950.

Layers
  graphs     seeded synthetic graphs (the benchmark configurations) as canonical CSR
  _native    ctypes binding of the C ABI (include/trspmm.h, libtrspmm.so) and the torch extension
  ops        Format (builder output, cache files), DeviceFormat (the builder on the GPU), Plan
             (device plan), spmm / sddmm on torch device tensors
  reorder    TCA row reorder (clusters rows with similar column sets into windows)
  matching   statistics-only 2:4 matcher (counts of pairs, groups, dense blocks, padding)
Drop-in module names live next to this package: Libra5BlockOnline, Libra6SpMMOnline, matching_utils.
"""
from .ops import (DeviceFormat, Format, Plan, build_format, build_format_cached,  # noqa: F401
                  build_format_device, spmm, sddmm)
