"""Drop-in for the reference builder module ``Libra5BlockOnline``
(TR-source/setup_online.py:8-15, TR-source/Block/block_online.cpp:873-876).

``block_sptc_2to4_online(row1, column1, values1, partSize_t, partSize_c, shortSize, density, window,
wide, tc_min_util, sptc_min_util, sptc_threshold)`` returns the same 30 tensors (29 arrays + build
time).  ``block_sptc_2to4_online_with_spill`` additionally returns the spill rows / columns /
values (entries the reference drops), which the parallel operator accepts as keyword arguments.
"""
from trspmm._native import ext as _ext

block_sptc_2to4_online = _ext().block_sptc_2to4_online
block_sptc_2to4_online_with_spill = _ext().block_sptc_2to4_online_with_spill
