"""Drop-in for the reference builder module ``Libra5BlockOnline``
(TR-source/setup_online.py:8-15, TR-source/Block/block_online.cpp:873-876).

``block_sptc_2to4_online(row1, column1, values1, partSize_t, partSize_c, shortSize, density, window,
wide, tc_min_util, sptc_min_util, sptc_threshold)`` returns the same 30 tensors (29 arrays + build
time).  ``block_sptc_2to4_online_with_spill`` additionally returns the spill rows / columns /
values (entries the reference drops), which the parallel operator accepts as keyword arguments.

The reference's 2:4 step keeps only the first two values of a row in each 4-column group, so the
29 arrays can describe fewer entries than the input (5.4% of R-MAT 2^20's entries).  This module
returns exactly the reference's arrays, and says so with a ``DroppedEntriesWarning`` (once per
process) the first time it drops anything: the operators then compute the product of what the
arrays carry, not A B, unless the spill is passed along.
"""
import warnings

from trspmm._native import ext as _ext


class DroppedEntriesWarning(UserWarning):
    """The builder's 2:4 groups dropped input entries (the reference's behaviour)."""


_warned = False


def block_sptc_2to4_online(*args):
    global _warned
    out = _ext().block_sptc_2to4_online_with_spill(*args)
    dropped = int(out[30].numel())
    if dropped and not _warned:
        _warned = True
        warnings.warn(f"block_sptc_2to4_online: the 2:4 groups keep two values per row and group, as the reference "
                      f"builder does, so {dropped} of {int(args[1].numel())} input entries are not in the 29 arrays and "
                      "the SpMM over them is not A B; block_sptc_2to4_online_with_spill returns those entries, "
                      "which forward_fp16_tcu_cuda_sptc_mma_parallel_online takes as spill_row / spill_col / "
                      "spill_val", DroppedEntriesWarning, stacklevel=2)
    return out[:30]


block_sptc_2to4_online_with_spill = _ext().block_sptc_2to4_online_with_spill
