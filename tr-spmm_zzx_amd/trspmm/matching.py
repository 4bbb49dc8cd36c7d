"""Statistics-only 2:4 matching (trs_match_2to4 in include/trspmm.h); the interface of the
reference's matching_utils.match_2to4 (TR-source/Block/block_matching_window_para_dr.cpp:361-451).

``match_2to4`` returns the reference's dict (same keys, same order, Python ints and a float) and
raises ``RuntimeError`` (a ``TrsError``) where the reference raises, plus on the inputs the reference
does not survive (dense_threshold < 1 loops forever there; negative columns and out-of-range row
pointers are read out of bounds).  With ``verbose`` (default, like the reference) the statistics
are printed as a table.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as nat

KEYS = tuple(f[0] for f in nat.MatchStats._fields_)


def match_2to4(row_ptr, col_ind, values=None, window_size: int = 16, dense_threshold: int = 8, t_max: int = 8,
               *, num_threads: int = 0, verbose: bool = True) -> dict:
    """row_ptr / col_ind: CSR (any integer dtype, converted to int32 like the reference's forcecast);
    values are accepted and unused, as in the reference."""
    rp = np.ascontiguousarray(row_ptr, dtype=np.int32)
    ci = np.ascontiguousarray(col_ind, dtype=np.int32)
    if rp.ndim != 1 or ci.ndim != 1 or rp.shape[0] < 1:
        raise nat.TrsError(1, "match_2to4", "row_ptr and col_ind must be 1-D, row_ptr non-empty")
    st = nat.MatchStats()
    rc = nat.lib().trs_match_2to4(ctypes.c_void_p(rp.ctypes.data), ctypes.c_void_p(ci.ctypes.data),
                                  rp.shape[0] - 1, ci.shape[0], int(window_size), int(dense_threshold), int(t_max),
                                  int(num_threads), ctypes.byref(st))
    nat.check(rc, "match_2to4")
    out = {k: getattr(st, k) for k in KEYS}
    if verbose:
        print(format_stats(out), flush=True)
    return out


def format_stats(d: dict) -> str:
    """The statistics as a text table (the reference prints the same fields, :392-428)."""
    lines = [f"matrix               {d['total_rows']} x {d['total_cols']}, nnz {d['total_nnz']}, "
             f"sparsity {100.0 * d['sparsity']:.4f}%",
             f"row panels           {d['num_row_panels']}",
             f"2:4 groups           {d['num_sptc_groups']}",
             f"dense TC blocks      {d['num_tc_blocks']}"]
    if d["tc_block_count"] > 0:
        avg = d["tc_total_nnz"] / d["tc_block_count"]
        lines.append(f"TC block nnz         avg {avg:.1f}  min {d['tc_block_min_nnz']}  max {d['tc_block_max_nnz']}"
                     f"  (density avg {avg / 128:.4f})")
    lines += [f"16x16 tiles          {d['num_16x16_blocks']} ({d['block_padding_groups']} padding groups)",
              f"fine fallback        {d['fine_fallback']} columns",
              f"coarse fallback      {d['coarse_fallback']} columns",
              f"fake zeros           {d['fake_zeros']}"]
    return "\n".join(lines)
