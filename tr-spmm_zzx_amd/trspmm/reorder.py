"""Row reorder before the builder: TCA clustering of rows with similar column sets
(trs_tca_reorder in include/trspmm.h; interface of spmm/tr_csr_fp16/tr_tca_reorder.py:44-357).

``apply_tca_reorder`` keeps the reference's signature and return values: the CSR of the first
``num_nodes`` rows in the new order (columns unchanged) and ``reorder_id[new] = old``.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np

from . import _native as nat


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def _params(**kw) -> nat.ReorderParams:
    p = nat.ReorderParams()
    nat.lib().trs_reorder_params_default(ctypes.byref(p))
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def tca_order(rowptr, col, ncols: int | None = None, thres: int = 16, cluster_thres: int = 128,
              num_perm: int = 128, lsh_threshold: float = 0.2, bucket_span: int = 64, exhaustive: bool = False,
              seed: int = 1, num_threads: int = 0, align_window: int = 0, minhash: int = 1) -> np.ndarray:
    """order[new_row] = old_row for the rows of the CSR (rowptr[rows+1], col[nnz]).
    minhash=1: the reference LSH library's MinHash family (bucket_span <= 0 then gives its
    candidate pairs exactly); align_window=W > 0 keeps clusters inside whole W-row windows (no
    reference counterpart)."""
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    col = np.ascontiguousarray(col, dtype=np.int32)
    rows = rowptr.shape[0] - 1
    if ncols is None:
        ncols = int(col.max()) + 1 if col.size else 0
    p = _params(thres=thres, cluster_thres=cluster_thres, num_perm=num_perm, lsh_threshold=lsh_threshold,
                bucket_span=bucket_span, exhaustive=int(bool(exhaustive)), seed=seed, num_threads=num_threads,
                align_window=align_window, minhash=minhash)
    order = np.empty(max(rows, 0), dtype=np.int32)
    nat.check(nat.lib().trs_tca_reorder(_ptr(rowptr), _ptr(col), rows, col.shape[0], int(ncols), ctypes.byref(p),
                                        _ptr(order)), "trs_tca_reorder")
    return order


def lsh_bands(threshold: float = 0.2, num_perm: int = 128) -> tuple:
    """(bands, rows per band) of the reorder's LSH for a Jaccard threshold."""
    b, r = ctypes.c_int32(), ctypes.c_int32()
    nat.check(nat.lib().trs_lsh_bands(threshold, num_perm, ctypes.byref(b), ctypes.byref(r)), "trs_lsh_bands")
    return b.value, r.value


def minhash_signatures(sets, count: int = 128, seed: int = 1, minhash: int = 1) -> np.ndarray:
    """[len(sets), count] uint32 MinHash values of the given sets of non-negative ints, as the
    reorder's LSH computes them."""
    off = np.zeros(len(sets) + 1, dtype=np.int64)
    np.cumsum([len(x) for x in sets], out=off[1:])
    elems = np.ascontiguousarray(np.concatenate([np.asarray(x, dtype=np.int32) for x in sets])
                                 if len(sets) and off[-1] else np.zeros(1, np.int32), dtype=np.int32)
    sig = np.empty((len(sets), count), dtype=np.uint32)
    p = _params(seed=seed, minhash=minhash)
    nat.check(nat.lib().trs_minhash_signatures(_ptr(off), _ptr(elems), len(sets), ctypes.byref(p), count, _ptr(sig)),
              "trs_minhash_signatures")
    return sig


def permute_rows(rowptr, col, order, *extra):
    """CSR whose row k is row order[k] of the input (entries keep their order); extra per-entry
    arrays are permuted alongside."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    order = np.asarray(order, dtype=np.int64)
    lens = rowptr[order + 1] - rowptr[order]
    new_ptr = np.zeros(order.shape[0] + 1, dtype=np.int64)
    np.cumsum(lens, out=new_ptr[1:])
    starts = np.repeat(rowptr[order] - new_ptr[:-1], lens)
    src = starts + np.arange(new_ptr[-1], dtype=np.int64)
    out = [new_ptr.astype(np.int32), np.asarray(col)[src]]
    out += [np.asarray(a)[src] for a in extra]
    return tuple(out)


def apply_tca_reorder(row_ptr, col_ind, num_nodes, thres=16, verbose=True, align_window=0):
    """Reorder the first ``num_nodes`` rows; returns (new_row_ptr, new_col_ind, reorder_id).
    align_window (not in the reference): see tca_order."""
    t0 = time.time()
    row_ptr = np.asarray(row_ptr, dtype=np.int32)[: num_nodes + 1]
    col_ind = np.asarray(col_ind, dtype=np.int32)[: int(row_ptr[-1])] if num_nodes > 0 else np.zeros(0, np.int32)
    order = tca_order(row_ptr, col_ind, thres=thres, align_window=align_window)
    new_ptr, new_col = permute_rows(row_ptr, col_ind, order)
    if verbose:
        print(f"TCA: total reorder time = {time.time() - t0:.2f}s")
    return new_ptr, new_col.astype(np.int32), order
