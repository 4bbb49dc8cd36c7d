"""CPU SpMM / SDDMM oracle and the meaning of the format arrays -- TEST INFRASTRUCTURE ONLY.

Functions
  csr_spmm(rowptr, col, val, B)        C = A B in float64 (A given as CSR; B dense).  The
                                        mathematics BASELINE.json fixes as the SpMM reference
                                        ("fp32 CSR SpMM", fp16 inputs).  Pinned by
                                        tests/test_oracle_spmm.py: dense brute force, identity,
                                        torch.sparse.mm CSR (fp32), linearity.
  csr_sddmm(rowptr, col, X, Y)         out[e] = X[row_e] . Y[col_e] in float64 (closed form).
                                        Pinned by the dense (X Y^T) sampled at the pattern and
                                        torch.sparse.sampled_addmm.
  format_to_coo(arrays, spill, window) every (row, col, value) the 29 builder arrays carry,
                                        decoded with the meaning the reference kernels give them:
                                          TC sub-blocks  mGCNkernel_online.cu:54-241
                                          2:4 groups     mGCNkernel_online.cu:248-337
                                          residual parts mGCNkernel.cu:976-1171
                                        Pinned by: format_to_coo(builder output incl. spill)
                                        reproduces the input CSR exactly (tests), and the packed
                                        tiles decode to the same 2:4 values (packed_to_coo).
  packed_to_coo(...)                   decode s_tile_column / s_packed_a / s_packed_meta
                                        (block_online.cpp:796-841, mGCNkernel_online.cu:812-933).
  spmm_error(C, R)                     the tolerance metric used by every parity test.
"""
from __future__ import annotations

import numpy as np


def csr_spmm(rowptr: np.ndarray, col: np.ndarray, val: np.ndarray, B: np.ndarray, m: int | None = None) -> np.ndarray:
    """C[m, K] = sum over stored entries val * B[col] (float64), rows [0, m)."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    m = rowptr.shape[0] - 1 if m is None else m
    B64 = np.asarray(B, dtype=np.float64)
    rows = np.repeat(np.arange(rowptr.shape[0] - 1), np.diff(rowptr))
    keep = rows < m
    C = np.zeros((m, B64.shape[1]), dtype=np.float64)
    np.add.at(C, rows[keep], np.asarray(val, dtype=np.float64)[keep, None] * B64[np.asarray(col)[keep]])
    return C


def coo_spmm(rows: np.ndarray, cols: np.ndarray, vals: np.ndarray, B: np.ndarray, m: int) -> np.ndarray:
    C = np.zeros((m, B.shape[1]), dtype=np.float64)
    keep = rows < m
    np.add.at(C, rows[keep], np.asarray(vals, dtype=np.float64)[keep, None] * np.asarray(B, dtype=np.float64)[cols[keep]])
    return C


def csr_sddmm(rowptr: np.ndarray, col: np.ndarray, X: np.ndarray, Y: np.ndarray) -> np.ndarray:
    rows = np.repeat(np.arange(len(rowptr) - 1), np.diff(rowptr))
    X64 = np.asarray(X, dtype=np.float64)
    Y64 = np.asarray(Y, dtype=np.float64)
    out = np.empty(len(col), dtype=np.float64)
    step = 1 << 18
    for s in range(0, len(col), step):
        out[s:s + step] = np.einsum("ij,ij->i", X64[rows[s:s + step]], Y64[col[s:s + step]])
    return out


def spmm_error(C: np.ndarray, R: np.ndarray) -> dict:
    """max |C - R| relative to max |R|, and the elementwise gate |C-R| <= 1e-2 |R| + 1e-3 max|R|
    (the floor absorbs cancellation: B entries in [-1, 1] make some outputs tiny)."""
    C = np.asarray(C, dtype=np.float64)
    R = np.asarray(R, dtype=np.float64)
    scale = float(np.max(np.abs(R))) if R.size else 0.0
    diff = np.abs(C - R)
    rel = float(diff.max() / scale) if R.size and scale > 0 else float(diff.max()) if R.size else 0.0
    ok = bool(np.all(diff <= 1e-2 * np.abs(R) + 1e-3 * max(scale, 1e-30))) if R.size else True
    return {"max_rel_to_max": rel, "elementwise_ok": ok}


def _tc_to_coo(a, rows, cols, vals):
    t_rowoff, t_blockoff, t_col, t_val, t_winrow, _t_atomic, t_bin = a[:7]
    for p in range(len(t_winrow)):
        for s in range(t_rowoff[p], t_rowoff[p + 1]):
            vi = int(t_blockoff[s])
            for half in range(2):
                bits = int(t_bin[2 * s + half]) & ((1 << 64) - 1)
                for b in range(64):
                    if bits >> b & 1:
                        r = half * 8 + b // 8
                        k = b % 8
                        c = int(t_col[8 * s + k])
                        if c >= 0:
                            rows.append(int(t_winrow[p]) + r)
                            cols.append(c)
                            vals.append(float(t_val[vi]))
                        vi += 1


def _residual_to_coo(off, row, col, val, rows, cols, vals):
    for i in range(len(row)):
        for e in range(off[i], off[i + 1]):
            rows.append(int(row[i]))
            cols.append(int(col[e]))
            vals.append(float(val[e]))


def format_to_coo(a: list, spill=None, window: int = 16, use_s_window: bool = True):
    """All (row, col, value) triples carried by the 29 arrays (+ spill when given), float64 values."""
    rows, cols, vals = [], [], []
    _tc_to_coo(a, rows, cols, vals)
    _residual_to_coo(a[7], a[8], a[10], a[11], rows, cols, vals)
    _residual_to_coo(a[12], a[13], a[15], a[16], rows, cols, vals)
    s_col, _s_mask, s_val, s_pos, s_win, s_off = a[17], a[18], a[19], a[20], a[21], a[22]
    G = s_col.shape[0]
    if G:
        wins = s_win if use_s_window else np.repeat(np.arange(len(s_off) - 1), np.diff(s_off))
        pos = s_pos.reshape(G, window, 2).astype(np.int64)
        valid = pos >= 0
        g_idx, lr, q = np.nonzero(valid)
        p = pos[g_idx, lr, q]
        c = s_col.reshape(G, 4)[g_idx, p]
        v = s_val.reshape(G, window, 2)[g_idx, lr, q]
        keep = c >= 0
        rows.extend((wins[g_idx] * window + lr)[keep].tolist())
        cols.extend(c[keep].tolist())
        vals.extend(v[keep].astype(np.float64).tolist())
    if spill is not None:
        rows.extend(np.asarray(spill[0]).tolist())
        cols.extend(np.asarray(spill[1]).tolist())
        vals.extend(np.asarray(spill[2], dtype=np.float64).tolist())
    return np.asarray(rows, dtype=np.int64), np.asarray(cols, dtype=np.int64), np.asarray(vals, dtype=np.float64)


def packed_to_coo(s_tile_column, s_packed_a, s_packed_meta, s_window_tile_offset, window: int = 16):
    """Decode the packed 2:4 tiles: (row, col, fp16 value as float64), zero entries omitted."""
    rows, cols, vals = [], [], []
    T = s_tile_column.shape[0]
    pa = np.asarray(s_packed_a, dtype=np.int64).reshape(T, 8, 4, 2) & 0xFFFFFFFF
    pm = np.asarray(s_packed_meta, dtype=np.int64).reshape(T, 8) & 0xFFFFFFFF
    tc = np.asarray(s_tile_column).reshape(T, 16)
    for w in range(len(s_window_tile_offset) - 1):
        for t in range(s_window_tile_offset[w], s_window_tile_offset[w + 1]):
            for rg in range(8):
                meta = int(pm[t, rg])
                for hsel in range(2):
                    lr = rg + 8 * hsel
                    if lr >= window:
                        continue
                    for c in range(4):
                        word = int(pa[t, rg, c, hsel])
                        m4 = (meta >> (16 * hsel + 4 * c)) & 15
                        for p, bits in ((m4 & 3, word & 0xFFFF), ((m4 >> 2) & 3, word >> 16)):
                            v = float(np.array([bits], dtype=np.uint16).view(np.float16)[0])
                            col = int(tc[t, 4 * c + p])
                            if v != 0.0 and col >= 0:
                                rows.append(w * window + lr)
                                cols.append(col)
                                vals.append(v)
    return np.asarray(rows, dtype=np.int64), np.asarray(cols, dtype=np.int64), np.asarray(vals, dtype=np.float64)


def coo_canonical(rows, cols, vals):
    """Sort triples by (row, col, value) for multiset comparison."""
    order = np.lexsort((vals, cols, rows))
    return rows[order], cols[order], vals[order]


def csr_to_coo(rowptr, col, val):
    rows = np.repeat(np.arange(len(rowptr) - 1), np.diff(rowptr)).astype(np.int64)
    return rows, np.asarray(col, dtype=np.int64), np.asarray(val, dtype=np.float64)


def torch_csr_spmm(rowptr, col, val, B, m: int | None = None, threads: int | None = None):
    """C = A B with torch.sparse.mm on CSR fp32 on the host CPU -- the "fp32 CSR SpMM" named as the
    reference result and as the CPU baseline (fp16 CSR is not implemented on CPU, so the
    fp16-exact values are upcast to fp32).  Pinned against csr_spmm (float64) in
    tests/test_oracle_spmm.py.  Returns a float32 numpy array."""
    import torch
    if threads:
        torch.set_num_threads(threads)
    m = len(rowptr) - 1 if m is None else m
    rp = torch.from_numpy(np.ascontiguousarray(rowptr[: m + 1], dtype=np.int64))
    nnz = int(rp[-1])
    A = torch.sparse_csr_tensor(rp, torch.from_numpy(np.ascontiguousarray(col[:nnz], dtype=np.int64)),
                                torch.from_numpy(np.ascontiguousarray(val[:nnz], dtype=np.float32)),
                                size=(m, B.shape[0]))
    Bt = B if isinstance(B, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(B, dtype=np.float32))
    return torch.sparse.mm(A, Bt.float())
