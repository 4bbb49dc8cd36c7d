"""Writes tests/golden/matching_2to4.npz: inputs, parameters and the statistics dict of the
reference's statistics-only 2:4 matcher (matching_utils.match_2to4,
TR-source/Block/block_matching_window_para_dr.cpp, compiled from its own source into oracle/_ref by
`make -C oracle ref`).  Run in the development container, where /root/reference exists:

    python tests/golden/make_golden_matching.py

Case k is stored as `rp<k>` (int32 row pointers), `ci<k>` (int32 columns), `prm<k>` = [window_size,
dense_threshold, t_max] and `st<k>` = the dict's values in KEYS order (float64: every count is far
below 2^53).  The reference prints a table per call on stdout; it is discarded.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import matching as om  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
KEYS = ("total_rows", "total_cols", "total_nnz", "sparsity", "num_row_panels", "num_sptc_groups",
        "num_tc_blocks", "num_16x16_blocks", "block_padding_groups", "fine_fallback", "coarse_fallback",
        "fake_zeros", "tc_total_nnz", "tc_block_count", "tc_block_max_nnz", "tc_block_min_nnz")


def csr(rows, row_cols):
    rp = np.zeros(rows + 1, np.int32)
    rp[1:] = np.cumsum([len(c) for c in row_cols])
    ci = np.concatenate([np.asarray(c, np.int32) for c in row_cols]) if rows else np.zeros(0, np.int32)
    return rp, ci.astype(np.int32)


def random_csr(rows, cols, p, seed, shuffle=False, dup=False):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(rows):
        c = np.flatnonzero(rng.random(cols) < p)
        if dup and len(c):
            c = np.concatenate([c, rng.choice(c, size=max(1, len(c) // 3))])
        if shuffle:
            rng.shuffle(c)
        out.append(c)
    return csr(rows, out)


def group_window_edge(distances=(1024, 1025)):
    """One 16-row window per distance d whose only compatible pair of pairs is d pairs apart.

    Columns by id: P = {1}, {2} (disjoint: paired at once; G1 = 0, G2 = {1,2}); d - 1 filler pairs
    {1..8}, {1,2,9..15} (overlap 2, the least on offer; G1 = {1,2}, G2 = {1..15}: they conflict with
    P, each other and Q); Q = {3,4}, {3,5} last (G1 = {3}, G2 = {3,4,5}: compatible with P only).
    P groups with Q iff d is within the reference's 1024-pair search."""
    masks = []
    for d in distances:
        win = [1 << 1, 1 << 2]
        win += [sum(1 << b for b in range(1, 9)), (1 << 1) | (1 << 2) | sum(1 << b for b in range(9, 16))] * (d - 1)
        win += [(1 << 3) | (1 << 4), (1 << 3) | (1 << 5)]
        masks.append(win)
    rows = []
    for w, win in enumerate(masks):
        base = sum(len(x) for x in masks[:w])
        for r in range(16):
            rows.append([base + c for c, m in enumerate(win) if m >> r & 1])
    return csr(len(rows), rows)


def cases():
    yield random_csr(200, 300, 0.05, 1), (16, 8, 8)
    yield random_csr(64, 40, 0.6, 2), (16, 8, 8)          # dense: conflicts, pool, TC blocks
    yield random_csr(96, 64, 0.35, 3), (16, 4, 2)
    yield random_csr(128, 90, 0.3, 4), (16, 3, 0)          # t_max 0: only disjoint pairs
    yield random_csr(100, 80, 0.4, 5), (16, 1, 16)         # every pool column is a TC block
    yield random_csr(77, 120, 0.1, 6), (7, 8, 8)           # partial last window
    yield random_csr(64, 200, 0.08, 7), (1, 8, 8)
    yield random_csr(96, 150, 0.1, 8), (32, 8, 8)          # rows 16.. of a window set no bit
    yield random_csr(192, 150, 0.06, 9), (64, 8, 8)        # rows 32..47 alias bits 0..15
    yield random_csr(130, 100, 0.2, 10, shuffle=True, dup=True), (24, 5, 4)   # unsorted, duplicates
    yield random_csr(16, 8000, 0.045, 11), (16, 8, 8)      # > 1024 pairs in one window
    yield random_csr(32, 3000, 0.3, 12), (16, 16, 3)       # wide and dense
    rng = np.random.default_rng(13)                         # empty windows and rows, a hub row
    rows = [[] for _ in range(80)]
    for r in range(40, 80):
        rows[r] = sorted(set(rng.integers(0, 500, size=int(rng.integers(0, 12))).tolist()))
    rows[50] = list(range(0, 1500, 2))
    yield csr(80, rows), (16, 8, 8)
    yield csr(1, [[5]]), (16, 8, 8)                         # one entry
    yield csr(3, [[0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3]]), (16, 2, 8)   # identical rows
    yield group_window_edge(), (16, 8, 8)                   # the 1024-pair limit, both sides


def run_reference(mod, rp, ci, prm):
    fd = os.dup(1)
    nul = os.open(os.devnull, os.O_WRONLY)
    sys.stdout.flush()
    os.dup2(nul, 1)
    try:
        d = mod.match_2to4(rp, ci, np.ones(len(ci), np.float32), *prm)
        ctypes.CDLL(None).fflush(None)          # the table is printed through C stdio
    finally:
        os.dup2(fd, 1)
        os.close(nul)
        os.close(fd)
    return d


def main():
    mod = om.reference_module()
    if mod is None:
        sys.exit("oracle/_ref is not built (make -C oracle ref, needs /root/reference)")
    blob = {"keys": np.asarray(KEYS)}
    for k, ((rp, ci), prm) in enumerate(cases()):
        d = run_reference(mod, rp, ci, prm)
        assert tuple(d.keys()) == KEYS, d.keys()
        blob[f"rp{k}"], blob[f"ci{k}"] = rp, ci
        blob[f"prm{k}"] = np.asarray(prm, np.int32)
        blob[f"st{k}"] = np.asarray([d[x] for x in KEYS], np.float64)
        print(k, "rows", len(rp) - 1, "nnz", len(ci), "params", prm, "groups", d["num_sptc_groups"],
              "tc", d["num_tc_blocks"], "fine", d["fine_fallback"], "coarse", d["coarse_fallback"])
    np.savez_compressed(os.path.join(HERE, "matching_2to4.npz"), **blob)


if __name__ == "__main__":
    main()
