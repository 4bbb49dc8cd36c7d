"""Restatement of the reference's statistics-only 2:4 matcher -- TEST INFRASTRUCTURE ONLY (see
oracle/__init__).  Pure Python, for small inputs.

Follows TR-source/Block/block_matching_window_para_dr.cpp (module `matching_utils`, built by
TR-source/setup_24matching.py:8-12):
  * per window of `window_size` rows: every distinct column gets a 16-bit row mask, bit
    (1 << local_row) cast to 16 bits -- rows 16..31 and 48..63 of a wider window set no bit but
    still create the column, rows 32..47 alias rows 0..15 (x86 shift count mod 32) (:289-307);
    nnz = popcount(mask)
  * columns by ascending id (:110-113); sliding 1:2 pairing: column i takes the first later
    unmatched column of zero overlap within 32 positions, else the first one of least overlap
    <= t_max, else it goes to the dense pool (fine fallback) (:120-157)
  * 2:4 grouping of the pairs: pair i takes the first later unused pair within 1024 positions
    with Z = (G1a & G2b) | (G2a & G1b) == 0; fake zeros += 2 * rows - nnz of the four columns;
    unmatched pairs put their two columns into the pool (coarse fallback += 2) (:166-210)
  * routing: full blocks of dense_threshold pool columns become TC blocks (nnz statistics), the
    rest go two per group into padded 2:4 groups (fake zeros) (:218-259)
  * tiles: groups per window rounded up to multiples of 4 (:264-270); totals summed over windows
    (:336-352)
The reference's counters are 32-bit ints; these are Python ints (they differ only on overflow).
"""
from __future__ import annotations

import glob
import os

HERE = os.path.dirname(os.path.abspath(__file__))
SEARCH_WINDOW = 32
GROUP_SEARCH_WINDOW = 1024


def _popcount(x: int) -> int:
    return bin(x).count("1")


def match_window(win_rows, columns, dense_threshold, t_max, st):
    """columns: list of (col_id, mask) sorted by col_id.  Updates the totals in st."""
    n = len(columns)
    nnz_of = {c: _popcount(m) for c, m in columns}
    matched = [False] * n
    pairs, pool = [], []
    for i in range(n):
        if matched[i]:
            continue
        ci, mi = columns[i]
        best, min_cost = -1, t_max + 1
        for j in range(i + 1, min(i + 1 + SEARCH_WINDOW, n)):
            if matched[j]:
                continue
            cost = _popcount(mi & columns[j][1])
            if cost == 0:
                best = j
                break
            if cost <= t_max and cost < min_cost:
                min_cost, best = cost, j
        if best != -1:
            cj, mj = columns[best]
            pairs.append((ci, cj, (mi & mj) & 0xFFFF, (mi | mj) & 0xFFFF, nnz_of[ci] + nnz_of[cj]))
            matched[i] = matched[best] = True
        else:
            pool.append(ci)
            matched[i] = True
            st["fine_fallback"] += 1
    sptc, tc = [], []
    used = [False] * len(pairs)
    for i, pa in enumerate(pairs):
        if used[i]:
            continue
        found = False
        for j in range(i + 1, min(i + 1 + GROUP_SEARCH_WINDOW, len(pairs))):
            if used[j]:
                continue
            pb = pairs[j]
            if ((pa[2] & pb[3]) | (pa[3] & pb[2])) & 0xFFFF == 0:
                sptc += [pa[0], pa[1], pb[0], pb[1]]
                st["fake_zeros"] += win_rows * 2 - (pa[4] + pb[4])
                used[i] = used[j] = True
                found = True
                break
        if not found:
            pool += [c for c in (pa[0], pa[1]) if c >= 0]
            used[i] = True
            st["coarse_fallback"] += 2
    nd, done = len(pool), 0
    while nd - done >= dense_threshold:
        block = sum(nnz_of[c] for c in pool[done:done + dense_threshold])
        tc += pool[done:done + dense_threshold]
        st["tc_total_nnz"] += block
        st["tc_block_count"] += 1
        st["tc_block_max_nnz"] = max(st["tc_block_max_nnz"], block)
        st["tc_block_min_nnz"] = min(st["tc_block_min_nnz"], block)
        done += dense_threshold
    idx = done
    for _ in range((nd - done + 1) // 2):
        fb = 0
        for k in range(4):
            if k < 2 and idx < nd:
                sptc.append(pool[idx])
                fb += nnz_of[pool[idx]]
                idx += 1
            else:
                sptc.append(-1)
        st["fake_zeros"] += win_rows * 2 - fb
    groups = len(sptc) // 4
    blocks = (groups + 3) // 4
    st["num_sptc_groups"] += groups
    st["num_tc_blocks"] += len(tc) // dense_threshold
    st["num_16x16_blocks"] += blocks
    st["block_padding_groups"] += blocks * 4 - groups


def match_2to4(row_ptr, col_ind, window_size=16, dense_threshold=8, t_max=8) -> dict:
    rows = len(row_ptr) - 1
    nnz = len(col_ind)
    cols = max(0, int(max(col_ind)) + 1) if nnz else 0
    if window_size < 1 or window_size > 64:
        raise RuntimeError("window_size must be in [1, 64]")
    if rows <= 0 or cols <= 0:
        raise RuntimeError("invalid matrix dimensions")
    st = dict(total_rows=rows, total_cols=cols, total_nnz=int(row_ptr[rows]),
              sparsity=1.0 - float(row_ptr[rows]) / (float(rows) * cols),
              num_row_panels=(rows + window_size - 1) // window_size, num_sptc_groups=0, num_tc_blocks=0,
              num_16x16_blocks=0, block_padding_groups=0, fine_fallback=0, coarse_fallback=0, fake_zeros=0,
              tc_total_nnz=0, tc_block_count=0, tc_block_max_nnz=0, tc_block_min_nnz=999999)
    for w in range(st["num_row_panels"]):
        r0, r1 = w * window_size, min(w * window_size + window_size, rows)
        masks = {}
        for r in range(r0, r1):
            # the reference shifts an int by local_row and stores 16 bits; x86 takes shift counts
            # mod 32, so rows 32..47 of a 64-row window reuse bits 0..15 and rows 16..31, 48..63
            # set none (block_matching_window_para_dr.cpp:298)
            bit = (1 << ((r - r0) & 31)) & 0xFFFF
            for e in range(row_ptr[r], row_ptr[r + 1]):
                masks[int(col_ind[e])] = masks.get(int(col_ind[e]), 0) | bit
        if not masks:
            continue
        match_window(r1 - r0, sorted(masks.items()), dense_threshold, t_max, st)
    return st


_ref_mod = None


def reference_module():
    """The reference matcher compiled from /root/reference into _ref/ (None when absent), loaded
    from its file without entering sys.modules (``import matching_utils`` elsewhere keeps
    resolving to the product's drop-in module).  It prints a statistics table on every call."""
    global _ref_mod
    if _ref_mod is None:
        import importlib.util
        hits = glob.glob(os.path.join(HERE, "_ref", "matching_utils*.so"))
        if not hits:
            return None
        spec = importlib.util.spec_from_file_location("matching_utils", hits[0])
        _ref_mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(_ref_mod)
    return _ref_mod
