"""Restatement of the reference's TCA row reorder -- TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Follows spmm/tr_csr_fp16/tr_tca_reorder.py:
  * Jaccard of two sets (:26-41)
  * greedy clustering over candidate pairs: max-similarity first, both ends roots -> merge the
    smaller-or-equal cluster into the other (equal sizes: p2 into p1), close a cluster once it
    reaches `thres`; otherwise re-queue the pair of roots scored by the roots' own sets unless
    that pair is queued (:145-190, level 2 :282-323)
  * clusters in first-appearance order of their roots, members ascending (:195-205, :325-331)
  * final order: level-2 groups, their level-1 clusters, their rows (:333-340)
Candidate pairs are every pair of non-empty sets, or those of the restated LSH library
(oracle/minhash_lsh.py, lsh=True); equal similarities pop in pair-key order, then by the first end
(the reference's queue order for ties is not reproducible: it follows Python's per-process string
hashing).  The clustering and ordering rules are pinned by hand-derived cases in
tests/test_reorder.py, the LSH restatement by numpy's RandomState and hashlib there.
"""
from __future__ import annotations

import heapq


def jaccard(a: frozenset, b: frozenset) -> float:
    if not a or not b:
        return 0.0
    inter = len(a & b)
    union = len(a | b)
    return inter / union if union else 0.0


def cluster(sets: list, thres: int, capped: bool = False, pairs=None) -> list:
    """Root of every set after the greedy union-find clustering; candidate pairs (a < b) given,
    or every pair of non-empty sets.  capped (the library's window-aligned extension, no reference
    counterpart): merges that would exceed `thres` members are skipped."""
    n = len(sets)
    key = lambda a, b: (min(a, b) * n + max(a, b))   # noqa: E731
    heap, queued = [], set()
    if pairs is None:
        pairs = [(a, b) for a in range(n) if sets[a] for b in range(a + 1, n) if sets[b]]
    for a, b in pairs:
        heapq.heappush(heap, (-jaccard(sets[a], sets[b]), key(a, b), a, b))
        queued.add(key(a, b))
    cid = list(range(n))
    size = [1] * n
    closed = [False] * n
    open_clusters = n

    def root(i):
        while i != cid[i]:
            cid[i] = cid[cid[i]]
            i = cid[i]
        return i

    while heap and open_clusters > 0:
        _, k, p1, p2 = heapq.heappop(heap)
        queued.discard(k)
        if p1 == cid[p1] and p2 == cid[p2]:
            if closed[p1] or closed[p2]:
                continue
            if capped and size[p1] + size[p2] > thres:
                continue
            into, frm = (p2, p1) if size[p1] < size[p2] else (p1, p2)
            cid[frm] = into
            open_clusters -= 1
            size[into] += size[frm]
            if size[into] >= thres:
                closed[into] = True
                open_clusters -= 1
        else:
            r1, r2 = root(p1), root(p2)
            if closed[r1] or closed[r2]:
                continue
            if r1 != r2 and key(r1, r2) not in queued:
                heapq.heappush(heap, (-jaccard(sets[r1], sets[r2]), key(r1, r2), r1, r2))
                queued.add(key(r1, r2))
    return [root(i) for i in range(n)]


def groups(roots: list) -> list:
    out, index = [], {}
    for i, r in enumerate(roots):
        if r not in index:
            index[r] = len(out)
            out.append([])
        out[index[r]].append(i)
    return out


def aligned_order(clusters: list, supers: list, W: int) -> list:
    """Window-aligned layout (extension): per level-2 group, first-fit-decreasing packing of its
    clusters into W-row bins; full bins in group order, the clusters of partial bins packed again
    at the end with full bins first."""
    def pack(ids):
        bins, fill = [], []
        for c in sorted(ids, key=lambda c: -len(clusters[c])):   # sorted() is stable
            for b in range(len(bins)):
                if fill[b] + len(clusters[c]) <= W:
                    bins[b].append(c)
                    fill[b] += len(clusters[c])
                    break
            else:
                bins.append([c])
                fill.append(len(clusters[c]))
        return bins, fill

    order, leftover = [], []
    for grp in supers:
        bins, fill = pack(grp)
        for b, f in zip(bins, fill):
            if f == W:
                order += [r for c in b for r in clusters[c]]
            else:
                leftover += b
    bins, fill = pack(leftover)
    order += [r for b, f in zip(bins, fill) if f == W for c in b for r in clusters[c]]
    order += [r for b, f in zip(bins, fill) if f != W for c in b for r in clusters[c]]
    return order


def tca_order(rowptr, col, thres: int = 16, cluster_thres: int = 128, align_window: int = 0,
              lsh: bool = False, seed: int = 1) -> list:
    """order[new_row] = old_row, both levels; candidates exhaustive, or (lsh) the restated LSH
    library's at the reference's settings (threshold 0.2, 128 permutations, :60-61, :213-214)."""
    rows = len(rowptr) - 1
    sets = [frozenset(int(c) for c in col[rowptr[i]:rowptr[i + 1]]) for i in range(rows)]

    def pairs(ss):
        if not lsh:
            return None
        from oracle import minhash_lsh
        return minhash_lsh.candidate_pairs(ss, 0.2, 128, seed)

    if align_window > 0:
        clusters = groups(cluster(sets, align_window, capped=True, pairs=pairs(sets)))
    else:
        clusters = groups(cluster(sets, thres, pairs=pairs(sets)))
    csets = [frozenset().union(*(sets[r] for r in cl)) for cl in clusters]
    supers = groups(cluster(csets, cluster_thres, pairs=pairs(csets)))
    if align_window > 0:
        return aligned_order(clusters, supers, align_window)
    return [r for grp in supers for c in grp for r in clusters[c]]
