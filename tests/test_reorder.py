"""TCA row reorder (trs_tca_reorder) on the CPU: permutation and determinism properties, the
clustering rules against the oracle restatement (exhaustive candidates), hand-derived cases that
pin that restatement, and recovery of planted communities with LSH candidates."""
import numpy as np
import pytest

import trspmm
from trspmm import graphs, reorder, _native as nat
from oracle import tca as otca


def csr(rows_sets):
    rp = np.zeros(len(rows_sets) + 1, dtype=np.int32)
    rp[1:] = np.cumsum([len(s) for s in rows_sets])
    col = np.array([c for s in rows_sets for c in sorted(s)], dtype=np.int32)
    return rp, col


# hand-derived from the reference's rules (tr_tca_reorder.py:145-210, :282-340)
def test_oracle_hand_cases():
    # sim-1 pairs (0,2) and (1,3) merge first (key order), each closes at thres=2; the two
    # clusters have Jaccard 0 but are still candidates and share one level-2 group
    rp, col = csr([{5}, {1, 2}, {5}, {1, 2}])
    assert otca.tca_order(rp, col, thres=2) == [0, 2, 1, 3]
    # equal sizes: the second end folds into the first -> roots 0 then 1; thres=3 lets the
    # sim-0.5 pair merge into the closed-at-3 check later
    rp, col = csr([{1, 2}, {7}, {1, 2}, {1, 3}, {7}])
    # pairs: (0,2)=1, (1,4)=1, (0,3)=1/3, (2,3)=1/3; (0,2) -> {0,2}; (1,4) -> {1,4}; (0,3): 0 root,
    # 3 root -> size 2 vs 1 -> 3 into 0 -> size 3 closes; (2,3): not roots, root 0 closed -> skip
    assert otca.cluster([frozenset(s) for s in ({1, 2}, {7}, {1, 2}, {1, 3}, {7})], 3) == [0, 1, 0, 0, 1]
    assert otca.tca_order(rp, col, thres=3) == [0, 2, 3, 1, 4]
    # identical disjoint groups of 16 rows come out as contiguous groups
    sets = [{100 * (i % 5) + j for j in range(4)} for i in range(80)]
    order = otca.tca_order(*csr(sets), thres=16)
    assert [o % 5 for o in order] == sorted(o % 5 for o in order)
    # empty rows are never paired: all-empty input keeps the identity order
    rp = np.zeros(9, dtype=np.int32)
    assert otca.tca_order(rp, np.zeros(0, np.int32)) == list(range(8))


def random_clustered(rows, seed):
    rng = np.random.default_rng(seed)
    sets = []
    for i in range(rows):
        if rng.random() < 0.08:
            sets.append(set())
            continue
        base = (i * 7 // 3) % 11
        s = {base * 20 + int(x) for x in rng.integers(0, 12, size=rng.integers(2, 8))}
        s |= {int(x) for x in rng.integers(0, 400, size=rng.integers(0, 3))}
        sets.append(s)
    return csr(sets)


@pytest.mark.parametrize("seed,rows,thres,cthres", [(1, 60, 16, 128), (2, 90, 4, 3), (3, 120, 8, 2),
                                                    (4, 75, 2, 5), (5, 40, 1, 1)])
def test_native_matches_oracle_exhaustive(seed, rows, thres, cthres):
    rp, col = random_clustered(rows, seed)
    got = reorder.tca_order(rp, col, ncols=420, thres=thres, cluster_thres=cthres, exhaustive=True)
    want = otca.tca_order(rp, col, thres=thres, cluster_thres=cthres)
    assert got.tolist() == want


def test_planted_oracle_case_matches_native():
    rp, col = csr([{5}, {1, 2}, {5}, {1, 2}])
    assert reorder.tca_order(rp, col, thres=2, exhaustive=True).tolist() == [0, 2, 1, 3]


def scrambled_sbm(communities, seed):
    g = graphs.sbm(communities=communities, seed=seed, val_seed=seed + 1)
    m = g.m
    perm = np.random.default_rng(seed).permutation(m)          # new label -> old label
    inv = np.empty(m, np.int64)
    inv[perm] = np.arange(m)
    rp, c = reorder.permute_rows(g.rowptr[: m + 1], g.col, perm)
    return rp, inv[c].astype(np.int32), perm


def test_lsh_recovers_communities_and_is_deterministic():
    rp, col, perm = scrambled_sbm(600, 4)
    a = reorder.tca_order(rp, col)
    assert np.array_equal(np.sort(a), np.arange(rp.shape[0] - 1))
    b = reorder.tca_order(rp, col, num_threads=1)
    assert np.array_equal(a, b)                                  # thread-count independent
    comm = (perm[a] // 16).reshape(-1, 16)
    dominant = np.mean([np.bincount(w).max() / 16 for w in comm])
    base = (perm // 16).reshape(-1, 16)
    assert np.mean([np.bincount(w).max() / 16 for w in base]) < 0.2
    assert dominant > 0.6, dominant
    c = reorder.tca_order(rp, col, seed=7)                       # another MinHash seed: a permutation too
    assert np.array_equal(np.sort(c), np.arange(rp.shape[0] - 1))


def test_reorder_raises_dense_share():
    rp, col, perm = scrambled_sbm(400, 9)
    val = np.ones(col.shape[0], np.float32)
    before = trspmm.build_format(rp, col, val).slot(3).size
    order = reorder.tca_order(rp, col)
    rp2, col2, val2 = reorder.permute_rows(rp, col, order, val)
    after = trspmm.build_format(rp2, col2, val2).slot(3).size
    assert before == 0 and after > 0.1 * col.shape[0], (before, after)


def test_apply_tca_reorder_interface():
    rp, col, perm = scrambled_sbm(100, 2)
    # padded rows past num_nodes are ignored, as the reference slices num_nodes rows
    m = rp.shape[0] - 1
    rp_pad = np.concatenate([rp, np.full(16, rp[-1], np.int32)])
    new_ptr, new_col, rid = reorder.apply_tca_reorder(rp_pad, col, m, thres=16, verbose=False)
    assert new_ptr.shape == (m + 1,) and new_ptr.dtype == np.int32 and new_col.dtype == np.int32
    assert rid.shape == (m,) and np.array_equal(np.sort(rid), np.arange(m))
    for k in (0, 5, m - 1):
        old = rid[k]
        assert np.array_equal(new_col[new_ptr[k]:new_ptr[k + 1]], col[rp[old]:rp[old + 1]])


def test_reorder_errors():
    rp, col = csr([{1}, {2}])
    with pytest.raises(nat.TrsError):
        reorder.tca_order(rp, col, ncols=2)                      # column 2 out of range
    with pytest.raises(nat.TrsError):
        reorder.tca_order(np.array([0, 2, 1], np.int32), np.array([0, 1], np.int32))
    with pytest.raises(nat.TrsError):
        reorder.tca_order(rp, col, thres=0)
    assert reorder.tca_order(np.zeros(1, np.int32), np.zeros(0, np.int32)).shape == (0,)


# ---- window-aligned extension (no reference counterpart) ----

def test_oracle_aligned_hand_case():
    # thres 4: sim-1 pairs {0,2} and {1,3} merge; {0,2} + {4} would make 3 <= 4 -> merges; the
    # size-3 and size-2 clusters pack into bins of 4 as [3] and [2] (3 + 2 > 4)
    rp, col = csr([{5}, {1, 2}, {5}, {1, 2}, {5, 9}])
    clusters = otca.groups(otca.cluster([frozenset(s) for s in ({5}, {1, 2}, {5}, {1, 2}, {5, 9})], 4, capped=True))
    assert clusters == [[0, 2, 4], [1, 3]]
    assert otca.tca_order(rp, col, align_window=4) == [0, 2, 4, 1, 3]


@pytest.mark.parametrize("seed,rows,W,cthres", [(1, 60, 16, 128), (2, 90, 4, 3), (3, 120, 8, 2), (6, 77, 5, 4)])
def test_native_aligned_matches_oracle_exhaustive(seed, rows, W, cthres):
    rp, col = random_clustered(rows, seed)
    got = reorder.tca_order(rp, col, ncols=420, cluster_thres=cthres, exhaustive=True, align_window=W)
    want = otca.tca_order(rp, col, cluster_thres=cthres, align_window=W)
    assert got.tolist() == want


def test_aligned_windows_recover_communities():
    rp, col, perm = scrambled_sbm(600, 4)
    m = rp.shape[0] - 1
    plain = reorder.tca_order(rp, col)
    aligned = reorder.tca_order(rp, col, align_window=16)
    assert np.array_equal(np.sort(aligned), np.arange(m))
    def purity(order):
        comm = (perm[order] // 16).reshape(-1, 16)
        return np.mean([np.bincount(w).max() / 16 for w in comm])
    assert purity(aligned) > purity(plain) and purity(aligned) > 0.85, (purity(aligned), purity(plain))
    val = np.ones(col.shape[0], np.float32)
    tc = lambda o: trspmm.build_format(*reorder.permute_rows(rp, col, o, val)).slot(3).size
    assert tc(aligned) > tc(plain)


# ---- the LSH library's MinHash family (oracle/minhash_lsh.py) -------------------------------------

def test_oracle_lsh_primitives_are_the_libraries():
    """The restatement's two primitives: SHA-1 (hashlib) and numpy's legacy RandomState draws."""
    from oracle import minhash_lsh as ml
    assert ml.sha1_hash32(b"abc") == 0x363e99a9           # SHA-1("abc") starts a9 99 3e 36
    a, b = ml.permutations(2, seed=1)
    gen = np.random.RandomState(1)
    want = [int(gen.randint(1, (1 << 61) - 1, dtype=np.uint64)), int(gen.randint(0, (1 << 61) - 1, dtype=np.uint64)),
            int(gen.randint(1, (1 << 61) - 1, dtype=np.uint64)), int(gen.randint(0, (1 << 61) - 1, dtype=np.uint64))]
    assert [int(a[0]), int(b[0]), int(a[1]), int(b[1])] == want
    # a set's MinHash is the elementwise minimum over its elements' permuted hashes
    v = ml.minhash([7, 11], num_perm=4)
    assert np.array_equal(v, np.minimum(ml.minhash([7], num_perm=4), ml.minhash([11], num_perm=4)))
    assert np.array_equal(ml.minhash([], num_perm=4), np.full(4, (1 << 32) - 1, dtype=np.uint64))


@pytest.mark.parametrize("seed", [1, 2022])
def test_native_signatures_equal_the_lsh_library_restatement(seed):
    from oracle import minhash_lsh as ml
    rng = np.random.default_rng(seed)
    sets = [sorted({int(x) for x in rng.integers(0, 5_000_000, size=rng.integers(0, 30))}) for _ in range(40)]
    sets.append([0, 9, 10, 99, 100, 2_147_483_647])      # decimal strings of every length
    got = reorder.minhash_signatures(sets, count=128, seed=seed)
    perms = ml.permutations(128, seed)
    want = np.stack([ml.minhash(s, 128, seed, perms) for s in sets]).astype(np.uint32)
    assert np.array_equal(got, want)


def test_native_bands_equal_the_lsh_library_optimisation():
    from oracle import minhash_lsh as ml
    for t, n in [(0.2, 128), (0.1, 64), (0.3, 128), (0.5, 32), (0.7, 128), (0.9, 64)]:
        assert reorder.lsh_bands(t, n) == ml.optimal_param(t, n), (t, n)


@pytest.mark.parametrize("seed,rows,thres,cthres", [(1, 60, 16, 128), (2, 90, 4, 3), (3, 120, 8, 2),
                                                    (4, 75, 2, 5), (7, 150, 16, 4)])
def test_native_matches_oracle_with_lsh_candidates(seed, rows, thres, cthres):
    """The reference's settings (MinHash family of its LSH library, seed 1, threshold 0.2, 128
    permutations, every pair of a bucket): the same order as the oracle with the restated
    library's candidate pairs -- which differs from the exhaustive order on these inputs."""
    rp, col = random_clustered(rows, seed)
    got = reorder.tca_order(rp, col, ncols=420, thres=thres, cluster_thres=cthres, bucket_span=0)
    want = otca.tca_order(rp, col, thres=thres, cluster_thres=cthres, lsh=True)
    assert got.tolist() == want


def test_lsh_candidates_are_a_strict_subset_on_these_inputs():
    from oracle import minhash_lsh as ml
    rp, col = random_clustered(120, 3)
    sets = [frozenset(int(c) for c in col[rp[i]:rp[i + 1]]) for i in range(len(rp) - 1)]
    lsh = ml.candidate_pairs(sets)
    every = [(a, b) for a in range(len(sets)) if sets[a] for b in range(a + 1, len(sets)) if sets[b]]
    assert 0 < len(lsh) < len(every) and set(lsh) < set(every)
