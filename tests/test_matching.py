"""Statistics-only 2:4 matcher: the drop-in ``matching_utils.match_2to4`` (libtrspmm,
trs_match_2to4) against the reference (TR-source/Block/block_matching_window_para_dr.cpp).

Pins, in order of strength:
  * golden fixtures written by the compiled reference (tests/golden/make_golden_matching.py) --
    oracle and native code must reproduce every statistic exactly;
  * hand-derived known answers and accounting identities that hold whatever the matching decides;
  * the oracle (oracle/matching.py) against the native code on seeded random inputs with varied
    parameters, and oracle/_ref itself on a large graph where it is built.
"""
import ctypes
import os

import numpy as np
import pytest

import matching_utils
from oracle import matching as om
from trspmm import graphs
from trspmm import _native as nat

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "matching_2to4.npz")


def _cases():
    z = np.load(FIXTURE)
    keys = [str(k) for k in z["keys"]]
    k = 0
    while f"rp{k}" in z:
        yield k, z[f"rp{k}"], z[f"ci{k}"], [int(x) for x in z[f"prm{k}"]], dict(zip(keys, z[f"st{k}"].tolist()))
        k += 1


CASES = list(_cases())


def native(rp, ci, ws=16, dt=8, tm=8, **kw):
    return matching_utils.match_2to4(rp, ci, np.ones(len(ci), np.float32), ws, dt, tm, verbose=False, **kw)


@pytest.mark.parametrize("k", range(len(CASES)))
def test_oracle_matches_reference_fixture(k):
    _, rp, ci, prm, want = CASES[k]
    got = om.match_2to4(rp, ci, *prm)
    assert {x: float(got[x]) for x in want} == want


@pytest.mark.parametrize("k", range(len(CASES)))
def test_native_matches_reference_fixture(k):
    _, rp, ci, prm, want = CASES[k]
    got = native(rp, ci, *prm)
    assert list(got) == list(want)                       # same keys, same order
    assert {x: float(got[x]) for x in want} == want
    assert all(isinstance(got[x], int) for x in want if x != "sparsity")


def test_fixture_set_covers_the_rules():
    prms = [tuple(c[3]) for c in CASES]
    assert {p[0] for p in prms} >= {1, 7, 16, 24, 32, 64}                 # window sizes
    assert any(c[4]["num_tc_blocks"] > 0 for c in CASES)                 # TC routing
    assert any(c[4]["fine_fallback"] > 0 and c[4]["coarse_fallback"] > 0 for c in CASES)
    assert any(c[4]["num_sptc_groups"] > 2048 // 2 for c in CASES if c[4]["num_row_panels"] == 1)   # > 1024 pairs


def _csr(rows):
    rp = np.zeros(len(rows) + 1, np.int32)
    rp[1:] = np.cumsum([len(r) for r in rows])
    return rp, np.asarray([c for r in rows for c in r], np.int32)


def test_known_answer_disjoint_rows():
    # masks: c0 = c1 = 0b01, c2 = c3 = 0b10.  1:2: c0 skips c1 (overlap 1), takes c2 (overlap 0);
    # c1 takes c3.  Pairs (G1, G2) = (0, 0b11) twice: Z = 0, one 2:4 group holding all 4 entries,
    # 2 rows * 2 - 4 = 0 fake zeros; one tile with 3 padding groups.
    d = native(*_csr([[0, 1], [2, 3]]))
    assert (d["num_sptc_groups"], d["num_16x16_blocks"], d["block_padding_groups"]) == (1, 1, 3)
    assert (d["fine_fallback"], d["coarse_fallback"], d["fake_zeros"], d["num_tc_blocks"]) == (0, 0, 0, 0)
    assert (d["total_rows"], d["total_cols"], d["total_nnz"]) == (2, 4, 4) and d["sparsity"] == 0.5
    assert d["tc_block_min_nnz"] == 999999 and d["tc_block_max_nnz"] == 0


def test_known_answer_identical_rows():
    # three equal rows over columns 0..3: every mask 0b111, pairs (0,1), (2,3) with overlap 3 <= 8,
    # G1 = G2 = 0b111 so the pairs conflict: 4 columns to the pool (coarse 4), two TC blocks of
    # 2 columns x 3 entries at dense_threshold 2; no groups, no fake zeros.
    d = native(*_csr([[0, 1, 2, 3]] * 3), dt=2)
    assert (d["num_tc_blocks"], d["tc_block_count"], d["tc_total_nnz"]) == (2, 2, 12)
    assert (d["tc_block_min_nnz"], d["tc_block_max_nnz"], d["coarse_fallback"], d["fine_fallback"]) == (6, 6, 4, 0)
    assert d["num_sptc_groups"] == 0 and d["fake_zeros"] == 0
    # t_max 2 forbids those pairs: all four columns are fine fallbacks
    d = native(*_csr([[0, 1, 2, 3]] * 3), dt=2, tm=2)
    assert (d["fine_fallback"], d["coarse_fallback"], d["num_tc_blocks"]) == (4, 0, 2)
    # dense_threshold 8: the 4 pooled columns fill 2 fallback groups of 2 columns, 3 rows:
    # 2 * (2*3 - 6) fake zeros
    d = native(*_csr([[0, 1, 2, 3]] * 3), dt=8, tm=2)
    assert (d["num_sptc_groups"], d["fake_zeros"], d["num_16x16_blocks"], d["block_padding_groups"]) == (2, 0, 1, 2)


def test_known_answer_group_search_limit():
    # tests/golden/make_golden_matching.py:group_window_edge: in window A the only compatible pair
    # of pairs is 1024 pairs apart (grouped: 1 group), in window B 1025 (not grouped).  Pools:
    # A = 1023 filler pairs = 2046 columns -> 255 TC blocks of 8 + 6 columns in 3 fallback groups;
    # B = 1024 filler pairs + P + Q = 2052 columns -> 256 TC blocks + 2 fallback groups.
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_golden_matching import group_window_edge
    d = native(*group_window_edge())
    assert (d["num_sptc_groups"], d["num_tc_blocks"], d["coarse_fallback"], d["fine_fallback"]) == (6, 511, 4098, 0)
    # a filler pair holds 8 + 9 = 17 entries, so a block of 4 filler pairs holds 68; window B's
    # pool starts with P's two 1-entry columns: its first block holds 2 + 3 * 17 = 53, and its
    # fallback groups hold one filler pair and Q (2 + 2 entries)
    assert d["tc_block_max_nnz"] == 68 and d["tc_block_min_nnz"] == 53
    # fake zeros = 32 slots per group minus its entries: A: P+Q 32 - 6, 3 x (32 - 17); B: 32 - 17, 32 - 4
    assert d["fake_zeros"] == 26 + 3 * 15 + 15 + 28


def _accounting(d, rp, ws, dt):
    """Identities that hold whatever pairs are chosen (window_size <= 16, unique columns)."""
    rows = rp.shape[0] - 1
    assert d["num_16x16_blocks"] * 4 - d["block_padding_groups"] == d["num_sptc_groups"]
    assert d["tc_block_count"] == d["num_tc_blocks"] and d["coarse_fallback"] % 2 == 0
    pool = d["fine_fallback"] + d["coarse_fallback"]
    assert pool >= d["num_tc_blocks"] * dt
    # every entry sits in a TC block or a 2:4 group of 2 * window_rows slots; per-window group
    # counts are not returned, so the identity is checked where all windows are full
    if rows % ws == 0:
        assert d["fake_zeros"] == 2 * ws * d["num_sptc_groups"] - (d["total_nnz"] - d["tc_total_nnz"])


@pytest.mark.parametrize("seed", range(12))
def test_native_matches_oracle_random(seed):
    rng = np.random.default_rng(100 + seed)
    ws = int(rng.choice([1, 2, 5, 8, 16, 16, 16, 20, 33, 48, 64]))
    dt = int(rng.choice([1, 2, 4, 8, 16]))
    tm = int(rng.choice([-1, 0, 1, 3, 8, 16]))
    rows = int(rng.integers(1, 300))
    cols = int(rng.integers(1, 400))
    p = float(rng.choice([0.01, 0.05, 0.2, 0.5]))
    lists = [np.flatnonzero(rng.random(cols) < p) for _ in range(rows)]
    if seed % 3 == 0:                     # unsorted rows with duplicates
        lists = [rng.permutation(np.concatenate([r, r[: len(r) // 2]])) for r in lists]
    rp, ci = _csr(lists)
    if ci.size == 0:
        rp, ci = _csr([[0]] + lists[1:])
    want = om.match_2to4(rp, ci, ws, dt, tm)
    got = native(rp, ci, ws, dt, tm)
    assert got == pytest.approx(want, rel=0, abs=0)
    if ws <= 16 and seed % 3 != 0:
        _accounting(got, rp, ws, dt)


def test_thread_count_does_not_change_the_result():
    g = graphs.rmat(scale=13, edge_factor=16, seed=3)
    rp, ci = g.rowptr.astype(np.int32), g.col.astype(np.int32)
    a = native(rp, ci, num_threads=1)
    for t in (2, 3, 8):
        assert native(rp, ci, num_threads=t) == a
    _accounting(a, rp, 16, 8)


def test_native_matches_compiled_reference_large():
    ref = om.reference_module()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    g = graphs.rmat(scale=15, edge_factor=16, seed=5)
    rp, ci = g.rowptr.astype(np.int32), g.col.astype(np.int32)
    for ws, dt, tm in ((16, 8, 8), (8, 4, 2), (32, 16, 8)):
        fd = os.dup(1)
        nul = os.open(os.devnull, os.O_WRONLY)
        os.dup2(nul, 1)
        try:
            want = ref.match_2to4(rp, ci, np.ones(len(ci), np.float32), ws, dt, tm)
            ctypes.CDLL(None).fflush(None)
        finally:
            os.dup2(fd, 1)
            os.close(nul)
            os.close(fd)
        assert native(rp, ci, ws, dt, tm) == want


@pytest.mark.parametrize("args,code", [
    (dict(ws=0), 1), (dict(ws=65), 1), (dict(dt=0), 1),
])
def test_bad_parameters_raise(args, code):
    rp, ci = _csr([[0, 1], [2]])
    with pytest.raises(RuntimeError) as e:
        native(rp, ci, **args)
    assert e.value.code == code


def test_bad_inputs_raise():
    with pytest.raises(RuntimeError, match="invalid matrix dimensions"):       # no rows
        native(np.zeros(1, np.int32), np.zeros(0, np.int32))
    with pytest.raises(RuntimeError, match="invalid matrix dimensions"):       # no columns
        native(np.zeros(5, np.int32), np.zeros(0, np.int32))
    with pytest.raises(nat.TrsError) as e:
        native(np.array([0, 2], np.int32), np.array([1, -3], np.int32))
    assert e.value.code == 5
    with pytest.raises(nat.TrsError, match="monotone"):
        native(np.array([0, 2, 1, 3], np.int32), np.array([0, 1, 2], np.int32))
    with pytest.raises(nat.TrsError, match=r"\[0, nnz\]"):
        native(np.array([0, 2, 9], np.int32), np.array([0, 1, 2], np.int32))


def test_verbose_prints_the_table(capsys):
    rp, ci = _csr([[0, 1], [2, 3]])
    matching_utils.match_2to4(rp, ci, None)
    out = capsys.readouterr().out
    assert "2:4 groups" in out and "fake zeros" in out
