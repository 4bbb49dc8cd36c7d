"""The builder oracle (oracle/builder_oracle.cpp) against the reference builder: committed golden
fixtures written by the compiled reference (tests/golden/make_golden.py), and oracle/_ref directly
when it is built in this container.  Plus the partition invariant and the fp16 packing rule."""
import os

import numpy as np
import pytest

from conftest import golden_files, load_golden, same_array
from oracle import builder as ob
from oracle import spmm as osp


@pytest.mark.parametrize("path", golden_files(), ids=lambda p: os.path.basename(p)[8:-4])
def test_oracle_matches_reference_fixture(path, golden_env):
    rowptr, col, val, params, env, outs = load_golden(path)
    golden_env(env)
    skip_tc = env.get("LIBRA_SKIP_TC") == "1"
    unit_min = int(env.get("LIBRA_SPTC_UNIT_MIN_NNZ", "2"))
    arrs, spill = ob.build(rowptr, col, val, skip_tc=skip_tc, unit_min_nnz=unit_min, **params)
    bad = [ob.SLOTS[i][0] for i in range(29) if not same_array(arrs[i], outs[i])]
    assert not bad, f"arrays differing from the reference: {bad}"


def test_golden_fixtures_present():
    assert len(golden_files()) >= 10


def _partition_fixtures():
    """Fixtures whose tuple partitions the input: not the non-canonical one (duplicates inside TC
    columns are carried twice by the reference TC values), and only window 16 (TC rows are encoded
    as window_id * 16 and the 64-bit row bitmaps wrap past row 15, block_online.cpp:474-494, so the
    TC arrays only mean what they say there)."""
    out = []
    for p in golden_files():
        if os.path.basename(p) == "builder_noncanonical.npz":
            continue
        if load_golden(p)[3]["window"] != 16:
            continue
        out.append(p)
    return out


@pytest.mark.parametrize("path", _partition_fixtures(), ids=lambda p: os.path.basename(p)[8:-4])
def test_partition_tuple_plus_spill_is_input(path, golden_env):
    rowptr, col, val, params, env, _ = load_golden(path)
    assert params["window"] == 16
    golden_env(env)
    arrs, spill = ob.build(rowptr, col, val, skip_tc=env.get("LIBRA_SKIP_TC") == "1",
                           unit_min_nnz=int(env.get("LIBRA_SPTC_UNIT_MIN_NNZ", "2")), **params)
    got = osp.coo_canonical(*osp.format_to_coo(arrs, spill, window=params["window"]))
    exp = osp.coo_canonical(*osp.csr_to_coo(rowptr, col, val))
    for g, e in zip(got, exp):
        assert np.array_equal(g, e)


def test_spill_is_what_2to4_drops():
    """A group whose 4 columns all hit one row keeps 2 values and spills 2 (block_online.cpp:690-694)."""
    # one window, one row with 4 count-1 columns -> one 4-column group, row keeps the first two
    rowptr = np.array([0, 4] + [4] * 15, dtype=np.int32)
    col = np.array([3, 5, 7, 9], dtype=np.int32)
    val = np.array([1, 2, 3, 4], dtype=np.float32)
    arrs, spill = ob.build(rowptr, col, val)
    assert arrs[17].tolist() == [[3, 5, 7, 9]]
    assert arrs[18][0, 0] == 0b1111
    assert arrs[19][0, 0].tolist() == [1.0, 2.0]
    assert arrs[20][0, 0].tolist() == [0, 1]
    assert spill[1].tolist() == [7, 9] and spill[2].tolist() == [3.0, 4.0]


@pytest.mark.parametrize("seed", range(4))
def test_oracle_matches_reference_module(seed, golden_env):
    import torch
    from trspmm import graphs
    # looked up in the body, not at collection: a `-m gpu` run never loads the compiled reference
    mod = ob.reference_module()
    if mod is None:
        pytest.skip("oracle/_ref not built (no /root/reference)")
    golden_env({})
    g = graphs.random_csr(150 + 40 * seed, 200, 0.04 * (seed + 1), seed=100 + seed)
    fd = os.dup(1)
    nul = os.open(os.devnull, os.O_WRONLY)
    os.dup2(nul, 1)
    try:
        ref = mod.block_sptc_2to4_online(torch.from_numpy(g.rowptr), torch.from_numpy(g.col), torch.from_numpy(g.val),
                                         32, 32, 3, 6, 16, 16, 0.0, 0.5, 12)
    finally:
        os.dup2(fd, 1)
        os.close(nul)
        os.close(fd)
    arrs, _ = ob.build(g.rowptr, g.col, g.val, density=6)
    for i in range(29):
        assert same_array(arrs[i], ref[i].numpy()), ob.SLOTS[i][0]


def test_half_packing_rule_matches_torch():
    """s_packed_a packs c10::Half (round to nearest even) pairs; pinned against torch's conversion."""
    import torch
    rng = np.random.default_rng(0)
    rowptr = np.arange(0, 17, dtype=np.int32)  # 16 rows, one entry each
    col = np.arange(16, dtype=np.int32) * 3
    val = (rng.standard_normal(16) * 10 ** rng.uniform(-6, 4, 16)).astype(np.float32)
    arrs, _ = ob.build(rowptr, col, val)
    decoded = osp.packed_to_coo(arrs[25], arrs[26], arrs[27], arrs[28])
    expect = torch.from_numpy(val).half().double().numpy()
    got = osp.coo_canonical(*decoded)
    exp = osp.coo_canonical(np.arange(16), col.astype(np.int64), expect)
    nz = exp[2] != 0
    assert np.array_equal(got[2], exp[2][nz])
