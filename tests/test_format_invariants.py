"""Structural invariants of the builder output (rules of TR-source/Block/block_online.cpp:
partition of the input, offsets, bit counts, tile counts, packing, atomic flags), checked on synthetic graphs larger than the golden fixtures and
with varied parameters.  The fixtures pin bit-exactness on their inputs; these pin the array
relations everywhere else."""
import numpy as np
import pytest

import trspmm
from trspmm import graphs

CASES = [
    ("rmat12", lambda: graphs.rmat(scale=12, edge_factor=16, seed=3), {}),
    ("sbm", lambda: graphs.sbm(communities=300, seed=4, val_seed=5), {}),
    ("grid", lambda: graphs.grid_hubs(side=64, hubs=3, hub_degree=900, seed=2, val_seed=3), {}),
    ("rand_small_parts", lambda: graphs.random_csr(500, 300, 0.08, seed=7),
     dict(part_t=2, part_c=5, short_size=2, density=3)),
    ("rand_w8", lambda: graphs.random_csr(400, 260, 0.1, seed=8, window=8), dict(window=8, density=4)),
]


def build(g, **p):
    return trspmm.build_format(g.rowptr, g.col, g.val, skip_tc=False, unit_min_nnz=2, **p)


def popcount64(x):
    x = x.astype(np.uint64)
    c = np.zeros(x.shape, np.int64)
    for s in range(0, 64, 8):
        c += np.array([bin(i).count("1") for i in range(256)], np.int64)[((x >> np.uint64(s)) & np.uint64(255)).astype(np.int64)]
    return c


@pytest.mark.parametrize("name,gen,over", CASES, ids=[c[0] for c in CASES])
def test_format_invariants(name, gen, over):
    g = gen()
    p = dict(part_t=32, part_c=32, short_size=3, density=8, window=16)
    p.update(over)
    f = build(g, **p)
    a = f.arrays()
    w = p["window"]
    rows = g.rowptr.shape[0] - 1
    nwin = (rows + w - 1) // w
    (t_rowoff, t_blockoff, t_col, t_val, t_winrow, t_atomic, t_bin, c_off, c_row, c_atomic, c_col, c_val,
     cs_off, cs_row, cs_atomic, cs_col, cs_val, s_col, s_mask, s_val, s_pos, s_win, s_off, tile_win,
     tile_group, tile_cols, packed_a, packed_meta, win_tile_off) = a

    # TC parts (a9, a10): offsets, part sizes, value counts = popcount of the two bitmaps
    S = t_blockoff.shape[0] - 1
    assert t_rowoff[0] == 0 and np.all(np.diff(t_rowoff) > 0) and t_rowoff[-1] == S
    assert np.all(np.diff(t_rowoff) <= p["part_t"])
    assert t_blockoff[0] == 0 and t_blockoff[-1] == t_val.shape[0] and t_bin.shape[0] == 2 * S
    assert np.array_equal(np.diff(t_blockoff), popcount64(t_bin[0::2]) + popcount64(t_bin[1::2]))
    assert t_col.shape[0] == 8 * S and np.all(t_winrow % 16 == 0)
    # a sub-block's columns ascend, padding last; every non-empty bitmap column exists
    tc = t_col.reshape(S, 8)
    for s in range(S):
        real = tc[s][tc[s] >= 0]
        assert np.all(np.diff(real) > 0) and np.all(tc[s][len(real):] == -1)

    # residual parts (a8): long parts <= part_c, short parts <= short_size, atomic flags 0/1
    for off, prow, at, lim in ((c_off, c_row, c_atomic, p["part_c"]), (cs_off, cs_row, cs_atomic, p["short_size"])):
        assert off[0] == 0 and np.all(np.diff(off) >= 1) and off.shape[0] == prow.shape[0] + 1
        assert np.all(np.diff(off) <= lim) and set(np.unique(at)) <= {0, 1}
        assert np.all((prow >= 0) & (prow < rows))
    # a row longer than part_c is split into atomic parts (block_online.cpp:415-439)
    lens = np.diff(c_off)
    full = lens == p["part_c"]
    if full.any():
        assert np.all(c_atomic[full] == 1)

    # 2:4 groups (a6, a7): offsets per window, window ids, columns ascending with -1 padding
    G = s_col.shape[0]
    assert s_off.shape[0] == nwin + 1 and s_off[0] == 0 and s_off[-1] == G and np.all(np.diff(s_off) >= 0)
    assert np.array_equal(s_win, np.repeat(np.arange(nwin), np.diff(s_off)))
    for r in s_col:
        real = r[r >= 0]
        assert np.all(np.diff(real) > 0) and np.all(r[len(real):] == -1) and len(real) >= 1
    # kept positions are mask bits, at most two per row, in ascending position order
    pos = s_pos.astype(np.int64)
    kept = pos >= 0
    assert np.all(kept[:, :, 0] | ~kept[:, :, 1])
    both = kept[:, :, 0] & kept[:, :, 1]
    assert np.all(pos[:, :, 0][both] < pos[:, :, 1][both])
    bits = (s_mask[:, :, None].astype(np.int64) >> np.clip(pos, 0, 3)) & 1
    assert np.all(bits[kept] == 1)
    # a row's first two present columns are the kept ones (the rest of the mask is what drops)
    nkept = kept.sum(2)
    npresent = np.array([[bin(int(x)).count("1") for x in row] for row in s_mask])
    assert np.array_equal(nkept, np.minimum(npresent, 2))
    assert np.all(s_val[~kept] == 0)

    # tiles of 4 groups per window (a11)
    ng_w = np.diff(s_off)
    assert np.array_equal(np.diff(win_tile_off), (ng_w + 3) // 4)
    T = tile_win.shape[0]
    assert win_tile_off[-1] == T and tile_cols.shape == (T, 16) and packed_a.shape == (T, 8, 4, 2)
    assert np.array_equal(tile_win, np.repeat(np.arange(nwin), np.diff(win_tile_off)))
    expect_first = np.concatenate([s_off[wi] + 4 * np.arange(n) for wi, n in enumerate(np.diff(win_tile_off))]) \
        if T else np.zeros(0, np.int64)
    assert np.array_equal(tile_group, expect_first)
    for t in range(T):
        g0 = tile_group[t]
        for k in range(16):
            gg = g0 + k // 4
            want = s_col[gg, k % 4] if gg < s_off[tile_win[t] + 1] else -1
            assert tile_cols[t, k] == want

    # every stored input entry is carried by exactly one share or the spill (covered elsewhere
    # bit-for-bit); here: the totals add up
    sp_r, sp_c, sp_v = f.spill()
    total = t_val.shape[0] + int(kept.sum()) + c_col.shape[0] + cs_col.shape[0] + sp_r.shape[0]
    assert total == g.nnz
