"""GPU format builder (trs_build_online_device) against the host builder (trs_build_online), which
the reference pins (tests/test_builder.py): all 32 slots -- the reference's 29 arrays and the spill
list -- bit for bit, on the reference-written golden fixtures, on graphs whose windows take each of
the device builder's window kernels (one wave; a workgroup with the unit order in LDS; in global
memory), with the builder parameters and environment settings varied, and at the full BASELINE
sizes of configurations 1, 2, 3 and 5.  Inputs the device builder does not take (rows not
strictly increasing, windows of more than 16 rows) are refused with the documented status."""
import os

import numpy as np
import pytest
import torch

from conftest import golden_files, load_golden, same_array
from trspmm import _native as nat
from trspmm import graphs
import trspmm

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.cuda.init()


DEFAULT = dict(part_t=32, part_c=32, short_size=3, density=8, window=16, tc_min_util=0.0)


def device_build(rowptr, col, val, p):
    rp = torch.from_numpy(np.ascontiguousarray(rowptr, dtype=np.int32)).cuda()
    c = torch.from_numpy(np.ascontiguousarray(col, dtype=np.int32)).cuda()
    v = torch.from_numpy(np.ascontiguousarray(val, dtype=np.float32)).cuda()
    return trspmm.build_format_device(rp, c, v, part_t=p["part_t"], part_c=p["part_c"], short_size=p["short_size"],
                                      density=p["density"], window=p["window"], tc_min_util=p["tc_min_util"])


def host_build(rowptr, col, val, p):
    return trspmm.build_format(rowptr, col, val, part_t=p["part_t"], part_c=p["part_c"], short_size=p["short_size"],
                               density=p["density"], window=p["window"], tc_min_util=p["tc_min_util"])


def assert_same_format(df, hf, what):
    f = df.download()
    assert f.rows == hf.rows and f.window == hf.window
    bad = [(trspmm.ops.SLOT_NAMES[i], f.slot(i).shape, hf.slot(i).shape)
           for i in range(32) if not same_array(f.slot(i), hf.slot(i))]
    assert not bad, f"{what}: slots differing from the host builder: {bad}"
    return f


@pytest.mark.parametrize("path", golden_files(), ids=lambda p: os.path.basename(p)[8:-4])
def test_device_builder_matches_golden_fixtures(path, golden_env):
    rowptr, col, val, params, env, outs = load_golden(path)
    golden_env(env)
    name = os.path.basename(path)
    say("case", name)
    p = dict(DEFAULT, **params)
    if name == "builder_noncanonical.npz":
        with pytest.raises(nat.TrsError) as e:
            device_build(rowptr, col, val, p)
        assert e.value.code == 4   # TRS_ENOTCANON: the host builder takes such input
        return
    if p["window"] > 16:
        with pytest.raises(nat.TrsError) as e:
            device_build(rowptr, col, val, p)
        assert e.value.code == 1 and "16" in str(e.value)
        return
    df = device_build(rowptr, col, val, p)
    f = assert_same_format(df, host_build(rowptr, col, val, p), name)
    arrs = f.arrays()
    for i in range(29):
        assert same_array(arrs[i], outs[i]), (name, trspmm.ops.SLOT_NAMES[i])


def hub_window(rows, per_row, n, seed):
    """One or a few windows of long random rows: thousands to ~100k distinct columns per window."""
    rng = np.random.default_rng(seed)
    cols = [np.sort(rng.choice(n, size=per_row, replace=False)) for _ in range(rows)]
    rowptr = np.concatenate([[0], np.cumsum([len(c) for c in cols])]).astype(np.int32)
    col = np.concatenate(cols).astype(np.int32)
    val = rng.uniform(-1, 1, col.shape[0]).astype(np.float16).astype(np.float32)
    return graphs.Graph(f"hub{rows}x{per_row}", rows, n, rowptr, col, val)


def blend(seed):
    """Windows of every size class at once: SBM blocks, hub windows, empty rows, a partial last
    window."""
    a = graphs.sbm(communities=256, seed=seed, val_seed=seed)
    b = hub_window(32, 3000, 200000, seed + 1)
    m = a.m + 40 + b.m + 7
    rng = np.random.default_rng(seed + 2)
    tail = [np.sort(rng.choice(5000, size=k, replace=False)) for k in (3, 0, 9, 1, 0, 17, 2)]
    rows = [a.col[a.rowptr[r]:a.rowptr[r + 1]] for r in range(a.m)] + [np.zeros(0, np.int32)] * 40
    rows += [b.col[b.rowptr[r]:b.rowptr[r + 1]] for r in range(b.m)] + tail
    rowptr = np.concatenate([[0], np.cumsum([len(x) for x in rows])]).astype(np.int32)
    col = np.concatenate(rows).astype(np.int32)
    val = rng.uniform(0, 1, col.shape[0]).astype(np.float16).astype(np.float32)
    return graphs.Graph("blend", m, 200000, rowptr, col, val)


CASES = [
    ("er4096", lambda: graphs.erdos_renyi_gcn(), {}),
    ("rmat14", lambda: graphs.rmat(scale=14, edge_factor=16, seed=21), {}),
    ("rmat16", lambda: graphs.rmat(scale=16, edge_factor=16, seed=26), {}),
    ("sbm4k", lambda: graphs.sbm(communities=4096, seed=22, val_seed=23), {}),
    ("grid256_hubs", lambda: graphs.grid_hubs(side=256, hubs=8, hub_degree=5000, seed=24, val_seed=25), {}),
    # one window with ~40k units (workgroup kernel, order in LDS)
    ("hub16_lds", lambda: hub_window(16, 5000, 1 << 22, 3), {}),
    # one window with ~80k units (workgroup kernel, order in global memory)
    ("hub16_global", lambda: hub_window(16, 10000, 1 << 22, 4), {}),
    ("blend", lambda: blend(7), {}),
    ("blend_params", lambda: blend(8), dict(part_t=3, part_c=5, short_size=1, density=5, tc_min_util=0.45)),
    ("w8", lambda: graphs.random_csr(600, 400, 0.05, seed=3, window=8), dict(window=8, density=3)),
    ("w1", lambda: graphs.random_csr(300, 100, 0.2, seed=4, window=1), dict(window=1, density=1)),
    ("w5_partial", lambda: graphs.random_csr(203, 300, 0.1, seed=5, window=5), dict(window=5, density=2)),
    ("rand_dense", lambda: graphs.random_csr(400, 300, 0.2, seed=1), {}),
]


@pytest.mark.parametrize("name,gen,over", CASES, ids=[c[0] for c in CASES])
def test_device_builder_matches_host_builder(name, gen, over, golden_env):
    golden_env({})
    g = gen()
    say("case", name, "rows", g.rowptr.shape[0] - 1, "nnz", g.nnz)
    p = dict(DEFAULT, **over)
    assert_same_format(device_build(g.rowptr, g.col, g.val, p), host_build(g.rowptr, g.col, g.val, p), name)


@pytest.mark.parametrize("env", [{"LIBRA_SKIP_TC": "1"}, {"LIBRA_SPTC_UNIT_MIN_NNZ": "5"},
                                 {"LIBRA_SPTC_UNIT_MIN_NNZ": "0"}])
def test_device_builder_reads_the_reference_environment(env, golden_env):
    golden_env(env)
    g = graphs.rmat(scale=13, edge_factor=12, seed=9)
    say("case env", env)
    assert_same_format(device_build(g.rowptr, g.col, g.val, DEFAULT), host_build(g.rowptr, g.col, g.val, DEFAULT),
                       str(env))


def test_device_builder_empty_and_single_entry(golden_env):
    golden_env({})
    cases = [("no rows", [0], []), ("5 empty rows", [0] * 6, []), ("one entry", [0, 1], [7]),
             ("entry in row 16", [0] * 17 + [1], [3]), ("one row of 3", [0, 3], [0, 5, 9])]
    for what, rowptr, col in cases:
        rowptr = np.asarray(rowptr, np.int32)
        c = np.asarray(col, np.int32)
        v = np.linspace(0.25, 1.0, len(col), dtype=np.float32)
        say("case tiny", what)
        assert_same_format(device_build(rowptr, c, v, DEFAULT), host_build(rowptr, c, v, DEFAULT), what)


FULL = [
    ("config1_er4096", lambda: graphs.erdos_renyi_gcn()),
    ("config2_rmat20", lambda: graphs.rmat()),
    ("config3_sbm1m", lambda: graphs.sbm()),
    ("config5_gridhubs4m", lambda: graphs.grid_hubs()),
]


@pytest.mark.parametrize("name,gen", FULL, ids=[c[0] for c in FULL])
def test_device_builder_full_size(name, gen, golden_env):
    golden_env({})
    g = gen()
    say("case full", name, "nnz", g.nnz)
    df = device_build(g.rowptr, g.col, g.val, DEFAULT)
    say("  device build", round(df.elapsed, 4), "s")
    hf = host_build(g.rowptr, g.col, g.val, DEFAULT)
    assert_same_format(df, hf, name)


def random_structured(seed):
    """A seeded random matrix with dense rectangles (TC chunks and 2:4 groups of every fill) over
    a uniform background, in a random shape, with random builder parameters."""
    rng = np.random.default_rng(seed)
    window = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 11, 13, 16, 16, 16]))
    m, n = int(rng.integers(1, 3000)), int(rng.integers(1, 5000))
    keys = [rng.integers(0, m * n, size=int(rng.integers(0, 4 * m + 1)), dtype=np.int64)]
    for _ in range(int(rng.integers(0, 12))):
        r0, c0 = int(rng.integers(0, m)), int(rng.integers(0, n))
        h, w = int(rng.integers(1, 48)), int(rng.integers(1, 64))
        rr, cc = np.meshgrid(np.arange(r0, min(m, r0 + h)), np.arange(c0, min(n, c0 + w)), indexing="ij")
        keep = rng.random(rr.shape) < rng.uniform(0.3, 1.0)
        keys.append(rr[keep].astype(np.int64) * n + cc[keep])
    keys = np.unique(np.concatenate(keys))
    m_pad = graphs.pad_rows(m, window)
    rowptr, col = graphs.csr_from_keys(keys, m, n, m_pad)
    val = rng.uniform(-1, 1, col.shape[0]).astype(np.float16).astype(np.float32)
    p = dict(part_t=int(rng.integers(1, 40)), part_c=int(rng.integers(1, 40)), short_size=int(rng.integers(0, 6)),
             density=int(rng.integers(1, window + 2)), window=window,
             tc_min_util=float(rng.choice([0.0, 0.0, 0.3, 0.7])))
    return graphs.Graph(f"rs{seed}", m, n, rowptr, col, val), p


@pytest.mark.parametrize("seed", range(24))
def test_device_builder_random_structured(seed, golden_env):
    """Random shapes, windows of 1..16 rows and random builder parameters: all 32 slots equal the
    host builder's; for 16-row windows the plan from the device format equals the plan from its
    download (statistics and SpMM output bitwise)."""
    golden_env({})
    g, p = random_structured(seed)
    say("case random", seed, "m", g.m, "n", g.n, "nnz", g.nnz, p)
    df = device_build(g.rowptr, g.col, g.val, p)
    f = assert_same_format(df, host_build(g.rowptr, g.col, g.val, p), f"seed {seed}")
    if p["window"] == 16 and g.n > 0:
        pd, ph = trspmm.Plan.from_format(df, g.m, g.n), trspmm.Plan.from_format(f, g.m, g.n)
        assert pd.stats() == ph.stats()
        B = torch.from_numpy(graphs.dense_operand(g.n, 32, seed=seed)).cuda()
        assert torch.equal(pd.spmm(B), ph.spmm(B))
