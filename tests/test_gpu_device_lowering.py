"""GPU: SpMM and SDDMM plans whose residual is built on the device from the format's input CSR.

trs_plan_create / trs_plan_create_sddmm lower on the device when the format holds its input CSR
(a format built in this process from canonical input): the MFMA tiles are cut from the format
arrays on the host, the residual -- the input rows minus the kept tiles' entries, XCD sub-rows
included, with the SDDMM output index of every entry -- is written by two kernels.  The plan must
be the host lowering's: equal statistics and bitwise equal SpMM / SDDMM outputs, on every
workload shape the host lowering is tested on (tiles kept or demoted, split rows, no tiles at all,
more or fewer plan rows than input rows), and within the tolerance of the float64 CSR oracle.
"""
import numpy as np
import pytest
import torch

from oracle import spmm as osp
from trspmm import graphs
import trspmm
from trspmm import _native as nat

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.cuda.init()


def run_plan(plan, Bh):
    """Output prefilled with NaN: an element no kernel writes fails the comparison."""
    B = torch.from_numpy(Bh).cuda()
    out = torch.full((plan.stats()["m"], Bh.shape[1]), float("nan"), device="cuda")
    C = plan.spmm(B, out=out)
    torch.cuda.synchronize()
    return C.cpu().numpy()


GRAPHS = [
    ("er4096", lambda: graphs.erdos_renyi_gcn()),
    ("rmat14", lambda: graphs.rmat(scale=14, edge_factor=16, seed=42)),
    ("sbm2k", lambda: graphs.sbm(communities=2048, seed=3, val_seed=3)),
    ("gridhubs", lambda: graphs.grid_hubs(side=256, hubs=8, hub_degree=20000, seed=6, val_seed=6)),
    ("rand", lambda: graphs.random_csr(1000, 3000, 0.01, seed=5)),
]

OPTIONS = [
    ("default", {}),
    ("tiles_kept", {"window_row_cap": 1 << 30}),
    ("split16", {"xcd_split": 16, "window_row_cap": 1 << 30}),
    ("no_tiles", {"mfma_tc": False, "mfma_sptc": False}),
    ("no_split", {"xcd_split": -1}),
]

_cache = {}


def graph(name, gen):
    if name not in _cache:
        g = gen()
        _cache[name] = (g, trspmm.build_format(g.rowptr, g.col, g.val))
    return _cache[name]


def run_sddmm(plan, Xh, Yh):
    """Output prefilled with NaN: an entry no kernel writes fails the comparison."""
    X, Y = torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()
    out = torch.full((plan.stats()["nnz"],), float("nan"), device="cuda")
    S = plan.sddmm(X, Y, out=out)
    torch.cuda.synchronize()
    return S.cpu().numpy()


def compare_sddmm(f, m, n, K, opts, what, seed=31):
    dev = trspmm.Plan.for_sddmm(f, m, n, **opts)
    host = trspmm.Plan.for_sddmm(f, m, n, host_lowering=True, **opts)
    sd, sh = dev.stats(), host.stats()
    assert sd["device_lowered"] == 1 and sh["device_lowered"] == 0, what
    sd.pop("device_lowered")
    sh.pop("device_lowered")
    assert sd == sh, f"{what}: SDDMM stats differ\n device {sd}\n host   {sh}"
    Xh = graphs.dense_operand(m, K, seed=seed)
    Yh = graphs.dense_operand(n, K, seed=seed + 1)
    Sd, Sh = run_sddmm(dev, Xh, Yh), run_sddmm(host, Xh, Yh)
    assert np.array_equal(Sd, Sh), f"{what}: SDDMM outputs differ"
    return Sd, Xh, Yh, sd


def compare(f, m, n, Bh, opts, what):
    dev = trspmm.Plan.from_format(f, m, n, **opts)
    host = trspmm.Plan.from_format(f, m, n, host_lowering=True, **opts)
    sd, sh = dev.stats(), host.stats()
    assert sd["device_lowered"] == 1 and sh["device_lowered"] == 0, what
    sd.pop("device_lowered")
    sh.pop("device_lowered")
    assert sd == sh, f"{what}: stats differ\n device {sd}\n host   {sh}"
    Cd, Ch = run_plan(dev, Bh), run_plan(host, Bh)
    assert np.array_equal(Cd, Ch), f"{what}: outputs differ (max |d| {np.nanmax(np.abs(Cd - Ch))})"
    return Cd, sd


@pytest.mark.parametrize("oname,opts", OPTIONS, ids=[o[0] for o in OPTIONS])
@pytest.mark.parametrize("name,gen", GRAPHS, ids=[g[0] for g in GRAPHS])
def test_device_lowering_equals_host_lowering(name, gen, oname, opts):
    say("device lowering", name, oname)
    g, f = graph(name, gen)
    Bh = graphs.dense_operand(g.n, 64, seed=21)
    C, s = compare(f, g.m, g.n, Bh, opts, f"{name}/{oname}")
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m)
    e = osp.spmm_error(C, R)
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, f"{name}/{oname}: {e}"
    say("  stats", s)


SDDMM_OPTIONS = [
    ("default", {}),
    ("split16", {"xcd_split": 16}),
    ("no_tiles", {"mfma_tc": False, "mfma_sptc": False}),
    ("no_split", {"xcd_split": -1}),
]


@pytest.mark.parametrize("oname,opts", SDDMM_OPTIONS, ids=[o[0] for o in SDDMM_OPTIONS])
@pytest.mark.parametrize("name,gen", GRAPHS, ids=[g[0] for g in GRAPHS])
@pytest.mark.parametrize("K", [64, 128, 256])
def test_device_lowering_equals_host_lowering_sddmm(name, gen, oname, opts, K):
    """K = 128 takes the split part of the SDDMM launcher, K = 64 the unsplit task list, K = 256
    two 128-feature passes, the second adding to the outputs (tile and split-part output indices
    included)."""
    say("device lowering sddmm", name, oname, K)
    g, f = graph(name, gen)
    S, Xh, Yh, s = compare_sddmm(f, g.m, g.n, K, opts, f"{name}/{oname}/K{K}")
    nnz = int(g.rowptr[g.m])
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col[:nnz], Xh, Yh)
    # fp16 products accumulated in fp32 (the SDDMM tolerance of the other SDDMM parity tests)
    tol = (1e-5 * np.sqrt(K) * 4 + 1e-6) * max(1.0, np.max(np.abs(R)))
    assert S.shape == R.shape and np.max(np.abs(S - R)) <= tol, f"{name}/{oname}: {np.max(np.abs(S - R))}"
    say("  stats", s)


def test_device_lowering_exercises_tiles_and_split_rows():
    """The option sets above reach both device kernels' branches: kept tiles whose entries are
    flagged out of their rows, and split rows scattered into XCD sub-rows."""
    g, f = graph("sbm2k", GRAPHS[2][1])
    s = trspmm.Plan.from_format(f, g.m, g.n, window_row_cap=1 << 30).stats()
    assert s["device_lowered"] == 1 and s["mfma_tiles"] > 0 and s["mfma_nnz"] > 0
    s = trspmm.Plan.for_sddmm(f, g.m, g.n).stats()
    assert s["device_lowered"] == 1 and s["mfma_tiles"] > 0
    g, f = graph("rmat14", GRAPHS[1][1])
    s = trspmm.Plan.from_format(f, g.m, g.n, xcd_split=16, window_row_cap=1 << 30).stats()
    assert s["device_lowered"] == 1 and s["split_rows"] > 0 and s["mfma_tiles"] > 0
    # SDDMM splits only without tiles; its sub-rows show as extra tasks
    s1 = trspmm.Plan.for_sddmm(f, g.m, g.n, xcd_split=16, mfma_tc=False, mfma_sptc=False).stats()
    s0 = trspmm.Plan.for_sddmm(f, g.m, g.n, xcd_split=-1, mfma_tc=False, mfma_sptc=False).stats()
    assert s1["device_lowered"] == 1 and s1["mfma_tiles"] == 0 and s1["tasks"] > s0["tasks"]


@pytest.mark.parametrize("extra", [-100, -7, 5])
def test_device_lowering_with_other_row_counts(extra):
    """m below the input's rows drops the rows beyond it (-100: whole windows of tiles past m,
    which the plan leaves out); m above adds empty rows."""
    g, f = graph("sbm2k", GRAPHS[2][1])
    m = g.m + extra
    say("device lowering m =", m)
    Bh = graphs.dense_operand(g.n, 32, seed=22)
    C, _ = compare(f, m, g.n, Bh, {"window_row_cap": 1 << 30}, f"m={m}")
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=min(m, g.m))
    assert np.array_equal(C[g.m:], np.zeros_like(C[g.m:]))
    e = osp.spmm_error(C[: min(m, g.m)], R[: min(m, g.m)])
    assert e["elementwise_ok"], e
    compare_sddmm(f, m, g.n, 64, {}, f"sddmm m={m}")


def test_device_lowering_rejects_columns_outside_n():
    """Columns >= n: the same TRS_ERANGE as the host lowering, before any device work."""
    g, f = graph("rand", GRAPHS[4][1])
    for host in (False, True):
        with pytest.raises(nat.TrsError) as ei:
            trspmm.Plan.from_format(f, g.m, g.n - 1, host_lowering=host)
        assert ei.value.code == 5


def test_format_read_back_lowers_on_host(tmp_path):
    """A format written and read back has no input CSR: its plan is lowered on the host."""
    g, f = graph("er4096", GRAPHS[0][1])
    p = str(tmp_path / "er.trsf")
    f.save(p)
    f2 = trspmm.Format.load(p)
    s = trspmm.Plan.from_format(f2, g.m, g.n).stats()
    assert s["device_lowered"] == 0
    Bh = graphs.dense_operand(g.n, 64, seed=23)
    assert np.array_equal(run_plan(trspmm.Plan.from_format(f2, g.m, g.n), Bh),
                          run_plan(trspmm.Plan.from_format(f, g.m, g.n), Bh))


def test_device_lowering_empty_and_tiny_graphs():
    """No entries at all, one row, one entry: the device path handles every empty case the host
    path does (same statistics, same outputs)."""
    cases = [
        (np.zeros(17, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32), 16, 8),
        (np.array([0, 1], np.int32), np.array([3], np.int32), np.array([2.5], np.float32), 1, 4),
        (np.array([0, 0, 2, 2], np.int32), np.array([0, 5], np.int32), np.array([1.0, -1.0], np.float32), 3, 6),
    ]
    for rowptr, col, val, m, n in cases:
        f = trspmm.build_format(rowptr, col, val)
        Bh = graphs.dense_operand(n, 16, seed=24)
        C, _ = compare(f, m, n, Bh, {}, f"m={m} nnz={len(col)}")
        R = osp.csr_spmm(rowptr, col, val, Bh, m=m)
        assert np.array_equal(np.isnan(C), np.zeros_like(C, bool))
        e = osp.spmm_error(C, R)
        assert e["elementwise_ok"], e
        compare_sddmm(f, m, n, 16, {}, f"sddmm m={m} nnz={len(col)}")
