"""GPU: plans made from a device-resident format (trs_plan_create_dformat,
trs_plan_create_sddmm_dformat) without bringing the format to the host.

Such a plan must be the plan trs_plan_create(_sddmm) makes from the same format on the host --
the device builder's output downloaded, which is bit-exact with the host builder's (that equality
has its own tests): equal statistics, device lowering included, and bitwise equal SpMM / SDDMM
outputs, over the workload shapes the device lowering is tested on (tiles kept or demoted, 2:4
group tiles passing or failing the fill rule, split rows, no tiles, other row counts, windows of 8
rows), the same error for columns outside n, and the host lowering on request.  SpMM results are
also checked against the oracle's reading of the format's arrays (TC, residual and 2:4 shares plus
the spill list), which for windows of 16 rows is the input CSR itself; windows of 8 rows place TC
entries at the window id * 16 as the reference's t_window_row does, and are lowered on the host.
"""
import numpy as np
import pytest
import torch

from oracle import spmm as osp
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


def dev_tensors(g):
    return (torch.from_numpy(np.ascontiguousarray(g.rowptr, dtype=np.int32)).cuda(),
            torch.from_numpy(np.ascontiguousarray(g.col, dtype=np.int32)).cuda(),
            torch.from_numpy(np.ascontiguousarray(g.val, dtype=np.float32)).cuda())


GRAPHS = [
    ("er4096", lambda: graphs.erdos_renyi_gcn(), {}),
    ("rmat14", lambda: graphs.rmat(scale=14, edge_factor=16, seed=42), {}),
    ("sbm2k", lambda: graphs.sbm(communities=2048, seed=3, val_seed=3), {}),
    ("gridhubs", lambda: graphs.grid_hubs(side=256, hubs=8, hub_degree=20000, seed=6, val_seed=6), {}),
    ("rand", lambda: graphs.random_csr(1000, 3000, 0.01, seed=5), {}),
    ("w8", lambda: graphs.random_csr(600, 400, 0.05, seed=3, window=8), dict(window=8, density=3)),
]

_cache = {}


def formats(name, gen, bp):
    """(graph, device format, its download) -- the download is the host plan's input."""
    if name not in _cache:
        g = gen()
        df = trspmm.build_format_device(*dev_tensors(g), **bp)
        _cache[name] = (g, df, df.download())
    return _cache[name]


def run_spmm(plan, Bh):
    """Output prefilled with NaN: an element no kernel writes fails the comparison."""
    B = torch.from_numpy(Bh).cuda()
    out = torch.full((plan.stats()["m"], Bh.shape[1]), float("nan"), device="cuda")
    C = plan.spmm(B, out=out)
    torch.cuda.synchronize()
    return C.cpu().numpy()


def run_sddmm(plan, Xh, Yh):
    X, Y = torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()
    out = torch.full((plan.stats()["nnz"],), float("nan"), device="cuda")
    S = plan.sddmm(X, Y, out=out)
    torch.cuda.synchronize()
    return S.cpu().numpy()


def format_oracle(hf, g, Bh, m, window):
    """float64 SpMM of every entry the format's arrays carry, rows [0, m)."""
    arrs = hf.arrays()
    spill = (hf.slot(29), hf.slot(30), hf.slot(31))
    r, c, v = osp.format_to_coo(arrs, spill, window=window)
    return osp.coo_spmm(r, c, v, Bh, m)


def same_plans(pd, ph, what):
    sd, sh = pd.stats(), ph.stats()
    assert sd == sh, f"{what}: stats differ\n device format {sd}\n host format   {sh}"
    return sd


def compare_spmm(df, hf, m, n, K, opts, what, seed=41):
    pd = trspmm.Plan.from_format(df, m, n, **opts)
    ph = trspmm.Plan.from_format(hf, m, n, **opts)
    s = same_plans(pd, ph, what)
    Bh = graphs.dense_operand(n, K, seed=seed)
    Cd, Ch = run_spmm(pd, Bh), run_spmm(ph, Bh)
    assert np.array_equal(Cd, Ch), f"{what}: SpMM outputs differ"
    return Cd, Bh, s


def compare_sddmm(df, hf, m, n, K, opts, what, seed=43):
    pd = trspmm.Plan.for_sddmm(df, m, n, **opts)
    ph = trspmm.Plan.for_sddmm(hf, m, n, **opts)
    s = same_plans(pd, ph, what)
    Xh = graphs.dense_operand(m, K, seed=seed)
    Yh = graphs.dense_operand(n, K, seed=seed + 1)
    Sd, Sh = run_sddmm(pd, Xh, Yh), run_sddmm(ph, Xh, Yh)
    assert np.array_equal(Sd, Sh), f"{what}: SDDMM outputs differ"
    return Sd, s


OPTIONS = [
    ("default", {}),
    ("tiles_kept", {"window_row_cap": 1 << 30}),
    ("split16", {"xcd_split": 16, "window_row_cap": 1 << 30}),
    ("no_tiles", {"mfma_tc": False, "mfma_sptc": False}),
    ("no_group_tiles", {"mfma_sptc": False, "window_row_cap": 1 << 30}),
    ("all_group_tiles", {"sptc_min_fill": 0.0, "window_row_cap": 1 << 30}),
    ("full_group_tiles_only", {"sptc_min_fill": 0.9, "window_row_cap": 1 << 30}),
    ("dense_2to4", {"sptc_sparse": False, "window_row_cap": 1 << 30}),
]


@pytest.mark.parametrize("oname,opts", OPTIONS, ids=[o[0] for o in OPTIONS])
@pytest.mark.parametrize("name,gen,bp", GRAPHS, ids=[g[0] for g in GRAPHS])
def test_dformat_plan_equals_format_plan(name, gen, bp, oname, opts):
    say("dformat plan", name, oname)
    g, df, hf = formats(name, gen, bp)
    C, Bh, s = compare_spmm(df, hf, g.m, g.n, 64, opts, f"{name}/{oname}")
    window = bp.get("window", 16)
    assert s["device_lowered"] == (window == 16)
    R = format_oracle(hf, g, Bh, g.m, window)
    if window == 16:   # the same entries as the CSR (float64 sums in another order)
        assert np.allclose(R, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), rtol=1e-12, atol=1e-9)
    e = osp.spmm_error(C, R)
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, f"{name}/{oname}: {e}"
    say("  stats", s)


SDDMM_OPTIONS = [
    ("default", {}),
    ("split16", {"xcd_split": 16}),
    ("no_tiles", {"mfma_tc": False, "mfma_sptc": False}),
    ("all_group_tiles", {"sptc_min_fill": 0.0}),
]


@pytest.mark.parametrize("K", [64, 128])
@pytest.mark.parametrize("oname,opts", SDDMM_OPTIONS, ids=[o[0] for o in SDDMM_OPTIONS])
@pytest.mark.parametrize("name,gen,bp", GRAPHS, ids=[g[0] for g in GRAPHS])
def test_dformat_sddmm_plan_equals_format_plan(name, gen, bp, oname, opts, K):
    say("dformat sddmm plan", name, oname, K)
    g, df, hf = formats(name, gen, bp)
    S, s = compare_sddmm(df, hf, g.m, g.n, K, opts, f"{name}/{oname}/K{K}")
    assert s["device_lowered"] == (bp.get("window", 16) == 16)


def test_dformat_plans_reach_tiles_groups_and_split_rows():
    """The cases above include plans with TC and 2:4 group tiles and with split rows."""
    g, df, hf = formats(*GRAPHS[2])
    s_all = trspmm.Plan.from_format(df, g.m, g.n, sptc_min_fill=0.0, window_row_cap=1 << 30).stats()
    s_tc = trspmm.Plan.from_format(df, g.m, g.n, mfma_sptc=False, window_row_cap=1 << 30).stats()
    assert s_tc["mfma_tiles"] > 0 and s_all["mfma_tiles"] > s_tc["mfma_tiles"]
    g, df, hf = formats(*GRAPHS[1])
    s = trspmm.Plan.from_format(df, g.m, g.n, xcd_split=16, window_row_cap=1 << 30).stats()
    assert s["split_rows"] > 0 and s["mfma_tiles"] > 0


@pytest.mark.parametrize("extra", [-100, -7, 5])
def test_dformat_plan_with_other_row_counts(extra):
    """m below the input's rows drops the rows beyond it (whole windows of tiles past m for -100);
    m above adds empty rows."""
    g, df, hf = formats(*GRAPHS[2])
    m = g.m + extra
    say("dformat plan m =", m)
    C, Bh, s = compare_spmm(df, hf, m, g.n, 32, {"window_row_cap": 1 << 30}, f"m={m}")
    assert s["device_lowered"] == 1
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=min(m, g.m))
    assert not C[g.m:].any()
    e = osp.spmm_error(C[: min(m, g.m)], R[: min(m, g.m)])
    assert e["elementwise_ok"], e
    compare_sddmm(df, hf, m, g.n, 64, {}, f"sddmm m={m}")


def test_dformat_plan_rejects_columns_outside_n():
    """Columns >= n: TRS_ERANGE with the message of the host format's plan."""
    g, df, hf = formats(*GRAPHS[4])
    for sddmm in (False, True):
        make = trspmm.Plan.for_sddmm if sddmm else trspmm.Plan.from_format
        with pytest.raises(nat.TrsError) as ed:
            make(df, g.m, g.n - 1)
        with pytest.raises(nat.TrsError) as eh:
            make(hf, g.m, g.n - 1)
        assert ed.value.code == eh.value.code == 5
        assert str(ed.value).split(":")[-1] == str(eh.value).split(":")[-1]


def test_dformat_plan_host_lowering_on_request():
    g, df, hf = formats(*GRAPHS[1])
    pd = trspmm.Plan.from_format(df, g.m, g.n, host_lowering=True)
    ph = trspmm.Plan.from_format(hf, g.m, g.n, host_lowering=True)
    s = same_plans(pd, ph, "host lowering")
    assert s["device_lowered"] == 0
    Bh = graphs.dense_operand(g.n, 32, seed=44)
    assert np.array_equal(run_spmm(pd, Bh), run_spmm(trspmm.Plan.from_format(df, g.m, g.n), Bh))


def test_dformat_plan_empty_and_tiny():
    cases = [
        (np.zeros(17, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32), 16, 8),
        (np.array([0, 1], np.int32), np.array([3], np.int32), np.array([2.5], np.float32), 1, 4),
        (np.array([0, 0, 2, 2], np.int32), np.array([0, 5], np.int32), np.array([1.0, -1.0], np.float32), 3, 6),
    ]
    for rowptr, col, val, m, n in cases:
        g = graphs.Graph("tiny", len(rowptr) - 1, n, rowptr, col, val)
        df = trspmm.build_format_device(*dev_tensors(g))
        hf = df.download()
        say("dformat tiny", m, len(col))
        compare_spmm(df, hf, m, n, 16, {}, f"m={m} nnz={len(col)}")
        compare_sddmm(df, hf, m, n, 16, {}, f"sddmm m={m} nnz={len(col)}")


def test_dformat_plan_full_size_rmat():
    """Configuration 2 at its full size (R-MAT 2^20): equal plans, bitwise equal SpMM at K = 128
    and SDDMM at K = 128."""
    g = graphs.rmat()
    say("dformat plan full size, nnz", g.nnz)
    df = trspmm.build_format_device(*dev_tensors(g))
    hf = df.download()
    compare_spmm(df, hf, g.m, g.n, 128, {}, "rmat20 spmm")
    compare_sddmm(df, hf, g.m, g.n, 128, {}, "rmat20 sddmm")


def test_dformat_plan_outlives_its_format():
    """A plan keeps nothing of the device format it was made from: freed format, same outputs."""
    g = graphs.sbm(communities=512, seed=8, val_seed=9)
    df = trspmm.build_format_device(*dev_tensors(g))
    keep = trspmm.Plan.from_format(df.download(), g.m, g.n)
    plan = trspmm.Plan.from_format(df, g.m, g.n)
    splan = trspmm.Plan.for_sddmm(df, g.m, g.n)
    del df
    torch.cuda.synchronize()
    Bh = graphs.dense_operand(g.n, 64, seed=3)
    assert np.array_equal(run_spmm(plan, Bh), run_spmm(keep, Bh))
    Xh, Yh = graphs.dense_operand(g.m, 64, seed=4), graphs.dense_operand(g.n, 64, seed=5)
    S = run_sddmm(splan, Xh, Yh)
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col[: int(g.rowptr[g.m])], Xh, Yh)
    assert np.max(np.abs(S - R)) <= (1e-5 * np.sqrt(64) * 4 + 1e-6) * max(1.0, float(np.max(np.abs(R))))
