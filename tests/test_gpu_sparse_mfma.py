"""GPU: 2:4 tiles on gfx950's sparse MFMA (v_smfmac_f32_16x16x64_f16, plan option sptc_sparse).

The reference runs its packed 2:4 tiles on mma.sp (TR-source/SpMM/mGCNkernel_online.cu:812-933).
With sptc_sparse, an SpMM plan stores each 2:4 tile (every row at most 2 entries per group of 4
columns) compressed -- two fp16 values and two 2-bit column positions per row and group -- and runs
four tiles per sparse MFMA instruction.  Checked against the float64 CSR oracle at the SpMM
tolerance, and against the dense-tile plan over the same tiles (the same fp16 products, summed in
another order inside the MFMA: equal to fp32 rounding), for feature widths that take each staging
load width (16-, 8-, 4- and 2-byte) and 1 and 2 MFMA n-tiles per wave.
"""
import numpy as np
import pytest
import torch

from oracle import spmm as osp
from trspmm import graphs
import trspmm

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
    # 2,478 well-filled 4-group tiles holding a quarter of the entries
    ("rand02", lambda: graphs.random_csr(2048, 2048, 0.2, seed=5)),
    # TC blocks and 2:4 tiles side by side in the same windows
    ("sbm_pin03", lambda: graphs.sbm(communities=2048, p_in=0.3, seed=3, val_seed=3)),
]

_cache = {}


def graph(name, gen):
    if name not in _cache:
        g = gen()
        _cache[name] = (g, trspmm.build_format(g.rowptr, g.col, g.val))
    return _cache[name]


@pytest.mark.parametrize("K", [256, 128, 100, 64, 34, 33, 16])
@pytest.mark.parametrize("name,gen", GRAPHS, ids=[g[0] for g in GRAPHS])
def test_sparse_mfma_matches_oracle_and_dense_tiles(name, gen, K):
    say("sparse mfma", name, K)
    g, f = graph(name, gen)
    sparse = trspmm.Plan.from_format(f, g.m, g.n, sptc_sparse=True, window_row_cap=1 << 30)
    dense = trspmm.Plan.from_format(f, g.m, g.n, sptc_sparse=False, window_row_cap=1 << 30)
    ss, sd = sparse.stats(), dense.stats()
    assert ss["sparse_tiles"] > 100 and sd["sparse_tiles"] == 0, (ss, sd)
    assert ss["mfma_tiles"] == sd["mfma_tiles"] and ss["mfma_nnz"] == sd["mfma_nnz"]
    Bh = graphs.dense_operand(g.n, K, seed=41)
    Cs, Cd = run_plan(sparse, Bh), run_plan(dense, Bh)
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m)
    e = osp.spmm_error(Cs, R)
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e
    # same products, fp32 sums in another order
    assert np.max(np.abs(Cs - Cd)) <= 1e-5 * max(1.0, np.max(np.abs(Cd))), np.max(np.abs(Cs - Cd))
    say("  stats", ss)


def test_sparse_mfma_is_deterministic_and_lowering_independent():
    """Two calls give the same bits; the device- and host-lowered sparse plans agree bitwise."""
    g, f = graph("rand02", GRAPHS[0][1])
    Bh = graphs.dense_operand(g.n, 128, seed=42)
    dev = trspmm.Plan.from_format(f, g.m, g.n, sptc_sparse=True, window_row_cap=1 << 30)
    host = trspmm.Plan.from_format(f, g.m, g.n, sptc_sparse=True, window_row_cap=1 << 30, host_lowering=True)
    assert dev.stats()["device_lowered"] == 1 and host.stats()["device_lowered"] == 0
    C1 = run_plan(dev, Bh)
    assert np.array_equal(C1, run_plan(dev, Bh))
    assert np.array_equal(C1, run_plan(host, Bh))


def test_sparse_mfma_single_entry_groups():
    """Rows with one entry per 4-column group (a zero paired at another position) and groups with
    entries only in the last column: a hand-built 2:4 pattern through the CSR plan builder."""
    m = n = 64
    rows, cols = [], []
    for r in range(m):
        for gq in range(16):
            base = 4 * gq
            pick = [(r + gq) % 4] if (r + gq) % 3 else sorted({(r * 7 + gq) % 4, (r + 2 * gq + 1) % 4})
            for p in pick:
                rows.append(r)
                cols.append(base + p)
    rows, cols = np.array(rows), np.array(cols)
    o = np.lexsort((cols, rows))
    rows, cols = rows[o], cols[o]
    rowptr = np.zeros(m + 1, np.int32)
    np.add.at(rowptr, rows + 1, 1)
    rowptr = np.cumsum(rowptr).astype(np.int32)
    vals = np.random.default_rng(7).standard_normal(len(cols)).astype(np.float32)
    f = trspmm.build_format(rowptr, cols.astype(np.int32), vals)
    Bh = graphs.dense_operand(n, 64, seed=43)
    R = osp.csr_spmm(rowptr, cols.astype(np.int32), vals, Bh, m=m)
    for sp in (False, True):
        plan = trspmm.Plan.from_format(f, m, n, sptc_sparse=sp, window_row_cap=1 << 30, sptc_min_fill=0.0)
        C = run_plan(plan, Bh)
        e = osp.spmm_error(C, R)
        assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, (sp, plan.stats(), e)


@pytest.mark.parametrize("m", [2000, 2047])
def test_sparse_mfma_rows_past_m(m):
    """Windows that run past the last row (m not a multiple of 16): the tiles' rows >= m carry no
    entries, and no output row past m is written."""
    g = graphs.random_csr(m, 2048, 0.2, seed=9)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n, window_row_cap=1 << 30)
    s = plan.stats()
    assert s["sparse_tiles"] > 0, s
    Bh = graphs.dense_operand(g.n, 128, seed=44)
    B = torch.from_numpy(Bh).cuda()
    out = torch.full((g.m + 16, 128), float("nan"), device="cuda")
    plan.spmm(B, out=out[: g.m])
    torch.cuda.synchronize()
    C = out.cpu().numpy()
    assert np.isnan(C[g.m:]).all()
    e = osp.spmm_error(C[: g.m], osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m))
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e
