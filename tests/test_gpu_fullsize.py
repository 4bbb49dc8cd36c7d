"""GPU parity at the BASELINE.json sizes, through size-independent properties:

* checksum: 1^T C == (1^T A) B, with the column sums of A and the product formed in float64 on the
  CPU (O(nnz + n K)) -- a dropped, duplicated or misplaced entry anywhere changes it;
* sampled rows (random rows plus the heaviest rows, which exercise split rows and MFMA windows)
  against the float64 oracle with the parity tolerance;
* linearity C(B1 + B2) == C(B1) + C(B2) up to fp32 rounding; bitwise determinism across calls;
* SDDMM: sampled entries against the closed form.
"""
import numpy as np
import pytest
import torch

from oracle import spmm as osp
from trspmm import graphs
import trspmm

pytestmark = pytest.mark.gpu

_cache = {}


def graph(name):
    if name not in _cache:
        _cache.clear()
        gen = {"rmat20": graphs.rmat, "sbm1m": graphs.sbm, "grid_hubs": graphs.grid_hubs}[name]
        g = gen()
        _cache[name] = (g, trspmm.build_format(g.rowptr, g.col, g.val))
    return _cache[name]


def sample_rows(g, count, seed):
    rng = np.random.default_rng(seed)
    deg = np.diff(g.rowptr[: g.m + 1])
    heavy = np.argsort(deg)[-min(64, g.m):]
    return np.unique(np.concatenate([rng.choice(g.m, size=count, replace=False), heavy]))


def rows_reference(g, rows, B64):
    out = np.zeros((len(rows), B64.shape[1]))
    for i, r in enumerate(rows):
        s, e = g.rowptr[r], g.rowptr[r + 1]
        out[i] = g.val[s:e].astype(np.float64) @ B64[g.col[s:e]]
    return out


# every BASELINE width on R-MAT (K = 256: two feature passes, 8 MB of staged rows), the two ends on
# SBM (MFMA windows of 32 and 128 features), grid+hubs at its headline width and at K = 128;
# grouped by graph so that each graph is generated once
@pytest.mark.parametrize("name,K", [("rmat20", 32), ("rmat20", 64), ("rmat20", 128), ("rmat20", 256),
                                    ("sbm1m", 32), ("sbm1m", 256), ("grid_hubs", 32), ("grid_hubs", 128)])
def test_fullsize_spmm_properties(name, K):
    print("fullsize", name, K, flush=True)
    g, f = graph(name)
    plan = trspmm.Plan.from_format(f, g.m, g.n)
    st = plan.stats()
    assert st["nnz"] == g.nnz
    Bh = graphs.dense_operand(g.n, K, seed=2)
    B = torch.from_numpy(Bh).cuda()
    C = torch.full((g.m, K), float("nan"), device="cuda")
    plan.spmm(B, out=C)
    torch.cuda.synchronize()
    assert not torch.isnan(C).any()
    B64 = Bh.astype(np.float64)

    # checksum 1^T C == (1^T A) B
    colsum = np.bincount(g.col, weights=g.val.astype(np.float64), minlength=g.n)
    expect = colsum @ B64
    got = C.double().sum(0).cpu().numpy()
    scale = np.abs(colsum) @ np.abs(B64)
    assert np.max(np.abs(got - expect) / scale) < 1e-5

    # sampled rows against the float64 oracle
    rows = sample_rows(g, 3000, seed=7)
    R = rows_reference(g, rows, B64)
    e = osp.spmm_error(C[torch.from_numpy(rows).cuda()].cpu().numpy(), R)
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e

    # linearity and determinism
    B2 = torch.from_numpy(graphs.dense_operand(g.n, K, seed=3)).cuda()
    C2 = plan.spmm(B2)
    C12 = plan.spmm((B.float() + B2.float()).half())
    Cagain = plan.spmm(B)
    torch.cuda.synchronize()
    assert torch.equal(Cagain, C)
    lin = (C12 - (C + C2)).abs().max().item()
    # B1 + B2 is rounded to fp16 once: bound by that rounding times the row sums of |A|
    rows_all = np.repeat(np.arange(g.m_pad), np.diff(g.rowptr))
    rowabs = np.bincount(rows_all, weights=np.abs(g.val.astype(np.float64)), minlength=g.m_pad).max()
    assert lin <= 2 * 2.0 ** -10 * rowabs + 1e-3


@pytest.mark.parametrize("K", [32, 64, 128, 256])
def test_fullsize_sddmm_sampled(K):
    print("fullsize sddmm", K, flush=True)
    g, f = graph("rmat20")
    plan = trspmm.Plan.for_sddmm(f, g.m, g.n)
    Xh = graphs.dense_operand(g.m, K, seed=4)
    Yh = graphs.dense_operand(g.n, K, seed=5)
    out = torch.full((g.nnz,), float("nan"), device="cuda")
    plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda(), out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert not np.isnan(got).any()
    rng = np.random.default_rng(1)
    idx = rng.choice(g.nnz, size=200_000, replace=False)
    rows = np.searchsorted(g.rowptr, idx, side="right") - 1
    ref = np.einsum("ij,ij->i", Xh[rows].astype(np.float64), Yh[g.col[idx]].astype(np.float64))
    assert np.max(np.abs(got[idx] - ref)) <= 1e-4 * np.sqrt(K)
    # total over all entries against sum_rows X[r] . (sum of Y over the row's columns)
    import scipy.sparse as sp
    pattern = sp.csr_matrix((np.ones(g.nnz), g.col, g.rowptr), shape=(g.m_pad, g.n))[: g.m]
    Ysum = pattern @ Yh.astype(np.float64)
    total = float(np.sum(Xh.astype(np.float64) * Ysum))
    assert abs(float(got.astype(np.float64).sum()) - total) <= 1e-7 * g.nnz * np.sqrt(K)


@pytest.mark.parametrize("name,K", [("rmat20", 128), ("sbm1m", 256)])
def test_fullsize_device_lowering_equals_host_lowering(name, K):
    """BASELINE configs 2 and 3 at full size: the plan whose residual is built on the device and
    the host-lowered plan have the same statistics and give bitwise equal SpMM and SDDMM outputs
    (compared on the device)."""
    print("fullsize lowering", name, K, flush=True)
    g, f = graph(name)
    dev = trspmm.Plan.from_format(f, g.m, g.n)
    host = trspmm.Plan.from_format(f, g.m, g.n, host_lowering=True)
    sd, sh = dev.stats(), host.stats()
    assert sd.pop("device_lowered") == 1 and sh.pop("device_lowered") == 0
    assert sd == sh, (sd, sh)
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=2)).cuda()
    Cd = dev.spmm(B)
    Ch = host.spmm(B)
    torch.cuda.synchronize()
    assert torch.equal(Cd, Ch)
    del Cd, Ch, dev, host
    sdev = trspmm.Plan.for_sddmm(f, g.m, g.n)
    shost = trspmm.Plan.for_sddmm(f, g.m, g.n, host_lowering=True)
    sd, sh = sdev.stats(), shost.stats()
    assert sd.pop("device_lowered") == 1 and sh.pop("device_lowered") == 0
    assert sd == sh, (sd, sh)
    X = torch.from_numpy(graphs.dense_operand(g.m, 128, seed=4)).cuda()
    Y = torch.from_numpy(graphs.dense_operand(g.n, 128, seed=5)).cuda()
    assert torch.equal(sdev.sddmm(X, Y), shost.sddmm(X, Y))


def test_fullsize_staged_hot_rows_equal_unstaged():
    """BASELINE config 2 (and 4 at K = 128): the plans stage 32,768 hot B (Y) rows by default; the
    outputs are bitwise those of the same plans with staging off."""
    print("fullsize staged rows", flush=True)
    g, f = graph("rmat20")
    K = 128
    hot = trspmm.Plan.from_format(f, g.m, g.n)
    plain = trspmm.Plan.from_format(f, g.m, g.n, hot_rows=-1)
    assert hot.stats()["hot_rows"] == 32768 and plain.stats()["hot_rows"] == 0
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=2)).cuda()
    assert torch.equal(hot.spmm(B), plain.spmm(B))
    del hot, plain
    sh = trspmm.Plan.for_sddmm(f, g.m, g.n)
    sp = trspmm.Plan.for_sddmm(f, g.m, g.n, hot_rows=-1)
    assert sh.stats()["hot_rows"] == 32768
    X = torch.from_numpy(graphs.dense_operand(g.m, K, seed=4)).cuda()
    assert torch.equal(sh.sddmm(X, B), sp.sddmm(X, B))
