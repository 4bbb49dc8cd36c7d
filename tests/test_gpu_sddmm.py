"""GPU parity of SDDMM (no reference counterpart; closed form out[e] = X[row_e] . Y[col_e])."""
import numpy as np
import pytest
import torch

from oracle import spmm as osp
from trspmm import _native as nat
from trspmm import graphs
import trspmm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("K", [1, 2, 3, 4, 6, 7, 8, 10, 12, 14, 16, 18, 24, 30, 32, 33, 36, 64, 65, 66, 82, 100, 128, 130, 256,
                               600])
def test_sddmm_matches_closed_form(K):
    print("sddmm K", K, flush=True)
    g = graphs.rmat(scale=12, edge_factor=16, seed=4)
    plan = trspmm.Plan.from_csr(g.rowptr, g.col, g.val.astype(np.float16), g.m, g.n)
    Xh = graphs.dense_operand(g.m, K, seed=4)
    Yh = graphs.dense_operand(g.n, K, seed=5)
    out = plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda())
    torch.cuda.synchronize()
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col, Xh, Yh)
    got = out.cpu().numpy()
    assert got.shape == R.shape
    # per-entry dot of K fp16 products, fp32 accumulation
    tol = 1e-5 * np.sqrt(K) * 4 + 1e-6
    assert np.max(np.abs(got - R)) <= tol * max(1.0, np.max(np.abs(R))), np.max(np.abs(got - R))


@pytest.mark.parametrize("K,pad", [(14, 2), (14, 1), (16, 1), (12, 2), (40, 2)])
def test_sddmm_strided_operands(K, pad):
    """X and Y as column slices of wider arrays (leading dimension K + pad): an even leading
    dimension keeps 4-byte loads (K = 9..16 and even widths not divisible by 4), an odd one falls
    back to 2-byte loads; both against the closed form."""
    print("sddmm strided", K, pad, flush=True)
    g = graphs.rmat(scale=11, edge_factor=8, seed=10)
    plan = trspmm.Plan.from_csr(g.rowptr, g.col, g.val.astype(np.float16), g.m, g.n)
    Xh = graphs.dense_operand(g.m, K, seed=21)
    Yh = graphs.dense_operand(g.n, K, seed=22)
    Xw = torch.zeros((g.m, K + pad), dtype=torch.float16, device="cuda")
    Yw = torch.zeros((g.n, K + pad), dtype=torch.float16, device="cuda")
    Xw[:, :K] = torch.from_numpy(Xh).cuda()
    Yw[:, :K] = torch.from_numpy(Yh).cuda()
    out = plan.sddmm(Xw[:, :K], Yw[:, :K])
    torch.cuda.synchronize()
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col, Xh, Yh)
    tol = (1e-5 * np.sqrt(K) * 4 + 1e-6) * max(1.0, np.max(np.abs(R)))
    assert np.max(np.abs(out.cpu().numpy() - R)) <= tol


@pytest.mark.parametrize("K", [8, 16, 32, 64])
def test_sddmm_long_rows_and_empty_rows(K):
    """A 30,000-entry row among empty and 4-entry ones: cut into pieces of 256 entries for 16-lane
    groups (K = 64) and of S entries for narrower groups (K <= 32, the narrow task list)."""
    rng = np.random.default_rng(1)
    m, n = 48, 50000
    degs = np.array([30000 if r == 5 else (0 if r % 3 == 0 else 4) for r in range(m)])
    cols = np.concatenate([np.sort(rng.choice(n, size=d, replace=False)) for d in degs]).astype(np.int32)
    rowptr = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
    plan = trspmm.Plan.from_csr(rowptr, cols, np.ones(len(cols), np.float16), m, n)
    Xh = graphs.dense_operand(m, K, seed=1)
    Yh = graphs.dense_operand(n, K, seed=2)
    out = plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda())
    torch.cuda.synchronize()
    R = osp.csr_sddmm(rowptr, cols, Xh, Yh)
    assert np.max(np.abs(out.cpu().numpy() - R)) < 1e-3


@pytest.mark.parametrize("K", [72, 128, 256])
def test_staged_and_unstaged_sddmm_agree(K):
    """16-lane groups (K = 65..128, and each 128-feature pass of K = 256) stage each task's column
    ids in LDS (16-byte chunks from an 8-entry-aligned base).  Tasks here start at every offset mod 8 and hold
    up to 256 entries (rows of 100-256 entries, split rows beyond): staged and unstaged
    (stage = -1) plans against the closed form, and bitwise equal to each other (same summation
    order)."""
    print("sddmm staged", K, flush=True)
    rng = np.random.default_rng(12)
    m, n = 3000, 20000
    degs = rng.integers(0, 40, size=m)
    degs[rng.choice(m, 50, replace=False)] = rng.integers(100, 257, size=50)
    degs[777] = 600
    cols = np.concatenate([np.sort(rng.choice(n, size=d, replace=False)) for d in degs]).astype(np.int32)
    rowptr = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
    vals = np.ones(len(cols), np.float16)
    Xh = graphs.dense_operand(m, K, seed=6)
    Yh = graphs.dense_operand(n, K, seed=7)
    X, Y = torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()
    staged = trspmm.Plan.from_csr(rowptr, cols, vals, m, n, task_nnz=128).sddmm(X, Y)
    plain = trspmm.Plan.from_csr(rowptr, cols, vals, m, n, task_nnz=128, stage=-1).sddmm(X, Y)
    torch.cuda.synchronize()
    R = osp.csr_sddmm(rowptr, cols, Xh, Yh)
    tol = (1e-5 * np.sqrt(K) * 4 + 1e-6) * max(1.0, np.max(np.abs(R)))
    got = staged.cpu().numpy()
    assert np.max(np.abs(got - R)) <= tol
    assert np.array_equal(got, plain.cpu().numpy())


@pytest.mark.parametrize("K", [4, 8, 16, 32, 72, 256])
def test_streaming_and_plain_sddmm_stores_agree(K):
    """Residual outputs go out with non-temporal stores where a lane group writes 8 consecutive
    sums (groups of >= 8 lanes), plain stores otherwise and when the plan asks (streaming = 0):
    bitwise equal, and on a hybrid plan whose residual outputs are scattered by res_pos."""
    print("sddmm streaming", K, flush=True)
    g = graphs.sbm(communities=512, seed=8, val_seed=9)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    nnz = int(g.rowptr[g.m])
    X = torch.from_numpy(graphs.dense_operand(g.m, K, seed=15)).cuda()
    Y = torch.from_numpy(graphs.dense_operand(g.n, K, seed=16)).cuda()
    outs = []
    for streaming in (None, 0):
        plan = trspmm.Plan.for_sddmm(f, g.m, g.n, streaming=streaming)
        out = torch.full((nnz,), float("nan"), device="cuda")
        plan.sddmm(X, Y, out=out)
        outs.append(out)
    torch.cuda.synchronize()
    a, b = (o.cpu().numpy() for o in outs)
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col[:nnz], X.cpu().numpy(), Y.cpu().numpy())
    assert not np.isnan(a).any()
    assert np.max(np.abs(a - R)) <= 1e-4 * np.sqrt(K) * max(1.0, np.abs(R).max())
    assert np.array_equal(a, b)


@pytest.mark.parametrize("K,lanes", [(128, 4), (64, 8), (40, 2)])
def test_sddmm_feature_lanes_option(K, lanes):
    """A plan may ask for fewer lanes per group than the width needs: each batch then loops over
    feature chunks (the X fragment is not carried across batches).  Against the closed form."""
    print("sddmm lanes", K, lanes, flush=True)
    g = graphs.rmat(scale=11, edge_factor=8, seed=13)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.for_sddmm(f, g.m, g.n, feature_lanes=lanes)
    Xh = graphs.dense_operand(g.m, K, seed=23)
    Yh = graphs.dense_operand(g.n, K, seed=24)
    out = plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda())
    torch.cuda.synchronize()
    nnz = int(g.rowptr[g.m])
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col[:nnz], Xh, Yh)
    got = out.cpu().numpy()
    assert np.max(np.abs(got - R)) <= 1e-4 * np.sqrt(K) * max(1.0, np.abs(R).max())


@pytest.mark.parametrize("K", [2, 4, 16, 32, 72, 128, 256])
def test_sddmm_four_entries_per_batch(K):
    """Plan option sddmm_unroll = 4: batches of 4 entries per lane group (4 sums per
    reduce-scatter, written with plain stores), on tasks with long and empty rows.  Against the
    closed form."""
    print("sddmm unroll4", K, flush=True)
    g = graphs.grid_hubs(side=64, hubs=2, hub_degree=2000, seed=3, val_seed=4)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.for_sddmm(f, g.m, g.n, sddmm_unroll=4)
    Xh = graphs.dense_operand(g.m, K, seed=25)
    Yh = graphs.dense_operand(g.n, K, seed=26)
    out = plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda())
    torch.cuda.synchronize()
    nnz = int(g.rowptr[g.m])
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col[:nnz], Xh, Yh)
    got = out.cpu().numpy()
    assert not np.isnan(got).any()
    assert np.max(np.abs(got - R)) <= 1e-4 * np.sqrt(K) * max(1.0, np.abs(R).max())


def test_sddmm_matches_torch_sampled_addmm():
    g = graphs.random_csr(200, 300, 0.05, seed=3)
    plan = trspmm.Plan.from_csr(g.rowptr[: g.m + 1], g.col, g.val.astype(np.float16), g.m, g.n)
    Xh = graphs.dense_operand(g.m, 48, seed=1)
    Yh = graphs.dense_operand(g.n, 48, seed=2)
    out = plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()).cpu().numpy()
    nnz = int(g.rowptr[g.m])
    A = torch.sparse_csr_tensor(torch.from_numpy(g.rowptr[: g.m + 1].astype(np.int64)),
                                torch.from_numpy(g.col[:nnz].astype(np.int64)), torch.ones(nnz), size=(g.m, g.n))
    ref = torch.sparse.sampled_addmm(A, torch.from_numpy(Xh).float(), torch.from_numpy(Yh).float().T, beta=0.0)
    assert np.allclose(out, ref.values().numpy(), atol=1e-4)


@pytest.mark.parametrize("name,gen,K", [
    ("sbm", lambda: graphs.sbm(communities=1024, seed=1, val_seed=2), 64),
    ("rmat", lambda: graphs.rmat(scale=13, edge_factor=16, seed=3), 128),
    ("er", lambda: graphs.erdos_renyi_gcn(nodes=2048, edges=16384), 40),
    ("gridhubs", lambda: graphs.grid_hubs(side=128, hubs=4, hub_degree=5000, seed=1, val_seed=2), 32),
])
@pytest.mark.parametrize("mfma", [True, False])
def test_hybrid_sddmm_matches_closed_form(name, gen, K, mfma):
    """SDDMM on the SpMM tiling: MFMA tiles + CSR dot products, outputs in input CSR order."""
    print("hybrid sddmm", name, K, mfma, flush=True)
    g = gen()
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.for_sddmm(f, g.m, g.n, mfma_tc=mfma, mfma_sptc=mfma, sptc_min_fill=0.1)
    st = plan.stats()
    nnz = int(g.rowptr[g.m])
    assert st["nnz"] == nnz
    if mfma and name == "sbm":
        assert st["mfma_tiles"] > 0 and st["mfma_nnz"] > 0
    Xh = graphs.dense_operand(g.m, K, seed=11)
    Yh = graphs.dense_operand(g.n, K, seed=12)
    out = torch.full((nnz,), float("nan"), device="cuda")
    plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda(), out=out)
    torch.cuda.synchronize()
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col[:nnz], Xh, Yh)
    got = out.cpu().numpy()
    assert not np.isnan(got).any()
    assert np.max(np.abs(got - R)) <= 1e-4 * np.sqrt(K) * max(1.0, np.abs(R).max())


@pytest.mark.parametrize("K", [8, 40, 128, 136, 264, 36, 6])
def test_sddmm_mfma_tiles_feature_widths(K):
    """Dense-tile SDDMM: K % 8 == 0 takes the 16x16x32 MFMA kernel (one 16-byte load per lane and
    32-feature step, up to 4 steps loaded ahead: K = 8 and 40 end inside a step, 136 and 264 run
    a second chunk); other widths the 16x16x16 kernel (8-byte loads for K % 4 == 0, guarded
    scalars otherwise).  Against the closed form, with most entries on tiles."""
    print("sddmm mfma K", K, flush=True)
    g = graphs.sbm(communities=512, seed=4, val_seed=5)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.for_sddmm(f, g.m, g.n)
    st = plan.stats()
    nnz = int(g.rowptr[g.m])
    assert st["mfma_tiles"] > 0 and st["mfma_nnz"] > nnz // 4
    Xh = graphs.dense_operand(g.m, K, seed=13)
    Yh = graphs.dense_operand(g.n, K, seed=14)
    out = torch.full((nnz,), float("nan"), device="cuda")
    plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda(), out=out)
    torch.cuda.synchronize()
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col[:nnz], Xh, Yh)
    got = out.cpu().numpy()
    assert not np.isnan(got).any()
    assert np.max(np.abs(got - R)) <= 1e-4 * np.sqrt(K) * max(1.0, np.abs(R).max())


def test_sddmm_zero_width_writes_zeros():
    g = graphs.random_csr(100, 90, 0.05, seed=6)
    plan = trspmm.Plan.from_csr(g.rowptr[: g.m + 1], g.col, g.val.astype(np.float16), g.m, g.n)
    X = torch.zeros(g.m, 0, dtype=torch.float16, device="cuda")
    Y = torch.zeros(g.n, 0, dtype=torch.float16, device="cuda")
    out = torch.full((g.nnz,), float("nan"), device="cuda")
    plan.sddmm(X, Y, out=out)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0


def test_sddmm_nonfinite_Y_reaches_only_entries_that_use_it():
    g = graphs.rmat(scale=11, edge_factor=8, seed=6)
    plan = trspmm.Plan.from_csr(g.rowptr[: g.m + 1], g.col, g.val.astype(np.float16), g.m, g.n)   # CSR dots only
    K = 64
    Xh = graphs.dense_operand(g.m, K, seed=1)
    Yh = graphs.dense_operand(g.n, K, seed=2)
    hub = int(np.argmax(np.bincount(g.col, minlength=g.n)))
    Yh[hub, 5] = np.float16(np.nan)
    out = plan.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()).cpu().numpy()
    assert np.array_equal(~np.isfinite(out), g.col[: g.nnz] == hub)


@pytest.mark.parametrize("K", [8, 16, 32])
def test_sddmm_narrow_task_list_equals_pieces_of_S(K):
    """Lane groups of <= 8 lanes (K <= 32) walk the plan's narrow task list, the unsplit layout in
    pieces of S entries: bitwise the outputs of a plan whose every piece is S entries long."""
    print("sddmm narrow list", K, flush=True)
    # large enough that S = 32 is not shrunk further (small matrices take pieces of 64 anyway)
    g = graphs.rmat(scale=15, edge_factor=16, seed=8)
    Xh = graphs.dense_operand(g.m, K, seed=3)
    Yh = graphs.dense_operand(g.n, K, seed=4)
    X, Y = torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    narrow = trspmm.Plan.for_sddmm(f, g.m, g.n, task_nnz=32)
    pieces = trspmm.Plan.for_sddmm(f, g.m, g.n, task_nnz=32, piece_nnz=32)
    assert int(g.rowptr[g.m]) // 32 >= 16384
    assert np.max(np.diff(g.rowptr[: g.m + 1])) > 256
    a, b = narrow.sddmm(X, Y), pieces.sddmm(X, Y)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col, Xh, Yh)
    assert np.max(np.abs(a.cpu().numpy() - R)) <= (1e-5 * np.sqrt(K) * 4 + 1e-6) * max(1.0, np.max(np.abs(R)))


def test_sddmm_xcd_column_split_is_bitwise_equal():
    """The XCD column split only reorders the residual tasks (pieces of long rows by column range);
    every output is the same dot product, bitwise."""
    print("sddmm xcd split", flush=True)
    g = graphs.rmat(scale=13, edge_factor=16, seed=8)
    Xh = graphs.dense_operand(g.m, 128, seed=3)
    Yh = graphs.dense_operand(g.n, 128, seed=4)
    X, Y = torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()
    outs = []
    for xs in (-1, 8, 64):
        plan = trspmm.Plan.from_csr(g.rowptr, g.col, g.val.astype(np.float16), g.m, g.n, xcd_split=xs)
        outs.append(plan.sddmm(X, Y))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col, Xh, Yh)
    assert np.max(np.abs(outs[1].cpu().numpy() - R)) <= (1e-5 * np.sqrt(128) * 4 + 1e-6) * max(1.0, np.max(np.abs(R)))


@pytest.mark.parametrize("K", [128, 136, 200, 256])
def test_sddmm_split_part_merged_equals_in_place(K):
    """From K = 128 an SDDMM call with a workspace writes its split part (XCD sub-rows of the long
    rows) into a buffer of its own and merges the split rows' outputs into place afterwards; the
    call without a workspace writes them in place.  Same dot products, same outputs bitwise, and
    against the closed form; both lowerings; feature passes (K > 128) accumulate in the buffer."""
    print("sddmm merge", K, flush=True)
    g = graphs.rmat(scale=16, edge_factor=16, seed=21)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    Xh = graphs.dense_operand(g.m, K, seed=70)
    Yh = graphs.dense_operand(g.n, K, seed=71)
    X, Y = torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col, Xh, Yh)
    first = None
    for host in (False, True):
        for hot in (None, -1):
            plan = trspmm.Plan.for_sddmm(f, g.m, g.n, host_lowering=host, hot_rows=hot)
            st = plan.stats()
            assert st["split_rows"] > 0, st
            need = plan.sddmm_workspace_bytes(K)
            assert need > 0   # the split part's output buffer (and the staged rows)
            merged = plan.sddmm(X, Y)
            inplace = torch.full((st["nnz"],), float("nan"), device="cuda")
            nat.check(nat.lib().trs_sddmm_f16(plan.handle, X.data_ptr(), K, Y.data_ptr(), K, K, inplace.data_ptr(),
                                              int(torch.cuda.current_stream().cuda_stream)), "trs_sddmm_f16")
            torch.cuda.synchronize()
            assert torch.equal(merged, inplace), (host, hot)
            if first is None:
                first = merged
                got = merged.cpu().numpy()
                tol = (1e-5 * np.sqrt(K) * 4 + 1e-6) * max(1.0, float(np.max(np.abs(R))))
                assert np.max(np.abs(got - R)) <= tol
            assert torch.equal(merged, first), (host, hot)
    # the plain-CSR plan (outputs in the given entry order) takes the same path
    plan = trspmm.Plan.from_csr(g.rowptr[: g.m + 1], g.col, g.val.astype(np.float16), g.m, g.n)
    assert plan.stats()["split_rows"] > 0
    assert torch.equal(plan.sddmm(X, Y), first)
