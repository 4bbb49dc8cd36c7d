"""GPU parity: hybrid fp16 SpMM through libtrspmm.so against the float64 CSR oracle.

Tolerance (fp16 inputs, fp32 accumulation): elementwise
|C - R| <= 1e-2 |R| + 1e-3 max|R|, and max|C - R| / max|R| <= 1e-2 (oracle.spmm.spmm_error).
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


def dense_B(n, K, seed):
    return graphs.dense_operand(n, K, seed)


def check(C, R, what):
    e = osp.spmm_error(C, R)
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, f"{what}: {e}"
    return e


def run_plan(plan, Bh, **kw):
    """Output prefilled with NaN: an element no kernel writes fails the comparison."""
    B = torch.from_numpy(Bh).cuda()
    if "out" not in kw:
        kw["out"] = torch.full((plan.stats()["m"], Bh.shape[1]), float("nan"), device="cuda")
    C = plan.spmm(B, **kw)
    torch.cuda.synchronize()
    return C.cpu().numpy()


GRAPHS = [
    ("er4096", lambda: graphs.erdos_renyi_gcn()),
    ("rmat14", lambda: graphs.rmat(scale=14, edge_factor=16, seed=42)),
    ("sbm2k", lambda: graphs.sbm(communities=2048, seed=3, val_seed=3)),
    ("gridhubs", lambda: graphs.grid_hubs(side=256, hubs=8, hub_degree=20000, seed=6, val_seed=6)),
    ("rand", lambda: graphs.random_csr(1000, 3000, 0.01, seed=5)),
]


@pytest.mark.parametrize("name,gen", GRAPHS, ids=[g[0] for g in GRAPHS])
@pytest.mark.parametrize("K", [64, 128])
def test_hybrid_spmm_matches_csr(name, gen, K):
    say("case", name, K)
    g = gen()
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n)
    Bh = dense_B(g.n, K, seed=K)
    C = run_plan(plan, Bh)
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh.astype(np.float64), m=g.m)
    e = check(C, R, name)
    say(name, K, plan.stats(), e)


@pytest.mark.parametrize("mfma_tc,mfma_sptc,fill", [(1, 1, 0.25), (0, 0, 1.0), (1, 1, 0.0), (1, 0, 1.0)])
def test_mfma_and_residual_routes_agree(mfma_tc, mfma_sptc, fill):
    say("routes", mfma_tc, mfma_sptc, fill)
    g = graphs.sbm(communities=1024, seed=11, val_seed=12)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n, mfma_tc=bool(mfma_tc), mfma_sptc=bool(mfma_sptc), sptc_min_fill=fill)
    st = plan.stats()
    if mfma_tc:
        assert st["mfma_tiles"] > 0 and st["mfma_nnz"] > 0
    else:
        assert st["mfma_tiles"] == 0
    assert st["nnz"] == g.nnz
    Bh = dense_B(g.n, 96, seed=5)
    C = run_plan(plan, Bh)
    check(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), "routes")


@pytest.mark.parametrize("K", [1, 2, 3, 4, 6, 8, 10, 12, 14, 16, 18, 20, 24, 30, 33, 36, 40, 65, 66, 81, 97, 98, 100,
                               130, 200, 256, 260, 520, 1030])
def test_feature_widths(K):
    say("K", K)
    g = graphs.sbm(communities=128, seed=1, val_seed=2)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n, sptc_min_fill=0.1)
    Bh = dense_B(g.n, K, seed=K)
    C = run_plan(plan, Bh)
    check(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), f"K={K}")


def test_strided_operands_and_output():
    g = graphs.random_csr(300, 500, 0.02, seed=9)
    plan = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    Bfull = torch.from_numpy(dense_B(g.n, 96, seed=1)).cuda()
    B = Bfull[:, 8:72]                       # ldb 96, K 64
    out_full = torch.full((g.m, 80), 7.0, device="cuda")
    out = out_full[:, 4:68]
    plan.spmm(B, out=out)
    torch.cuda.synchronize()
    R = osp.csr_spmm(g.rowptr, g.col, g.val, B.cpu().numpy(), m=g.m)
    check(out.cpu().numpy(), R, "strided")
    assert torch.all(out_full[:, :4] == 7.0) and torch.all(out_full[:, 68:] == 7.0)


@pytest.mark.parametrize("K,off,vec", [(100, 4, 4), (36, 4, 4), (132, 4, 4), (98, 4, 2), (18, 4, 2),
                                       (66, 4, 2), (100, 2, 2), (98, 1, 1)])
def test_narrow_load_paths_long_rows_and_offsets(K, off, vec):
    """B as a view starting `off` halves into its buffer: K % 4 == 0 with rows 8-byte aligned takes
    8-byte loads, even K with rows 4-byte aligned 4-byte loads, the rest 2-byte loads (`vec`
    features per load).  Split rows and their fixups, and the MFMA window kernel."""
    say("vec", K, off, vec)
    g = graphs.rmat(scale=12, edge_factor=16, seed=12)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n, piece_nnz=64)
    assert plan.stats()["split_rows"] > 0
    Bfull = torch.from_numpy(dense_B(g.n + 1, K, seed=K).reshape(-1)[: (g.n + 1) * K]).cuda()
    B = Bfull[off: off + g.n * K].view(g.n, K)
    assert B.data_ptr() % 16 == 2 * off
    C = plan.spmm(B)
    torch.cuda.synchronize()
    check(C.cpu().numpy(), osp.csr_spmm(g.rowptr, g.col, g.val, B.cpu().numpy(), m=g.m), f"K={K}")
    s = graphs.sbm(communities=128, seed=5, val_seed=6)
    sp = trspmm.Plan.from_format(trspmm.build_format(s.rowptr, s.col, s.val), s.m, s.n)
    assert sp.stats()["mfma_tiles"] > 0
    Bsf = torch.from_numpy(dense_B(s.n + 1, K, seed=K + 1).reshape(-1)[: (s.n + 1) * K]).cuda()
    Bs = Bsf[off: off + s.n * K].view(s.n, K)
    Cs = sp.spmm(Bs)
    torch.cuda.synchronize()
    check(Cs.cpu().numpy(), osp.csr_spmm(s.rowptr, s.col, s.val, Bs.cpu().numpy(), m=s.m), f"sbm K={K}")


def test_long_rows_are_split_and_fixed_up():
    say("long rows")
    # a few rows with 20k-60k entries next to short rows: pieces + fixup, no atomics
    rng = np.random.default_rng(4)
    m, n = 64, 80000
    degs = np.array([60000 if r % 16 == 3 else (20000 if r == 40 else int(rng.integers(0, 5))) for r in range(m)])
    rows = np.repeat(np.arange(m), degs)
    cols = np.concatenate([np.sort(rng.choice(n, size=d, replace=False)) for d in degs])
    rowptr = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
    val = rng.uniform(0, 1, size=len(cols)).astype(np.float16).astype(np.float32)
    plan = trspmm.Plan.from_format(trspmm.build_format(rowptr, cols.astype(np.int32), val), m, n)
    st = plan.stats()
    assert st["split_rows"] >= 4 and st["partial_slots"] > st["split_rows"]
    Bh = dense_B(n, 128, seed=3)
    C = run_plan(plan, Bh)
    check(C, osp.csr_spmm(rowptr, cols, val, Bh, m=m), "long rows")
    del rows


def test_empty_rows_and_empty_matrix_are_zero():
    rowptr = np.zeros(33, np.int32)
    plan = trspmm.Plan.from_format(trspmm.build_format(rowptr, np.zeros(0, np.int32), np.zeros(0, np.float32)), 32, 10)
    B = torch.ones(10, 64, dtype=torch.float16, device="cuda")
    out = torch.full((32, 64), 3.0, device="cuda")
    plan.spmm(B, out=out)
    torch.cuda.synchronize()
    assert torch.all(out == 0)


def test_rows_beyond_m_are_dropped_like_reference():
    # mOri smaller than the padded row count: rows >= m are not written (mGCNkernel_online.cu `row < mOri`)
    g = graphs.random_csr(40, 50, 0.2, seed=2)            # padded to 48 rows
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, 40, g.n)
    Bh = dense_B(g.n, 32, seed=1)
    C = run_plan(plan, Bh)
    assert C.shape == (40, 32)
    check(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=40), "m<rows")


@pytest.mark.parametrize("K", [4, 32, 128])
def test_streaming_hints_do_not_change_results(K):
    """Plan option `streaming`: bit 0 streams the column/value loads, bit 1 the C stores (the
    default; plain below 8 features).  Cache hints only: all four settings bitwise equal, on a
    plan with MFMA windows, residual tasks and split rows."""
    say("streaming", K)
    g = graphs.sbm(communities=200, seed=21, val_seed=22)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    Bh = dense_B(g.n, K, seed=7)
    outs = [run_plan(trspmm.Plan.from_format(f, g.m, g.n, streaming=st, piece_nnz=32), Bh) for st in (0, 1, 2, 3)]
    check(outs[0], osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), f"streaming K={K}")
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


@pytest.mark.parametrize("K,lanes", [(128, 4), (64, 2), (40, 8), (66, 16)])
def test_feature_lanes_option(K, lanes):
    """Plan option feature_lanes: fewer lanes per group than the width needs, the features split
    into passes over the tasks (grid dimension y).  Against the oracle."""
    say("lanes", K, lanes)
    g = graphs.rmat(scale=12, edge_factor=16, seed=14)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    Bh = dense_B(g.n, K, seed=8)
    C = run_plan(trspmm.Plan.from_format(f, g.m, g.n, feature_lanes=lanes, piece_nnz=64), Bh)
    check(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), f"lanes K={K}")


@pytest.mark.parametrize("cap", [1, 8])
def test_window_row_cap_option(cap):
    """Plan option window_row_cap: windows whose residual rows are longer than the cap hand their
    tiles back to the residual path.  Against the oracle, with a dense-block graph."""
    say("cap", cap)
    g = graphs.sbm(communities=200, seed=23, val_seed=24)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    Bh = dense_B(g.n, 64, seed=9)
    C = run_plan(trspmm.Plan.from_format(f, g.m, g.n, window_row_cap=cap), Bh)
    check(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), f"cap={cap}")


def _blocks_with_long_rows(extra, seed):
    """64 windows of 16 rows, each window a dense 16x16 block on its own 16 columns (TC tiles)
    plus `extra` random residual entries in every row (uniformly long rows)."""
    rng = np.random.default_rng(seed)
    m, n = 1024, 200_000
    rows = []
    for r in range(m):
        w = r // 16
        cols = set(range(16 * w, 16 * w + 16)) | {int(x) for x in rng.integers(2048, n, size=extra)}
        rows.append(sorted(cols))
    rowptr = np.zeros(m + 1, np.int32)
    rowptr[1:] = np.cumsum([len(c) for c in rows])
    col = np.concatenate([np.array(c, np.int32) for c in rows])
    val = rng.uniform(-1, 1, size=len(col)).astype(np.float32)
    return m, n, rowptr, col, val


@pytest.mark.parametrize("extra,kept", [(200, True), (700, False)])
def test_windows_of_uniformly_long_rows(extra, kept):
    """A window whose residual rows are all long keeps its tiles up to 4 x window_row_cap (512)
    entries per row, and hands them back beyond that (the window kernel walks each row with one
    lane group); with the cap lifted every window keeps them.  Against the oracle either way."""
    say("long rows", extra)
    m, n, rowptr, col, val = _blocks_with_long_rows(extra, seed=extra)
    f = trspmm.build_format(rowptr, col, val)
    Bh = dense_B(n, 128, seed=3)
    R = osp.csr_spmm(rowptr, col, val, Bh, m=m)
    for cap in (0, 1 << 30):
        plan = trspmm.Plan.from_format(f, m, n, window_row_cap=cap)
        windows = plan.stats()["mfma_windows"]
        assert (windows > 0) == (kept or cap > 0), (extra, cap, plan.stats())
        check(run_plan(plan, Bh), R, f"long rows {extra} cap {cap}")


@pytest.mark.parametrize("xcd_run", [1, 3, 16, 64])
@pytest.mark.parametrize("m", [997, 40000])
def test_xcd_remap_covers_every_work_item(xcd_run, m):
    """Workgroup remapping must be a bijection for any grid size (NaN-prefilled output)."""
    g = graphs.random_csr(m, 5000, 3.0 / 5000, seed=m)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    for K in (32, 128):
        plan = trspmm.Plan.from_format(f, g.m, g.n, xcd_run=xcd_run, task_nnz=32)
        Bh = dense_B(g.n, K, seed=1)
        check(run_plan(plan, Bh), osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), f"xcd_run={xcd_run}")


def test_deterministic_bitwise():
    g = graphs.rmat(scale=13, edge_factor=16, seed=1)
    plan = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    B = torch.from_numpy(dense_B(g.n, 128, seed=2)).cuda()
    c1 = plan.spmm(B).clone()
    c2 = plan.spmm(B).clone()
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)


def test_plan_from_plain_csr_is_sddmm_only():
    g = graphs.random_csr(50, 50, 0.1, seed=1)
    plan = trspmm.Plan.from_csr(g.rowptr[:51], g.col, g.val.astype(np.float16), g.m, g.n)
    B = torch.zeros(g.n, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="SDDMM"):
        plan.spmm(B)


@pytest.mark.parametrize("K", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("task_nnz", [32, 128])
def test_pipelined_and_plain_streams(K, task_nnz):
    """Lane groups of <= 8 lanes take the pipelined residual stream for tasks of >= 64 entries
    (quad-shared column loads for the 4-lane groups of K = 16, 32), and 8-lane groups (K = 8, 64)
    for any task length; 4-lane groups with shorter tasks and 16-lane groups take the plain
    stream.  Each against the oracle."""
    say("streams", K, task_nnz)
    g = graphs.rmat(scale=12, edge_factor=16, seed=8)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    Bh = dense_B(g.n, K, seed=3)
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m)
    C = run_plan(trspmm.Plan.from_format(f, g.m, g.n, task_nnz=task_nnz), Bh)
    check(C, R, f"K={K} S={task_nnz}")


@pytest.mark.parametrize("K", [72, 128])
def test_staged_and_unstaged_streams_agree(K):
    """16-lane groups (K = 65..128) stage each task's column ids and values in LDS when every task
    holds <= 256 entries.  Tasks here start at every offset mod 8 and hold up to 256 entries; one
    row of 280 entries is split in two pieces with piece_nnz = 256 (staged) and kept whole with
    piece_nnz = 300 (a 280-entry task: the plan falls back to the unstaged stream).  Both against
    the oracle; every other row is summed in the same order, so bitwise equal."""
    say("staged", K)
    rng = np.random.default_rng(11)
    m, n = 4000, 20000
    degs = rng.integers(0, 40, size=m)
    degs[rng.choice(m, 60, replace=False)] = rng.integers(100, 257, size=60)
    degs[1234] = 280
    cols = np.concatenate([np.sort(rng.choice(n, size=d, replace=False)) for d in degs]).astype(np.int32)
    rowptr = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
    val = rng.uniform(-1, 1, size=len(cols)).astype(np.float16).astype(np.float32)
    f = trspmm.build_format(rowptr, cols, val, skip_tc=True)
    Bh = dense_B(n, K, seed=5)
    R = osp.csr_spmm(rowptr, cols, val, Bh, m=m)
    opts = dict(mfma_tc=False, mfma_sptc=False, task_nnz=128, xcd_split=-1)
    staged = trspmm.Plan.from_format(f, m, n, piece_nnz=256, **opts)
    whole = trspmm.Plan.from_format(f, m, n, piece_nnz=300, **opts)
    assert staged.stats()["split_rows"] == 1 and whole.stats()["split_rows"] == 0
    C1 = run_plan(staged, Bh)
    C2 = run_plan(whole, Bh)
    check(C1, R, f"staged K={K}")
    check(C2, R, f"unstaged K={K}")
    keep = np.arange(m) != 1234
    assert np.array_equal(C1[keep], C2[keep])
    # the same plan with staging switched off (stage = -1): every row bitwise equal
    C3 = run_plan(trspmm.Plan.from_format(f, m, n, piece_nnz=256, stage=-1, **opts), Bh)
    assert np.array_equal(C1, C3)


@pytest.mark.parametrize("K", [16, 32, 64, 128])
def test_occupancy_cap_does_not_change_results(K):
    """The residual task kernel's occupancy cap (dynamic LDS that limits workgroups per CU; 2 waves
    per SIMD by default for K <= 64) only changes how many tasks run at once: every output is
    bitwise the same with the cap at 2, 5 or off, and matches the oracle."""
    say("occupancy", K)
    g = graphs.rmat(scale=12, edge_factor=16, seed=9)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    Bh = dense_B(g.n, K, seed=4)
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m)
    outs = [run_plan(trspmm.Plan.from_format(f, g.m, g.n, occupancy=o), Bh) for o in (0, 2, 5, -1)]
    check(outs[0], R, f"occupancy K={K}")
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)


def test_leading_dimension_beyond_int32_is_refused():
    from trspmm import _native as nat
    import ctypes
    g = graphs.random_csr(64, 64, 0.1, seed=2)
    plan = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    B = torch.zeros(g.n, 16, dtype=torch.float16, device="cuda")
    C = torch.zeros(g.m, 16, device="cuda")
    need = plan.workspace_bytes(16)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    rc = nat.lib().trs_spmm_f16(plan.handle, B.data_ptr(), 1 << 31, 16, C.data_ptr(), 16, ws.data_ptr(), need,
                                int(torch.cuda.current_stream().cuda_stream))
    assert rc == 5, nat.lib().trs_last_error()          # TRS_ERANGE, nothing launched
    assert "2^31" in nat.lib().trs_last_error().decode()


@pytest.mark.parametrize("K", [8, 18, 24, 32, 128, 200])
def test_nonfinite_B_reaches_only_rows_that_use_it(K):
    """Padded batch slots re-read a real B row and lanes past K read real features (branch-free
    loads): a NaN / Inf in B must show up exactly in the outputs whose rows reference that B row
    (and only in its own feature column), never elsewhere.  Residual path only: a dense MFMA tile
    multiplies its absent entries as zeros, so 0 x Inf spreads a non-finite B row over the tile's
    window, as the reference's dense TC blocks do."""
    say("nonfinite", K)
    g = graphs.rmat(scale=11, edge_factor=8, seed=5)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    for task_nnz in (32, 128):
        plan = trspmm.Plan.from_format(f, g.m, g.n, mfma_tc=False, mfma_sptc=False, task_nnz=task_nnz)
        Bh = dense_B(g.n, K, seed=4)
        hub = int(np.argmax(np.bincount(g.col, minlength=g.n)))    # most referenced B row
        lone = int(np.argmin(np.where(np.bincount(g.col, minlength=g.n) > 0,
                                      np.bincount(g.col, minlength=g.n), 1 << 30)))
        Bh[hub, K - 1] = np.float16(np.nan)
        Bh[lone, 0] = np.float16(np.inf)
        C = run_plan(plan, Bh)
        rows = np.repeat(np.arange(g.m_pad), np.diff(g.rowptr))[: g.nnz]
        uses_hub = np.zeros(g.m, bool)
        uses_hub[rows[(g.col == hub) & (rows < g.m)]] = True
        uses_lone = np.zeros(g.m, bool)
        uses_lone[rows[(g.col == lone) & (rows < g.m)]] = True
        bad = ~np.isfinite(C)
        assert np.array_equal(bad[:, K - 1], uses_hub), "NaN column"
        assert np.array_equal(bad[:, 0], uses_lone), "Inf column"
        assert not bad[:, 1:K - 1].any(), "non-finite values leaked into other features"


@pytest.mark.parametrize("K", [16, 32, 64, 96, 128])
def test_xcd_column_split_matches_oracle_and_unsplit_rows(K):
    """Rows of >= xcd_split residual entries cut by 8 column ranges (one queue per XCD): against
    the oracle, deterministic from call to call, and every row left whole bitwise equal to the
    plan without the split (same entries, same order).  The widths cover each lane-group width of
    16-byte loads, whose split part takes batches of another size than the main part (8 lanes at
    K = 64, 4 at K = 32, 16 at K = 96 and 128), and 8-byte loads (K = 16)."""
    say("xcd split", K)
    g = graphs.rmat(scale=14, edge_factor=16, seed=12)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    Bh = dense_B(g.n, K, seed=13)
    R = osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m)
    split = trspmm.Plan.from_format(f, g.m, g.n, xcd_split=48)
    whole = trspmm.Plan.from_format(f, g.m, g.n, xcd_split=-1)
    assert split.stats()["split_rows"] > whole.stats()["split_rows"]
    C1 = run_plan(split, Bh)
    C2 = run_plan(whole, Bh)
    check(C1, R, f"xcd split K={K}")
    assert np.array_equal(C1, run_plan(split, Bh))
    deg = np.diff(g.rowptr[: g.m + 1])
    keep = deg < 48
    assert keep.sum() > g.m // 2 and np.array_equal(C1[keep], C2[keep])


@pytest.mark.parametrize("K", [200, 256, 520])
def test_feature_passes_with_split_rows(K):
    """K > 128 runs the residual kernel in passes of 128 features (16-lane groups): every pass
    writes its features of the main rows and of the split rows' partial slots, and the fixup sums
    each pass's slots.  Against the oracle on an R-MAT graph with many XCD-split rows."""
    say("feature passes", K)
    g = graphs.rmat(scale=14, edge_factor=16, seed=12)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n, xcd_split=48)
    assert plan.stats()["split_rows"] > 100
    Bh = dense_B(g.n, K, seed=13)
    C = run_plan(plan, Bh)
    check(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), f"passes K={K}")
    assert np.array_equal(C, run_plan(plan, Bh))


@pytest.mark.parametrize("K", [64, 256])
def test_dense_blocks_run_on_mfma_only(K):
    """bench.py's configuration 6 at a smaller size: every intra-community edge of 16-node
    communities aligned with the windows and no other edge, so every entry sits in a dense 16x16
    tile on MFMA and the window kernel runs no residual row; against the oracle."""
    say("dense blocks", K)
    g = graphs.sbm(communities=4096, p_in=1.0, inter_per_node=0, seed=5, val_seed=6)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n)
    st = plan.stats()
    nnz = int(g.rowptr[g.m])
    assert nnz == 4096 * 16 * 15 and st["mfma_nnz"] == nnz and st["csr_nnz"] == 0 and st["mfma_tiles"] == 4096
    Bh = dense_B(g.n, K, seed=7)
    check(run_plan(plan, Bh), osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m), f"dense blocks K={K}")


def test_plan_stats_size_is_checked_with_a_real_plan():
    """trs_plan_stats_get on a device plan: a stats struct of another header's size (12 fields in
    the first one) gets TRS_EINVAL and nothing is written past it; the right size succeeds."""
    import ctypes
    from trspmm import _native as nat
    say("case stats size")
    g = graphs.random_csr(64, 64, 0.1, seed=2)
    plan = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    lib = nat.lib()
    for size in (12 * 8, 15 * 8, 17 * 8):
        buf = ctypes.create_string_buffer(b"\xa5" * (size + 256), size + 256)
        rc = lib.trs_plan_stats_get(plan.handle, ctypes.cast(buf, ctypes.POINTER(nat.PlanStats)), size)
        assert rc == 1 and buf.raw == b"\xa5" * (size + 256), size
    s = nat.PlanStats()
    assert lib.trs_plan_stats_get(plan.handle, ctypes.byref(s), ctypes.sizeof(s)) == 0
    assert s.m == g.m and s.nnz == g.nnz
