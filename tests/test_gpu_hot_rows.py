"""GPU: staged hot rows (plan option hot_rows).

A plan with a hot set keeps a second copy of its column ids in which every entry of the most
gathered columns is renumbered ~rank; at K >= 128 a call copies those B (Y) rows into a dense
buffer in the workspace and the task kernels gather them there.  Only where a row is read from
changes, so the outputs are bitwise equal to the unstaged plan's (same products, same order), and
both match the float64 oracle.  Covered: the automatic choice (R-MAT stages, a block graph does
not), widths that stage (128, 136, 256, 200) and ones that do not (64, 120), the split part (XCD
sub-rows) and MFMA windows beside staged rows (whose residual entries the choice does not count), workspace sizes, a workspace too small, the
entry point without workspace (trs_sddmm_f16) and the one that allocates nothing.
"""
import ctypes

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


_cache = {}


def rmat():
    if "rmat" not in _cache:
        g = graphs.rmat(scale=16, edge_factor=16, seed=21)
        _cache["rmat"] = (g, trspmm.build_format(g.rowptr, g.col, g.val))
    return _cache["rmat"]


def run_spmm(plan, Bh, ws_pad=0):
    B = torch.from_numpy(Bh).cuda()
    K = Bh.shape[1]
    out = torch.full((plan.stats()["m"], K), float("nan"), device="cuda")
    need = plan.workspace_bytes(K)
    ws = torch.empty(need + ws_pad, dtype=torch.uint8, device="cuda")
    plan.spmm(B, out=out, workspace=ws[ws_pad:] if ws_pad else ws)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_automatic_choice():
    g, f = rmat()
    p = trspmm.Plan.from_format(f, g.m, g.n)
    s = p.stats()
    say("rmat16", s)
    # n / 16 rows at most; they carry >= 30% of the gathers
    assert 0 < s["hot_rows"] <= g.n // 16 and s["hot_entries"] * 10 >= 3 * s["csr_nnz"], s
    off = trspmm.Plan.from_format(f, g.m, g.n, hot_rows=-1).stats()
    assert off["hot_rows"] == 0 and off["hot_entries"] == 0
    assert s["device_bytes"] > off["device_bytes"]
    # a block graph has no hot columns
    b = graphs.sbm(communities=4096, seed=3, val_seed=3)
    fb = trspmm.build_format(b.rowptr, b.col, b.val)
    assert trspmm.Plan.from_format(fb, b.m, b.n).stats()["hot_rows"] == 0


@pytest.mark.parametrize("K", [128, 136, 256, 200, 64, 120])
def test_spmm_staged_equals_unstaged(K):
    g, f = rmat()
    hot = trspmm.Plan.from_format(f, g.m, g.n)
    plain = trspmm.Plan.from_format(f, g.m, g.n, hot_rows=-1)
    assert hot.stats()["split_rows"] > 0   # the split part reads staged rows too
    H = hot.stats()["hot_rows"]
    partial = plain.workspace_bytes(K)
    staged = K >= 128 and K % 8 == 0
    want = ((partial + 255) // 256) * 256 + H * K * 2 if staged else partial
    assert hot.workspace_bytes(K) == want, (K, hot.workspace_bytes(K), want)
    Bh = graphs.dense_operand(g.n, K, seed=K)
    say("hot spmm K", K, "rows", H, "workspace", hot.workspace_bytes(K))
    C = run_spmm(hot, Bh)
    assert np.array_equal(C, run_spmm(plain, Bh))
    e = osp.spmm_error(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m))
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e
    # a workspace that is not 16-byte aligned runs unstaged with narrower loads: same sums
    C8 = run_spmm(hot, Bh, ws_pad=8)
    assert np.max(np.abs(C8 - C)) <= 1e-5 * max(1.0, float(np.max(np.abs(C))))


def sbm_with_plain_rows():
    """Block graph (every window owns MFMA tiles) followed by 1024 rows of 8 random columns from a
    pool of 4096: count-1 columns, whose 2:4 tiles are too sparse for MFMA, so those rows run on the
    task kernel, each pool column gathered about twice there."""
    if "sbm_plain" not in _cache:
        g = graphs.sbm(communities=4096, seed=5, val_seed=5)
        rng = np.random.default_rng(5)
        extra = np.sort(np.stack([rng.choice(4096, size=8, replace=False) for _ in range(1024)]), axis=1)
        col = np.concatenate([g.col[: g.rowptr[g.m]], (extra * 7 % g.n).astype(np.int32).ravel()])
        order = np.concatenate([np.arange(g.rowptr[g.m]),
                                g.rowptr[g.m] + np.argsort(col[g.rowptr[g.m]:].reshape(1024, 8), axis=1,
                                                           kind="stable").ravel()
                                + np.repeat(np.arange(1024) * 8, 8)])
        col = col[order].astype(np.int32)
        val = np.concatenate([g.val[: g.rowptr[g.m]],
                              rng.uniform(0, 1, 8192).astype(np.float16).astype(np.float32)])
        rowptr = np.concatenate([g.rowptr[: g.m + 1], g.rowptr[g.m] + 8 * np.arange(1, 1025)]).astype(np.int32)
        _cache["sbm_plain"] = graphs.Graph("sbm4096_plain", g.m + 1024, g.n, rowptr, col, val)
    return _cache["sbm_plain"]


def test_hot_rows_ignore_window_rows():
    """Staging counts only the task kernels' gathers: on a block graph whose residual entries all
    sit in MFMA-window rows (read through the plain ids by the window kernel) even an explicit row
    count stages nothing."""
    g = graphs.sbm(communities=4096, seed=5, val_seed=5)
    p = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n, hot_rows=100)
    s = p.stats()
    assert s["mfma_windows"] > 0 and s["window_csr_nnz"] == s["csr_nnz"], s   # every residual entry in a window
    assert s["hot_rows"] == 0 and s["hot_entries"] == 0, s


@pytest.mark.parametrize("H", [1, 100, 2000])
def test_spmm_explicit_hot_rows_with_windows(H):
    """An explicit row count stages whatever the share; a graph with MFMA windows keeps their B
    reads on the plain column ids."""
    g = sbm_with_plain_rows()
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    p = trspmm.Plan.from_format(f, g.m, g.n, hot_rows=H)
    s = p.stats()
    assert s["hot_rows"] == H and s["mfma_windows"] > 0, s
    assert 0 < s["hot_entries"] <= 8192, s
    Bh = graphs.dense_operand(g.n, 128, seed=7)
    C = run_spmm(p, Bh)
    assert np.array_equal(C, run_spmm(trspmm.Plan.from_format(f, g.m, g.n, hot_rows=-1), Bh))
    e = osp.spmm_error(C, osp.csr_spmm(g.rowptr, g.col, g.val, Bh, m=g.m))
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e


def test_spmm_workspace_too_small_is_refused():
    g, f = rmat()
    p = trspmm.Plan.from_format(f, g.m, g.n)
    K = 128
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=1)).cuda()
    C = torch.empty((g.m, K), dtype=torch.float32, device="cuda")
    need = p.workspace_bytes(K)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    rc = nat.lib().trs_spmm_f16(p.handle, B.data_ptr(), K, K, C.data_ptr(), K, ws.data_ptr(), need - 1,
                                int(torch.cuda.current_stream().cuda_stream))
    assert rc == 1 and b"workspace" in nat.lib().trs_last_error()


def test_noalloc_with_staged_rows():
    """trs_spmm_f16_noalloc takes the hot buffer from its static array too: equal to the call with
    a workspace, twice in a row (the second at a smaller width)."""
    g, f = rmat()
    p = trspmm.Plan.from_format(f, g.m, g.n)
    for K in (256, 128):
        assert p.workspace_bytes(K) <= 128 << 20
        Bh = graphs.dense_operand(g.n, K, seed=3 + K)
        B = torch.from_numpy(Bh).cuda()
        C = torch.full((g.m, K), float("nan"), dtype=torch.float32, device="cuda")
        nat.check(nat.lib().trs_spmm_f16_noalloc(p.handle, B.data_ptr(), K, K, C.data_ptr(), K,
                                                 int(torch.cuda.current_stream().cuda_stream)),
                  "trs_spmm_f16_noalloc")
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy(), run_spmm(p, Bh))


@pytest.mark.parametrize("K", [128, 256, 200, 64, 136, 264])
def test_sddmm_staged_equals_unstaged(K):
    """K = 136 and 264 end in a feature pass of 8 features (under 16 lanes), which reads the plain
    column ids while the earlier passes read the staged rows, accumulating into the same outputs."""
    g, f = rmat()
    hot = trspmm.Plan.for_sddmm(f, g.m, g.n)
    plain = trspmm.Plan.for_sddmm(f, g.m, g.n, hot_rows=-1)
    H = hot.stats()["hot_rows"]
    assert H > 0 and plain.stats()["hot_rows"] == 0
    # the split part's output buffer (both plans), then the staged rows
    base = plain.sddmm_workspace_bytes(K)
    staged = K >= 128 and K % 8 == 0
    assert hot.sddmm_workspace_bytes(K) == ((base + 255) // 256 * 256 + H * K * 2 if staged else base)
    Xh = graphs.dense_operand(g.m, K, seed=30 + K)
    Yh = graphs.dense_operand(g.n, K, seed=31 + K)
    X, Y = torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda()
    say("hot sddmm K", K, "rows", H)
    S = hot.sddmm(X, Y).cpu().numpy()
    assert np.array_equal(S, plain.sddmm(X, Y).cpu().numpy())
    # the entry point without a workspace runs unstaged
    out = torch.full((hot.stats()["nnz"],), float("nan"), device="cuda")
    nat.check(nat.lib().trs_sddmm_f16(hot.handle, X.data_ptr(), K, Y.data_ptr(), K, K, out.data_ptr(),
                                      int(torch.cuda.current_stream().cuda_stream)), "trs_sddmm_f16")
    torch.cuda.synchronize()
    assert np.array_equal(S, out.cpu().numpy())
    R = osp.csr_sddmm(g.rowptr[: g.m + 1], g.col, Xh, Yh)
    tol = (1e-5 * np.sqrt(K) * 4 + 1e-6) * max(1.0, float(np.max(np.abs(R))))
    assert np.max(np.abs(S - R)) <= tol


def test_sddmm_workspace_too_small_is_refused():
    g, f = rmat()
    p = trspmm.Plan.for_sddmm(f, g.m, g.n)
    K = 128
    need = p.sddmm_workspace_bytes(K)
    X = torch.from_numpy(graphs.dense_operand(g.m, K, seed=1)).cuda()
    Y = torch.from_numpy(graphs.dense_operand(g.n, K, seed=2)).cuda()
    out = torch.empty(p.stats()["nnz"], dtype=torch.float32, device="cuda")
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    rc = nat.lib().trs_sddmm_f16_ws(p.handle, X.data_ptr(), K, Y.data_ptr(), K, K, out.data_ptr(), ws.data_ptr(),
                                    need - 2, int(torch.cuda.current_stream().cuda_stream))
    assert rc == 1 and b"workspace" in nat.lib().trs_last_error()


def test_device_and_host_lowering_choose_the_same_rows():
    g, f = rmat()
    d = trspmm.Plan.from_format(f, g.m, g.n).stats()
    h = trspmm.Plan.from_format(f, g.m, g.n, host_lowering=True).stats()
    assert d["device_lowered"] == 1 and h["device_lowered"] == 0
    assert (d["hot_rows"], d["hot_entries"]) == (h["hot_rows"], h["hot_entries"])


def test_graph_replays_restage_the_rows():
    """Captured SpMM and SDDMM calls of a staging plan: each replay copies the hot rows again, so a
    replay after new data is written into B (Y) matches an eager call on that data."""
    g, f = rmat()
    K = 128
    sp = trspmm.Plan.from_format(f, g.m, g.n)
    dp = trspmm.Plan.for_sddmm(f, g.m, g.n)
    assert sp.stats()["hot_rows"] > 0 and dp.sddmm_workspace_bytes(K) > 0
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=50)).cuda()
    X = torch.from_numpy(graphs.dense_operand(g.m, K, seed=51)).cuda()
    C = torch.empty((g.m, K), device="cuda")
    S = torch.empty(dp.stats()["nnz"], device="cuda")
    ws = torch.empty(sp.workspace_bytes(K), dtype=torch.uint8, device="cuda")
    wd = torch.empty(dp.sddmm_workspace_bytes(K), dtype=torch.uint8, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        sp.spmm(B, out=C, workspace=ws, stream=s)
        dp.sddmm(X, B, out=S, workspace=wd, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sp.spmm(B, out=C, workspace=ws, stream=torch.cuda.current_stream())
        dp.sddmm(X, B, out=S, workspace=wd, stream=torch.cuda.current_stream())
    for seed in (52, 53, 54):
        B.copy_(torch.from_numpy(graphs.dense_operand(g.n, K, seed=seed)).cuda())
        C.fill_(float("nan"))
        S.fill_(float("nan"))
        ws.fill_(0xff)                     # stale staged rows would show
        wd.fill_(0xff)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say("graph replay", seed)
        assert torch.equal(C, sp.spmm(B)), seed
        assert torch.equal(S, dp.sddmm(X, B)), seed


def test_threads_share_a_staging_plan():
    """Staged rows live in each call's workspace: threads on their own streams with their own
    workspaces get the default-stream result bitwise."""
    import threading
    g, f = rmat()
    K = 128
    p = trspmm.Plan.from_format(f, g.m, g.n)
    Bs = [torch.from_numpy(graphs.dense_operand(g.n, K, seed=60 + t)).cuda() for t in range(4)]
    want = [p.spmm(B) for B in Bs]
    torch.cuda.synchronize()
    got, errors = [None] * 4, []

    def work(t):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                ws = torch.empty(p.workspace_bytes(K), dtype=torch.uint8, device="cuda")
                for _ in range(3):
                    got[t] = p.spmm(Bs[t], workspace=ws, stream=s)
            s.synchronize()
        except Exception as e:   # reported below
            errors.append(e)

    th = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for x in th:
        x.start()
    for x in th:
        x.join()
    assert not errors, errors
    for t in range(4):
        assert torch.equal(got[t], want[t]), t


def test_wide_sparse_matrix_stages_nothing():
    """n far above the entry count: the per-column counts are not taken, even when asked for."""
    m, n = 64, 1 << 20
    rng = np.random.default_rng(3)
    rowptr = np.arange(0, 4 * m + 1, 4, dtype=np.int32)
    col = np.sort(rng.choice(n, size=(m, 4), replace=False), axis=1).reshape(-1).astype(np.int32)
    val = rng.uniform(-1, 1, size=col.size).astype(np.float32)
    f = trspmm.build_format(rowptr, col, val)
    p = trspmm.Plan.from_format(f, m, n, hot_rows=100)
    assert p.stats()["hot_rows"] == 0
    Bh = graphs.dense_operand(n, 128, seed=4)
    C = run_spmm(p, Bh)
    e = osp.spmm_error(C, osp.csr_spmm(rowptr, col, val, Bh, m=m))
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e


@pytest.mark.parametrize("pad", [16, 8])
def test_staged_rows_from_strided_operands(pad):
    """B and Y as column slices of wider arrays (leading dimension K + pad, a multiple of 8): the
    rows are staged from the strided operand into the dense buffer; bitwise equal to unstaged."""
    g, f = rmat()
    K = 128
    hot = trspmm.Plan.from_format(f, g.m, g.n)
    plain = trspmm.Plan.from_format(f, g.m, g.n, hot_rows=-1)
    Bw = torch.zeros((g.n, K + pad), dtype=torch.float16, device="cuda")
    Bw[:, :K] = torch.from_numpy(graphs.dense_operand(g.n, K, seed=80)).cuda()
    B = Bw[:, :K]
    assert B.stride(0) == K + pad
    assert torch.equal(hot.spmm(B), plain.spmm(B))
    sh = trspmm.Plan.for_sddmm(f, g.m, g.n)
    sp = trspmm.Plan.for_sddmm(f, g.m, g.n, hot_rows=-1)
    X = torch.from_numpy(graphs.dense_operand(g.m, K, seed=81)).cuda()
    assert torch.equal(sh.sddmm(X, B), sp.sddmm(X, B))


def _brute_force_hot(col, n, want):
    """The hot set the plan documents: among the columns gathered at least twice, the `want` first
    in the order (count desc, column asc); returns (rows, their entries)."""
    cnt = np.bincount(col, minlength=n)
    cand = np.nonzero(cnt >= 2)[0]
    order = cand[np.lexsort((cand, -cnt[cand]))][:want]
    return len(order), int(cnt[order].sum())


@pytest.mark.parametrize("name,gen,want", [
    ("rmat16", lambda: graphs.rmat(scale=16, edge_factor=16, seed=21), 0),
    ("rmat16_2048", lambda: graphs.rmat(scale=16, edge_factor=16, seed=21), 2048),
    # many columns tied at each count: the cut falls inside a run of equal counts
    ("ties", lambda: graphs.random_csr(30000, 20000, 0.0006, seed=9), 700),
])
def test_hot_selection_equals_brute_force(name, gen, want):
    """The plan picks its hot rows through a histogram of the column counts; the rows and their
    entries equal a plain sort's choice (no tiles, no split: every entry is a task entry)."""
    g = gen()
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    s = trspmm.Plan.from_format(f, g.m, g.n, mfma_tc=False, mfma_sptc=False, xcd_split=-1,
                                hot_rows=want).stats()
    w = want if want > 0 else min(32768, g.n // 16)
    nnz = int(g.rowptr[g.m])
    rows, entries = _brute_force_hot(g.col[:nnz], g.n, w)
    say("hot selection", name, s["hot_rows"], s["hot_entries"], rows, entries)
    assert (s["hot_rows"], s["hot_entries"]) == (rows, entries)
