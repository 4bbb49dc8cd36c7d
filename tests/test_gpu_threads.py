"""A plan shared by host threads, each calling on its own stream.

Plans are immutable after creation and every call takes its workspace from the caller, so one
plan serves concurrent callers.  Results are compared bitwise with calls on the default stream
(same kernels, same summation order)."""
import threading

import pytest
import torch

from trspmm import graphs
import trspmm

pytestmark = pytest.mark.gpu


def _grid_plan():
    # mesh rows plus hub rows that are split into pieces, so the fixup kernel runs as well
    g = graphs.grid_hubs(side=96, hubs=3, hub_degree=3000, seed=1, val_seed=2)
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    plan = trspmm.Plan.from_format(f, g.m, g.n)
    assert plan.stats()["split_rows"] > 0
    return g, plan


def test_plan_shared_by_threads_on_own_streams():
    print("threads", flush=True)
    g, plan = _grid_plan()
    K = 64
    Bs = [torch.from_numpy(graphs.dense_operand(g.n, K, seed=20 + i)).cuda() for i in range(4)]
    ref = [plan.spmm(B).clone() for B in Bs]
    torch.cuda.synchronize()
    results = [[None] * 10 for _ in Bs]
    errors = []

    def work(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                ws = torch.empty(max(plan.workspace_bytes(K), 1), dtype=torch.uint8, device="cuda")
                for j in range(10):
                    results[i][j] = plan.spmm(Bs[i], workspace=ws, stream=s)
            s.synchronize()
        except Exception as e:  # reported in the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(Bs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(len(Bs)):
        for j in range(10):
            assert torch.equal(results[i][j], ref[i]), (i, j)


def test_stream_argument_without_workspace_matches_default_stream():
    """stream= names a side stream while the current stream stays the default one, and neither
    `out` nor the workspace is given: the temporaries must belong to the launch stream (the caching
    allocator may otherwise hand them to other work while the kernels still use them)."""
    print("side stream, library-allocated workspace", flush=True)
    g, plan = _grid_plan()
    K = 64
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=31)).cuda()
    ref = plan.spmm(B).clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    outs = []
    for _ in range(8):
        outs.append(plan.spmm(B, stream=s))
        # churn on the current (default) stream: would reuse a freed block allocated on it
        junk = torch.empty(plan.workspace_bytes(K) // 4 + 1024, dtype=torch.float32, device="cuda")
        junk.fill_(float("nan"))
    s.synchronize()
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, ref), i


def test_sddmm_output_validation_refuses_before_launch():
    """A caller's `out` for sddmm must be a contiguous CUDA float32 tensor of at least nnz
    elements; every other kind is refused with ValueError (no kernel is launched)."""
    print("sddmm out validation", flush=True)
    g = graphs.rmat(scale=10, edge_factor=8, seed=3)
    plan = trspmm.Plan.from_csr(g.rowptr, g.col, g.val.astype("float16"), g.m, g.n)
    nnz = plan.stats()["nnz"]
    X = torch.from_numpy(graphs.dense_operand(g.m, 32, seed=1)).cuda()
    Y = torch.from_numpy(graphs.dense_operand(g.n, 32, seed=2)).cuda()
    bad = [torch.empty(nnz, dtype=torch.float32),                                  # host memory
           torch.empty(nnz, dtype=torch.float16, device="cuda"),                   # wrong dtype
           torch.empty(nnz - 1, dtype=torch.float32, device="cuda"),               # too short
           torch.empty(2 * nnz, dtype=torch.float32, device="cuda")[::2]]          # not contiguous
    for out in bad:
        with pytest.raises(ValueError):
            plan.sddmm(X, Y, out=out)
    with pytest.raises(ValueError):
        plan.sddmm(X.cpu(), Y)
    good = torch.full((nnz + 3,), -7.0, dtype=torch.float32, device="cuda")
    plan.sddmm(X, Y, out=good)
    torch.cuda.synchronize()
    assert torch.equal(good[:nnz], plan.sddmm(X, Y)) and bool((good[nnz:] == -7.0).all())
