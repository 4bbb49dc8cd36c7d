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
