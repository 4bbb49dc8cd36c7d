"""trs_spmm_f16_noalloc (the SpMM entry point that allocates nothing) against trs_spmm_f16, both
called through the C ABI: bitwise equal outputs on two calls in a row, the second with a smaller
input (the static scratch array keeps the first call's partial slots), a plan without split rows,
and a plan whose partial slots exceed the scratch array, refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from trspmm import _native as nat
from trspmm import graphs
import trspmm

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 128 << 20   # TRS_NOALLOC_SCRATCH_BYTES


def _stream():
    return int(torch.cuda.current_stream().cuda_stream)


def _with_workspace(plan, B):
    K = B.shape[1]
    C = torch.full((plan.stats()["m"], K), float("nan"), dtype=torch.float32, device="cuda")
    need = plan.workspace_bytes(K)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    nat.check(nat.lib().trs_spmm_f16(plan.handle, B.data_ptr(), B.stride(0), K, C.data_ptr(), C.stride(0),
                                     ws.data_ptr() if need else 0, need, _stream()), "trs_spmm_f16")
    torch.cuda.synchronize()
    return C


def _noalloc(plan, B):
    K = B.shape[1]
    C = torch.full((plan.stats()["m"], K), float("nan"), dtype=torch.float32, device="cuda")
    rc = nat.lib().trs_spmm_f16_noalloc(plan.handle, B.data_ptr(), B.stride(0), K, C.data_ptr(), C.stride(0),
                                        _stream())
    torch.cuda.synchronize()
    return rc, C


def _split_plan(side, hubs, hub_degree, seed):
    g = graphs.grid_hubs(side=side, hubs=hubs, hub_degree=hub_degree, seed=seed, val_seed=seed + 1)
    plan = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    assert plan.stats()["split_rows"] > 0 and plan.stats()["partial_slots"] > 0
    return g, plan


def test_noalloc_equals_workspace_call_twice_second_smaller():
    print("noalloc: large then small", flush=True)
    cases = [(_split_plan(128, 4, 8000, 3), 128), (_split_plan(48, 2, 1500, 5), 64)]
    assert cases[1][0][1].workspace_bytes(cases[1][1]) < cases[0][0][1].workspace_bytes(cases[0][1])
    for (g, plan), K in cases:
        B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=K)).cuda()
        ref = _with_workspace(plan, B)
        rc, C = _noalloc(plan, B)
        assert rc == 0, nat.lib().trs_last_error().decode()
        assert torch.equal(C, ref), (g.m, K)


def test_noalloc_without_split_rows():
    print("noalloc: no partial slots", flush=True)
    g = graphs.sbm(communities=128, seed=3, val_seed=4)
    plan = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    assert plan.workspace_bytes(32) == 0
    B = torch.from_numpy(graphs.dense_operand(g.n, 32, seed=9)).cuda()
    rc, C = _noalloc(plan, B)
    assert rc == 0, nat.lib().trs_last_error().decode()
    assert torch.equal(C, _with_workspace(plan, B))


def test_noalloc_refuses_plans_beyond_the_scratch_array():
    print("noalloc: beyond the scratch array", flush=True)
    g = graphs.random_csr(4096, 4096, 0.5, seed=7)
    # every row of ~2048 entries split into pieces of 32: over 262K partial slots
    f = trspmm.build_format(g.rowptr, g.col, g.val, skip_tc=True)
    plan = trspmm.Plan.from_format(f, g.m, g.n, mfma_tc=False, mfma_sptc=False, piece_nnz=32, task_nnz=32)
    K = 256
    need = plan.workspace_bytes(K)
    assert need > SCRATCH_BYTES, need
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=1)).cuda()
    rc, C = _noalloc(plan, B)
    assert rc == 1 and "scratch" in nat.lib().trs_last_error().decode()
    assert bool(torch.isnan(C).all())    # nothing was launched
    # the array still serves a plan that fits, after the refusal
    g2, plan2 = _split_plan(48, 2, 1500, 5)
    B2 = torch.from_numpy(graphs.dense_operand(g2.n, 96, seed=2)).cuda()
    rc, C2 = _noalloc(plan2, B2)
    assert rc == 0 and torch.equal(C2, _with_workspace(plan2, B2))


def test_noalloc_captured_in_a_graph_after_a_warm_up_call():
    """The header's graph-capture use: after one call outside capture on the device (which looks up
    the scratch array's address), a noalloc call is captured into a HIP graph and replayed three
    times, with eager work between replays that overwrites the shared scratch array (a noalloc call
    of another plan); every replay equals the eager trs_spmm_f16 result bitwise."""
    print("noalloc: graph capture after warm-up", flush=True)
    g, plan = _split_plan(128, 4, 8000, 3)
    g2, plan2 = _split_plan(48, 2, 1500, 5)
    K = 128
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=11)).cuda()
    B2 = torch.from_numpy(graphs.dense_operand(g2.n, 64, seed=12)).cuda()
    ref = _with_workspace(plan, B)
    rc, _ = _noalloc(plan, B)          # warm-up outside capture
    assert rc == 0, nat.lib().trs_last_error().decode()
    C = torch.full((plan.stats()["m"], K), float("nan"), dtype=torch.float32, device="cuda")
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = nat.lib().trs_spmm_f16_noalloc(plan.handle, B.data_ptr(), B.stride(0), K, C.data_ptr(), C.stride(0),
                                                int(side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert rc == 0, nat.lib().trs_last_error().decode()
    for i in range(3):
        rc2, _ = _noalloc(plan2, B2)   # eager work that rewrites the scratch array
        assert rc2 == 0
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, ref), f"replay {i}"
