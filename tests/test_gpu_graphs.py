"""HIP graph capture of the SpMM and SDDMM calls: they issue kernels only (no memset nodes, no
allocation with preallocated outputs and workspace), so a captured call replays.  Every replay is
checked against the eager result, with eager work and synchronisation between replays."""
import numpy as np
import pytest
import torch

import trspmm
from trspmm import graphs

pytestmark = pytest.mark.gpu


def test_spmm_graph_replays_match_eager():
    print("graph spmm", flush=True)
    g = graphs.sbm(communities=400, seed=11, val_seed=12)      # MFMA windows + residual tasks + fixups
    plan = trspmm.Plan.from_format(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    K = 64
    B = torch.from_numpy(graphs.dense_operand(g.n, K, seed=3)).cuda()
    C = torch.empty(g.m, K, device="cuda")
    ws = torch.empty(max(plan.workspace_bytes(K), 1), dtype=torch.uint8, device="cuda")
    eager = plan.spmm(B, out=C.clone(), workspace=ws).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):                                   # warm up on the capture stream
        plan.spmm(B, out=C, workspace=ws, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.spmm(B, out=C, workspace=ws, stream=torch.cuda.current_stream())
    for i in range(4):
        C.fill_(float("nan"))                                    # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(C, eager), f"replay {i}"
    B2 = torch.from_numpy(graphs.dense_operand(g.n, K, seed=4)).cuda()
    B.copy_(B2)                                                  # same buffers, new data
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(C, plan.spmm(B2, workspace=ws))


def test_sddmm_graph_replays_match_eager():
    print("graph sddmm", flush=True)
    g = graphs.rmat(scale=11, edge_factor=8, seed=9)
    plan = trspmm.Plan.for_sddmm(trspmm.build_format(g.rowptr, g.col, g.val), g.m, g.n)
    K = 32
    X = torch.from_numpy(graphs.dense_operand(g.m, K, seed=1)).cuda()
    Y = torch.from_numpy(graphs.dense_operand(g.n, K, seed=2)).cuda()
    out = torch.empty(plan.stats()["nnz"], device="cuda")
    eager = plan.sddmm(X, Y).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.sddmm(X, Y, out=out, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.sddmm(X, Y, out=out, stream=torch.cuda.current_stream())
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
