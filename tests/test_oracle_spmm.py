"""Pins the numeric oracle: CSR SpMM / SDDMM against independent computations."""
import numpy as np
import torch

from oracle import spmm as osp
from trspmm import graphs


def dense_of(g):
    A = np.zeros((g.m_pad, g.n))
    rows = np.repeat(np.arange(g.m_pad), np.diff(g.rowptr))
    np.add.at(A, (rows, g.col), g.val)
    return A


def test_csr_spmm_equals_dense_bruteforce():
    g = graphs.random_csr(70, 90, 0.1, seed=1)
    B = graphs.dense_operand(g.n, 13, seed=2).astype(np.float64)
    assert np.allclose(osp.csr_spmm(g.rowptr, g.col, g.val, B), dense_of(g) @ B, rtol=0, atol=1e-12)


def test_csr_spmm_identity_and_blocks():
    n = 48
    rowptr = np.arange(n + 1, dtype=np.int32)
    col = np.arange(n, dtype=np.int32)
    B = graphs.dense_operand(n, 8, seed=3).astype(np.float64)
    assert np.array_equal(osp.csr_spmm(rowptr, col, np.ones(n, np.float32), B), B)
    # all-ones 16x16 diagonal blocks: every output row is the block's column sum of B
    rows = np.repeat(np.arange(n), 16)
    cols = (rows // 16) * 16 + np.tile(np.arange(16), n)
    rp = np.arange(0, 16 * n + 1, 16, dtype=np.int32)
    C = osp.csr_spmm(rp, cols.astype(np.int32), np.ones(16 * n, np.float32), B)
    for b in range(3):
        assert np.allclose(C[16 * b:16 * b + 16], B[16 * b:16 * b + 16].sum(0, keepdims=True))


def test_torch_csr_spmm_matches_float64():
    g = graphs.rmat(scale=10, edge_factor=8, seed=3)
    B = graphs.dense_operand(g.n, 32, seed=4)
    R = osp.csr_spmm(g.rowptr, g.col, g.val, B, m=g.m)
    T = osp.torch_csr_spmm(g.rowptr, g.col, g.val, B.astype(np.float32), m=g.m).numpy()
    e = osp.spmm_error(T, R)
    assert e["elementwise_ok"] and e["max_rel_to_max"] < 1e-5


def test_spmm_linearity():
    g = graphs.random_csr(64, 64, 0.2, seed=5)
    B1 = graphs.dense_operand(64, 8, 1).astype(np.float64)
    B2 = graphs.dense_operand(64, 8, 2).astype(np.float64)
    lhs = osp.csr_spmm(g.rowptr, g.col, g.val, 3 * B1 - B2)
    rhs = 3 * osp.csr_spmm(g.rowptr, g.col, g.val, B1) - osp.csr_spmm(g.rowptr, g.col, g.val, B2)
    assert np.allclose(lhs, rhs, atol=1e-12)


def test_sddmm_closed_form():
    g = graphs.random_csr(40, 30, 0.2, seed=6)
    X = graphs.dense_operand(g.m_pad, 5, 1)
    Y = graphs.dense_operand(g.n, 5, 2)
    out = osp.csr_sddmm(g.rowptr, g.col, X, Y)
    full = X.astype(np.float64) @ Y.astype(np.float64).T
    rows = np.repeat(np.arange(g.m_pad), np.diff(g.rowptr))
    assert np.allclose(out, full[rows, g.col], atol=1e-12)
    A = torch.sparse_csr_tensor(torch.from_numpy(g.rowptr.astype(np.int64)), torch.from_numpy(g.col.astype(np.int64)),
                                torch.ones(g.nnz, dtype=torch.float64), size=(g.m_pad, g.n))
    ref = torch.sparse.sampled_addmm(A, torch.from_numpy(X).double(), torch.from_numpy(Y).double().T, beta=0.0)
    assert np.allclose(out, ref.values().numpy(), atol=1e-12)


def test_error_metric_catches_a_planted_mistake():
    g = graphs.random_csr(50, 50, 0.2, seed=7)
    B = graphs.dense_operand(50, 8, 1)
    R = osp.csr_spmm(g.rowptr, g.col, g.val, B)
    wrong = osp.csr_spmm(g.rowptr, (g.col + 1) % 50, g.val, B)   # off-by-one column
    assert not osp.spmm_error(wrong, R)["elementwise_ok"]
    dropped = osp.csr_spmm(g.rowptr, g.col, np.where(np.arange(g.nnz) % 97 == 0, 0, g.val), B)
    assert not osp.spmm_error(dropped, R)["elementwise_ok"]
