"""GPU: seeded random sparse matrices of varied shape through the default plans (device lowering,
2:4 tiles on the sparse MFMA, XCD split where it applies) against the float64 oracle, and device-
against host-lowered plans bitwise.

Each case mixes what the fixed graphs keep apart: empty rows, rows of a few entries, long rows
(split rows and pieces), dense column blocks inside 16-row windows (TC tiles), half-dense blocks
(2:4 group tiles), a row count that is not a multiple of 16, and a feature width drawn from the
load-width classes (including K > 128, which runs in feature passes).
"""
import numpy as np
import pytest
import torch

from oracle import spmm as osp
import trspmm

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.cuda.init()


def random_matrix(seed):
    rng = np.random.default_rng(seed)
    m = int(rng.integers(200, 3000))
    n = int(rng.integers(64, 4000))
    rows = []
    for r in range(m):
        kind = rng.random()
        if kind < 0.15:
            cols = np.zeros(0, np.int64)                                   # empty row
        elif kind < 0.85:
            cols = rng.choice(n, size=min(n, int(rng.integers(1, 24))), replace=False)
        elif kind < 0.95:
            cols = rng.choice(n, size=min(n, int(rng.integers(100, 900))), replace=False)  # long row
        else:
            cols = rng.choice(n, size=min(n, int(rng.integers(900, 3000))), replace=False)
        rows.append(cols)
    # dense and half-dense column blocks inside some 16-row windows
    for w in range(0, m, 16):
        u = rng.random()
        if u < 0.2 and n >= 32:
            c0 = int(rng.integers(0, n - 32))
            fill = 0.9 if u < 0.1 else 0.45
            for r in range(w, min(m, w + 16)):
                block = c0 + np.nonzero(rng.random(32) < fill)[0]
                rows[r] = np.concatenate([rows[r], block])
    rowptr = np.zeros(m + 1, np.int64)
    cols_all = []
    for r, cols in enumerate(rows):
        cols = np.unique(cols)
        cols_all.append(cols)
        rowptr[r + 1] = rowptr[r] + len(cols)
    col = np.concatenate(cols_all).astype(np.int32) if rowptr[-1] else np.zeros(0, np.int32)
    val = rng.uniform(-1, 1, size=len(col)).astype(np.float16).astype(np.float32)
    return m, n, rowptr.astype(np.int32), col, val


WIDTHS = [1, 6, 16, 33, 64, 100, 128, 200, 256]


@pytest.mark.parametrize("seed", range(12))
def test_random_matrix_spmm_sddmm(seed):
    m, n, rowptr, col, val = random_matrix(seed)
    K = WIDTHS[seed % len(WIDTHS)]
    say("random matrix", seed, "m", m, "n", n, "nnz", len(col), "K", K)
    f = trspmm.build_format(rowptr, col, val)
    rng = np.random.default_rng(100 + seed)
    Bh = rng.uniform(-1, 1, size=(n, K)).astype(np.float16)
    R = osp.csr_spmm(rowptr, col, val, Bh, m=m)
    # default window demotion, or none (every window with tiles stays an MFMA window)
    dev = trspmm.Plan.from_format(f, m, n, window_row_cap=int(rng.choice([0, 1 << 30])))
    B = torch.from_numpy(Bh).cuda()
    C = dev.spmm(B)
    torch.cuda.synchronize()
    e = osp.spmm_error(C.cpu().numpy(), R)
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, (dev.stats(), e)
    say("  stats", dev.stats())
    # the same options on both lowerings: bitwise equal
    cap = 1 << 30
    d2 = trspmm.Plan.from_format(f, m, n, window_row_cap=cap)
    h2 = trspmm.Plan.from_format(f, m, n, window_row_cap=cap, host_lowering=True)
    assert torch.equal(d2.spmm(B), h2.spmm(B))
    # SDDMM against the closed form
    Xh = rng.uniform(-1, 1, size=(m, K)).astype(np.float16)
    Yh = rng.uniform(-1, 1, size=(n, K)).astype(np.float16)
    sp = trspmm.Plan.for_sddmm(f, m, n)
    S = sp.sddmm(torch.from_numpy(Xh).cuda(), torch.from_numpy(Yh).cuda())
    torch.cuda.synchronize()
    Rs = osp.csr_sddmm(rowptr, col, Xh, Yh)
    tol = (1e-5 * np.sqrt(K) * 4 + 1e-6) * max(1.0, float(np.max(np.abs(Rs))) if len(Rs) else 1.0)
    assert S.shape[0] == len(col) and (len(col) == 0 or np.max(np.abs(S.cpu().numpy() - Rs)) <= tol)
