"""Seeded synthetic graphs for the five benchmark configurations, as canonical CSR.

Every generator returns a :class:`Graph`: int32 ``rowptr``/``col`` with sorted, unique columns per
row, and float32 ``val`` holding fp16-representable numbers (values are drawn, then rounded to
fp16 once, so fp16 and fp32 consumers see the same matrix).  Row counts are padded to a multiple of
the 16-row window the same way the reference dataset layer pads them
(spmm/tr_csr_fp16/mdataset2_online.py:58-70): ``m_pad`` rows, of which the first ``m`` are real.

The reference loads ``.npz`` edge lists and assigns unseeded ``torch.randn`` values
(mdataset2_online.py:98); these generators replace that with fixed seeds so results are
reproducible.  ``load_npz`` reads the reference's dataset format for real graphs.
"""
from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass
class Graph:
    name: str
    m: int            # real rows (mOri)
    n: int            # columns = rows of the dense operand (kOri)
    rowptr: np.ndarray  # int32 [m_pad + 1]
    col: np.ndarray     # int32 [nnz]
    val: np.ndarray     # float32 [nnz], fp16-representable

    @property
    def nnz(self) -> int:
        return int(self.col.shape[0])

    @property
    def m_pad(self) -> int:
        return int(self.rowptr.shape[0] - 1)


def _round_fp16(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16).astype(np.float32)


def csr_from_keys(keys: np.ndarray, m: int, n: int, m_pad: int) -> tuple[np.ndarray, np.ndarray]:
    """Sorted unique int64 keys ``row * n + col`` -> (rowptr, col)."""
    rows = (keys // n).astype(np.int64)
    cols = (keys % n).astype(np.int32)
    counts = np.bincount(rows, minlength=m_pad).astype(np.int64)
    rowptr = np.zeros(m_pad + 1, dtype=np.int64)
    np.cumsum(counts, out=rowptr[1:])
    if rowptr[-1] > np.iinfo(np.int32).max:
        raise ValueError("nnz exceeds int32 range")
    return rowptr.astype(np.int32), cols


def pad_rows(m: int, window: int = 16) -> int:
    return m if m % window == 0 else m + window - m % window


def from_edges(name: str, src: np.ndarray, dst: np.ndarray, m: int, n: int, val_seed: int,
               symmetric: bool, window: int = 16, val_kind: str = "uniform01") -> Graph:
    """Edge list -> canonical CSR (dedup; optionally symmetrised), values drawn per stored entry."""
    src = src.astype(np.int64)
    dst = dst.astype(np.int64)
    if symmetric:
        src, dst = np.concatenate([src, dst]), np.concatenate([dst, src])
    keys = np.unique(src * n + dst)
    m_pad = pad_rows(m, window)
    rowptr, col = csr_from_keys(keys, m, n, m_pad)
    rng = np.random.default_rng(val_seed)
    if val_kind == "uniform01":
        val = _round_fp16(rng.random(col.shape[0], dtype=np.float32))
    elif val_kind == "normal":
        val = _round_fp16(rng.standard_normal(col.shape[0], dtype=np.float32))
    else:
        raise ValueError(val_kind)
    return Graph(name, m, n, rowptr, col, val)


def erdos_renyi_gcn(nodes: int = 4096, edges: int = 32768, seed: int = 0, window: int = 16) -> Graph:
    """Config 1: symmetric G(n, m) graph + self loops, values D^-1/2 (A+I) D^-1/2 in fp16."""
    rng = np.random.default_rng(seed)
    chosen = np.zeros(0, dtype=np.int64)
    while chosen.shape[0] < edges:
        need = edges - chosen.shape[0]
        u = rng.integers(0, nodes, size=2 * need + 16)
        v = rng.integers(0, nodes, size=2 * need + 16)
        keep = u != v
        a = np.minimum(u[keep], v[keep])
        b = np.maximum(u[keep], v[keep])
        cand = a * nodes + b
        # keep first occurrences in draw order, then merge with what we have
        _, first = np.unique(cand, return_index=True)
        cand = cand[np.sort(first)]
        cand = cand[~np.isin(cand, chosen)]
        chosen = np.concatenate([chosen, cand[:need]])
    a, b = chosen // nodes, chosen % nodes
    loops = np.arange(nodes, dtype=np.int64)
    src = np.concatenate([a, b, loops])
    dst = np.concatenate([b, a, loops])
    keys = np.unique(src * nodes + dst)
    m_pad = pad_rows(nodes, window)
    rowptr, col = csr_from_keys(keys, nodes, nodes, m_pad)
    deg = np.diff(rowptr)[:nodes].astype(np.float64)
    rows = np.repeat(np.arange(m_pad), np.diff(rowptr))
    val = _round_fp16((1.0 / np.sqrt(deg[rows] * deg[col])).astype(np.float32))
    return Graph("er4096_gcn", nodes, nodes, rowptr, col, val)


def rmat_edges(scale: int, edges: int, a: float, b: float, c: float, seed: int,
               chunk: int = 1 << 22) -> tuple[np.ndarray, np.ndarray]:
    """Recursive-matrix edge sampler (no noise): one quadrant draw per bit level."""
    rng = np.random.default_rng(seed)
    src = np.empty(edges, dtype=np.int64)
    dst = np.empty(edges, dtype=np.int64)
    ab, abc = a + b, a + b + c
    for s in range(0, edges, chunk):
        e = min(edges, s + chunk)
        u = np.zeros(e - s, dtype=np.int64)
        v = np.zeros(e - s, dtype=np.int64)
        for _ in range(scale):
            r = rng.random(e - s, dtype=np.float32)
            bit_u = r >= ab                      # quadrants c, d -> lower half
            bit_v = ((r >= a) & (r < ab)) | (r >= abc)  # quadrants b, d -> right half
            u = (u << 1) | bit_u
            v = (v << 1) | bit_v
        src[s:e] = u
        dst[s:e] = v
    return src, dst


def rmat(scale: int = 20, edge_factor: int = 16, seed: int = 42, val_seed: int = 1,
         abcd=(0.57, 0.19, 0.19, 0.05), window: int = 16) -> Graph:
    """Config 2: R-MAT power-law graph, deduplicated and symmetrised, values U[0,1) fp16."""
    n = 1 << scale
    src, dst = rmat_edges(scale, edge_factor * n, abcd[0], abcd[1], abcd[2], seed)
    return from_edges(f"rmat{scale}", src, dst, n, n, val_seed, symmetric=True, window=window)


def sbm(communities: int = 62500, size: int = 16, p_in: float = 0.6, inter_per_node: int = 4,
        seed: int = 3, val_seed: int = 3, window: int = 16) -> Graph:
    """Config 3: stochastic block model, communities aligned with 16-row windows and node labels
    permuted inside each window."""
    rng = np.random.default_rng(seed)
    n = communities * size
    iu, ju = np.triu_indices(size, k=1)
    take = rng.random((communities, iu.shape[0])) < p_in
    comm, pair = np.nonzero(take)
    src = comm * size + iu[pair]
    dst = comm * size + ju[pair]
    # inter-community edges: target drawn from the other communities
    u = np.repeat(np.arange(n, dtype=np.int64), inter_per_node)
    off = rng.integers(1, communities, size=u.shape[0])
    tc = (u // size + off) % communities
    v = tc * size + rng.integers(0, size, size=u.shape[0])
    src = np.concatenate([src, u])
    dst = np.concatenate([dst, v])
    perm = (np.arange(n) // size) * size + rng.permuted(np.tile(np.arange(size), (communities, 1)), axis=1).reshape(-1)
    return from_edges("sbm1m", perm[src], perm[dst], n, n, val_seed, symmetric=True, window=window)


def grid_hubs(side: int = 2048, hubs: int = 64, hub_degree: int = 100_000, seed: int = 6,
              val_seed: int = 6, window: int = 16) -> Graph:
    """Config 5: 4-neighbour 2-D grid plus hub rows with many random distinct neighbours
    (hub rows only; the hub edges are not mirrored)."""
    n = side * side
    idx = np.arange(n, dtype=np.int64)
    r, c = idx // side, idx % side
    parts_s, parts_d = [], []
    for dr, dc in ((0, 1), (0, -1), (1, 0), (-1, 0)):
        ok = (r + dr >= 0) & (r + dr < side) & (c + dc >= 0) & (c + dc < side)
        parts_s.append(idx[ok])
        parts_d.append((r[ok] + dr) * side + c[ok] + dc)
    rng = np.random.default_rng(seed)
    hub_rows = rng.choice(n, size=hubs, replace=False)
    for h in hub_rows:
        parts_s.append(np.full(hub_degree, h, dtype=np.int64))
        parts_d.append(rng.choice(n, size=hub_degree, replace=False).astype(np.int64))
    return from_edges("grid2048_hubs", np.concatenate(parts_s), np.concatenate(parts_d), n, n,
                      val_seed, symmetric=False, window=window)


def random_csr(m: int, n: int, density: float, seed: int, window: int = 16) -> Graph:
    """Uniform random sparse matrix (test helper)."""
    rng = np.random.default_rng(seed)
    cnt = rng.binomial(m * n, density)
    keys = np.unique(rng.integers(0, m * n, size=cnt, dtype=np.int64))
    m_pad = pad_rows(m, window)
    rowptr, col = csr_from_keys(keys, m, n, m_pad)
    val = _round_fp16(rng.uniform(-1, 1, size=col.shape[0]).astype(np.float32))
    return Graph(f"rand{m}x{n}", m, n, rowptr, col, val)


def dense_operand(rows: int, k: int, seed: int) -> np.ndarray:
    """fp16 matrix with entries U[-1, 1), returned as float16 numpy array [rows, k]."""
    rng = np.random.default_rng(seed)
    return rng.uniform(-1.0, 1.0, size=(rows, k)).astype(np.float32).astype(np.float16)


def load_npz(path: str, window: int = 16, val_seed: int = 0) -> Graph:
    """Reference dataset format {src_li, dst_li, num_nodes_src, num_nodes_dst}
    (spmm/tr_csr_fp16/tr_paths.py:22-30, mdataset2_online.py:58-70): rows padded to the window,
    duplicates merged, values drawn with a fixed seed."""
    with np.load(path, allow_pickle=False) as z:
        src = np.asarray(z["src_li"], dtype=np.int64)
        dst = np.asarray(z["dst_li"], dtype=np.int64)
        m = int(z["num_nodes_src"])
        n = int(z["num_nodes_dst"])
    g = from_edges(path, src, dst, m, n, val_seed, symmetric=False, window=window, val_kind="normal")
    return g


CONFIGS = {
    1: dict(graph=lambda: erdos_renyi_gcn(), k=64, b_seed=1),
    2: dict(graph=lambda: rmat(), k=128, b_seed=2),
    3: dict(graph=lambda: sbm(), k=256, b_seed=3),
    5: dict(graph=lambda: grid_hubs(), k=32, b_seed=7),
}
