"""Writes tests/golden/builder_*.npz: inputs and the 29 output arrays of the reference format builder
(TR-source/Block/block_online.cpp, compiled from its own source into oracle/_ref by
`make -C oracle ref`).  Run in the development container, where /root/reference exists:

    python tests/golden/make_golden.py

Each fixture holds `rowptr`, `col`, `val`, the builder parameters and `out_<slot>` for slots 0..28
(slot 29, the build time, is not deterministic and is not stored).  The reference prints per-window
diagnostics on stdout; they are discarded.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tr-spmm_zzx_amd"))

from oracle import builder as ob  # noqa: E402
from trspmm import graphs  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT = dict(part_t=32, part_c=32, short_size=3, density=8, window=16, tc_min_util=0.0)


def noncanonical(seed: int = 11):
    """Rows with unsorted columns and duplicate entries (exercises first-occurrence rules)."""
    rng = np.random.default_rng(seed)
    rows, cols = [], []
    for r in range(48):
        k = int(rng.integers(0, 30))
        c = rng.integers(0, 40, size=k)
        rows.extend([r] * k)
        cols.extend(c.tolist())
    rowptr = np.zeros(49, dtype=np.int32)
    np.add.at(rowptr, np.asarray(rows) + 1, 1)
    rowptr = np.cumsum(rowptr).astype(np.int32)
    val = rng.uniform(-1, 1, size=len(cols)).astype(np.float16).astype(np.float32)
    return rowptr, np.asarray(cols, dtype=np.int32), val


def cases():
    g = graphs.erdos_renyi_gcn(nodes=512, edges=4096, seed=0)
    yield "er512", g.rowptr, g.col, g.val, {}, {}
    g = graphs.rmat(scale=10, edge_factor=8, seed=5, val_seed=6)
    yield "rmat10", g.rowptr, g.col, g.val, {}, {}
    g = graphs.sbm(communities=64, seed=3, val_seed=4)
    yield "sbm64", g.rowptr, g.col, g.val, {}, {}
    g = graphs.grid_hubs(side=64, hubs=2, hub_degree=1500, seed=6, val_seed=7)
    yield "gridhubs64", g.rowptr, g.col, g.val, {}, {}
    g = graphs.random_csr(300, 250, 0.08, seed=3, window=8)
    yield "rand_w8", g.rowptr, g.col, g.val, dict(window=8, density=3), {}
    g = graphs.random_csr(200, 120, 0.2, seed=4, window=32)
    yield "rand_w32", g.rowptr, g.col, g.val, dict(window=32), {}
    g = graphs.random_csr(130, 90, 0.25, seed=5, window=1)   # 130 rows: last window partial
    yield "rand_params", g.rowptr, g.col, g.val, dict(part_t=2, part_c=5, short_size=2, density=5,
                                                      tc_min_util=0.4), {}
    g = graphs.random_csr(160, 100, 0.15, seed=6)
    yield "rand_env", g.rowptr, g.col, g.val, {}, {"LIBRA_SKIP_TC": "1", "LIBRA_SPTC_UNIT_MIN_NNZ": "3"}
    r, c, v = noncanonical()
    yield "noncanonical", r, c, v, {}, {}
    yield "empty_rows", np.zeros(33, dtype=np.int32), np.zeros(0, dtype=np.int32), np.zeros(0, dtype=np.float32), {}, {}


def run_reference(mod, rowptr, col, val, p):
    import torch
    fd = os.dup(1)
    nul = os.open(os.devnull, os.O_WRONLY)
    os.dup2(nul, 1)
    try:
        out = mod.block_sptc_2to4_online(torch.from_numpy(rowptr), torch.from_numpy(col), torch.from_numpy(val),
                                         p["part_t"], p["part_c"], p["short_size"], p["density"], p["window"], 16,
                                         float(p["tc_min_util"]), 0.5, 12)
    finally:
        os.dup2(fd, 1)
        os.close(nul)
        os.close(fd)
    return [t.numpy().copy() for t in out]


def main():
    mod = ob.reference_module()
    if mod is None:
        sys.exit("oracle/_ref is not built (make -C oracle ref, needs /root/reference)")
    for name, rowptr, col, val, over, env in cases():
        p = dict(DEFAULT, **over)
        old = {k: os.environ.get(k) for k in env}
        os.environ.update(env)
        try:
            out = run_reference(mod, rowptr, col, val, p)
        finally:
            for k, v in old.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v
        blob = {"rowptr": rowptr, "col": col, "val": val}
        for k, v in p.items():
            blob["param_" + k] = np.asarray(v)
        for k, v in env.items():
            blob["env_" + k] = np.asarray(v)
        for i in range(29):
            blob[f"out_{i}"] = out[i]
        np.savez_compressed(os.path.join(HERE, f"builder_{name}.npz"), **blob)
        print(name, "nnz", len(col), "groups", out[17].shape[0], "tiles", out[23].shape[0])


if __name__ == "__main__":
    main()
