"""Writes tests/golden/builder_*.npz: inputs and the 29 output arrays of the reference format builder
(TR-source/Block/block_online.cpp, compiled from its own source into oracle/_ref by
`make -C oracle ref`).  Run in the development container, where /root/reference exists:

    python tests/golden/make_golden.py

Each fixture holds `rowptr`, `col`, `val`, the builder parameters and `out_<slot>` for slots 0..28
(slot 29, the build time, is not deterministic and is not stored).  The reference prints per-window
diagnostics on stdout; they are discarded.

    python tests/golden/make_golden.py digests

writes tests/golden/builder_digests.json instead: for the full-size BASELINE configurations 1
(Erdos-Renyi 4096), 3 (SBM, 1M rows, 17.0M entries) and 5 (2048 x 2048 grid + 64 hub rows of 100k
columns, 23.2M entries) and for R-MAT 2^18 (7.6M entries), too large to commit as arrays, the
SHA-256 of the input CSR and of each of the reference's 29 output arrays (dtype, shape and bytes;
see `array_digest`).  Configurations 1 and 3 and R-MAT 2^18 take about two minutes of reference
time; configuration 5 takes much longer, because the reference builds the complete unit graph of
each hub window (about 50k units, O(n^2) memory and time).

    python tests/golden/make_golden.py digests gridhubs4m_config5

(re)computes only the named cases and keeps the other entries of the file.
"""
from __future__ import annotations

import hashlib
import json
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


def array_digest(a) -> str:
    """SHA-256 of an array's dtype, shape and little-endian bytes (C order)."""
    a = np.ascontiguousarray(a)
    h = hashlib.sha256()
    h.update(f"{a.dtype.str}|{tuple(int(x) for x in a.shape)}|".encode())
    h.update(a.tobytes())
    return h.hexdigest()


def csr_digest(rowptr, col, val) -> str:
    return hashlib.sha256("|".join(array_digest(a) for a in (rowptr, col, val)).encode()).hexdigest()


def digest_cases():
    """(name, graph generator) of the full-size cases; the test regenerates the same graphs."""
    return [("er4096_config1", lambda: graphs.erdos_renyi_gcn()),
            ("sbm1m_config3", lambda: graphs.sbm()),
            ("rmat18", lambda: graphs.rmat(scale=18, edge_factor=16, seed=31)),
            ("gridhubs4m_config5", lambda: graphs.grid_hubs())]


def write_digests(mod, only=()):
    import time
    path = os.path.join(HERE, "builder_digests.json")
    out = {}
    if only and os.path.exists(path):
        with open(path) as f:
            out = json.load(f)
    for name, gen in digest_cases():
        if only and name not in only:
            continue
        g = gen()
        t0 = time.time()
        arrs = run_reference(mod, g.rowptr, g.col, g.val, DEFAULT)
        out[name] = {"m": g.m, "nnz": g.nnz, "input": csr_digest(g.rowptr, g.col, g.val),
                     "slots": [array_digest(arrs[i]) for i in range(29)],
                     "shapes": [list(arrs[i].shape) for i in range(29)]}
        print(name, "nnz", g.nnz, f"reference {time.time() - t0:.1f}s", flush=True)
        del arrs, g
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


def main():
    mod = ob.reference_module()
    if mod is None:
        sys.exit("oracle/_ref is not built (make -C oracle ref, needs /root/reference)")
    if sys.argv[1:2] == ["digests"]:
        write_digests(mod, tuple(sys.argv[2:]))
        return
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
