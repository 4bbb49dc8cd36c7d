"""Headline benchmark: hybrid fp16 SpMM on the R-MAT 2^20-node graph at K = 128 (one MI355X).

    python bench.py [--steps K] [--warmup W] [--config 2|3|5|4] [--no-cpu-baseline]

A step is one SpMM C = A B over the whole graph with A (device plan) and B already resident in
HBM.  Prints one JSON line with GFLOP/s (2 nnz K / t), the roofline object of the dominant kernel
(algorithmic bytes per launch / its HIP-event duration on the launch stream), and the CPU baseline
(torch.sparse.mm CSR fp32 on the host cores, the oracle's CPU SpMM) timed on a bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "tr-spmm_zzx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "SpMM GFLOP/s (2·nnz·K) + % HBM roofline, R-MAT 2^20 nodes K=128 fp16"
OTHER_METRIC = "SpMM GFLOP/s (2·nnz·K) + % HBM roofline, {workload} fp16"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_workload(cfg: int):
    from trspmm import graphs
    if cfg == 2 or cfg == 4:
        return "rmat20_k128", graphs.rmat(), 128, 2
    if cfg == 3:
        return "sbm1m_k256", graphs.sbm(), 256, 3
    if cfg == 5:
        return "grid2048_hubs_k32", graphs.grid_hubs(), 32, 7
    if cfg == 1:
        return "er4096_k64", graphs.erdos_renyi_gcn(), 64, 1
    raise SystemExit(f"unknown config {cfg}")


def kernel_ms(plan, B, C, ws, need, iters=10):
    import torch
    from trspmm import _native as nat
    ms = (ctypes.c_float * 3)()
    nat.check(nat.lib().trs_spmm_f16_kernel_ms(plan.handle, B.data_ptr(), B.stride(0), B.shape[1], C.data_ptr(),
                                               C.stride(0), ws.data_ptr() if need else 0, need,
                                               int(torch.cuda.current_stream().cuda_stream), iters, ms),
              "trs_spmm_f16_kernel_ms")
    return list(ms)


def cpu_baseline(g, Bh, flops):
    """torch.sparse.mm CSR fp32 on all host cores: 1 warm-up + median of up to 5 runs, bounded to
    about 20 s of CPU time (fewer runs on a slow host)."""
    import numpy as np
    import torch
    from oracle import spmm as osp
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B32 = torch.from_numpy(Bh.astype(np.float32))
    t0 = time.perf_counter()
    osp.torch_csr_spmm(g.rowptr, g.col, g.val, B32, m=g.m)
    first = time.perf_counter() - t0
    runs = max(1, min(5, int(20.0 / max(first, 1e-3))))
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        osp.torch_csr_spmm(g.rowptr, g.col, g.val, B32, m=g.m)
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    return {"value": round(flops / t / 1e9, 3), "unit": "GFLOP/s", "cores": cores, "kind": "port",
            "sample": f"full workload, torch.sparse.mm CSR fp32, median of {runs} after 1 warm-up "
                      f"({t * 1e3:.1f} ms/run)"}


def load_traffic(workload: str):
    path = os.path.join(ROOT, "profiles", f"spmm_tasks_{workload}_pmc.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    return d.get("hbm_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (asked for {args.gpus}): this build has no multi-GPU path; "
              "row windows would shard across GPUs with one all-gather of B (see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import trspmm
    from trspmm import graphs

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    t0 = time.time()
    workload, g, K, bseed = make_workload(args.config)
    log(f"[bench] graph {workload}: m={g.m} nnz={g.nnz} ({time.time() - t0:.1f}s)")
    t0 = time.time()
    fmt = trspmm.build_format(g.rowptr, g.col, g.val)
    log(f"[bench] format built in {fmt.elapsed:.2f}s")
    plan = trspmm.Plan.from_format(fmt, g.m, g.n)
    st = plan.stats()
    del fmt
    log(f"[bench] plan {st} ({time.time() - t0:.1f}s)")
    Bh = graphs.dense_operand(g.n, K, seed=bseed)
    B = torch.from_numpy(Bh).cuda()
    C = torch.empty((g.m, K), dtype=torch.float32, device="cuda")
    need = plan.workspace_bytes(K)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")

    if args.calibrate_copy_mib:
        n_el = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n_el, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    for _ in range(args.warmup):
        plan.spmm(B, out=C, workspace=ws)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        plan.spmm(B, out=C, workspace=ws)
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    flops = 2.0 * g.nnz * K
    gflops = flops / (ms_step * 1e-3) / 1e9
    log(f"[bench] {ms_step:.4f} ms/step, {gflops:.1f} GFLOP/s")

    # dominant kernel: per-kernel HIP events on the launch stream
    kms = kernel_ms(plan, B, C, ws, need)
    names = ["spmm_tasks", "spmm_mfma_win", "spmm_fixup"]
    dom = int(np.argmax(kms))
    M, N = g.m, g.n
    rows_w = min(M, 16 * st["mfma_windows"])
    nnz_w = st["window_csr_nnz"]
    if dom == 0:    # residual tasks: its entries, row pointers, one pass over B, its output rows
        nnz_k = st["csr_nnz"] - nnz_w
        rows_k = M - rows_w
        bytes_k = 6 * nnz_k + 4 * (rows_k + 1) + 16 * st["tasks"] + 2 * N * K + 4 * rows_k * K \
            + 4 * st["partial_slots"] * K
    elif dom == 1:  # MFMA windows: dense 16x16 fp16 tiles + 16 column ids, window residual, B once, C
        bytes_k = st["mfma_tiles"] * (512 + 64) + 6 * nnz_w + 2 * N * K + 4 * rows_w * K
    else:           # fixup: read partial slots, write split rows
        bytes_k = 4 * st["partial_slots"] * K + 4 * st["split_rows"] * K
    achieved = bytes_k / (kms[dom] * 1e-3) / 1e9
    alg_total = 6 * g.nnz + 4 * (M + 1) + 2 * N * K + 4 * M * K
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": load_traffic(workload),
            "kernel": names[dom], "kernel_ms": round(kms[dom], 4),
            "kernel_ms_all": {n: round(v, 4) for n, v in zip(names, kms)},
            "whole_step_frac": round(alg_total / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"[bench] kernels {kms}, roofline {roof}")

    metric = METRIC if args.config in (2, 4) else OTHER_METRIC.format(workload=workload)
    out = {"metric": metric, "value": round(gflops, 2), "unit": "GFLOP/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f16", "data": "synthetic",
           "config": {"workload": workload, "m": g.m, "n": g.n, "nnz": g.nnz, "K": K,
                      "mfma_tiles": st["mfma_tiles"], "mfma_nnz": st["mfma_nnz"], "parallelism": "none"},
           "roofline": roof}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(g, Bh, flops)
        log(f"[bench] cpu baseline {out['cpu_baseline']}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
