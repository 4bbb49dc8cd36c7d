"""Headline benchmark: hybrid fp16 SpMM on the R-MAT 2^20-node graph at K = 128 (one MI355X).

    python bench.py [--steps K] [--warmup W] [--config 2|3|5|4] [--no-cpu-baseline]
                    [--scramble SEED] [--reorder tca]

A step is one SpMM C = A B over the whole graph with A (device plan) and B already resident in
HBM.  Prints one JSON line with GFLOP/s (2 nnz K / t), the roofline object of the dominant kernel
(compulsory bytes of the share it computes -- A's entries and row pointers, B once, C once -- per
launch / its HIP-event duration on the launch stream; the bytes its data layout adds on top, task
descriptors, partial slots and dense tile padding, are reported apart as `impl_bytes`), and the
CPU baseline (torch.sparse.mm CSR fp32 on the host cores, the oracle's CPU SpMM) timed on a bounded
sample.
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
    if cfg == 2:
        return "rmat20_k128", graphs.rmat(), 128, 2
    if cfg == 4:
        return "rmat20_sddmm", graphs.rmat(), 128, 4
    if cfg == 3:
        return "sbm1m_k256", graphs.sbm(), 256, 3
    if cfg == 5:
        return "grid2048_hubs_k32", graphs.grid_hubs(), 32, 7
    if cfg == 1:
        return "er4096_k64", graphs.erdos_renyi_gcn(), 64, 1
    if cfg == 6:
        # not a BASELINE configuration: config 3's windows with every intra-community edge and no
        # other, so that every entry sits in a dense 16x16 tile on MFMA (the MFMA path on its own)
        return "blockdiag1m_k256", graphs.sbm(p_in=1.0, inter_per_node=0), 256, 3
    raise SystemExit(f"unknown config {cfg}")


def scramble(g, seed: int):
    """Relabel the nodes of a square graph with a seeded random permutation (rows and columns):
    the same matrix up to P A P^T, with any locality of the node numbering destroyed."""
    import numpy as np
    from trspmm import graphs, reorder
    assert g.m == g.n, "scramble needs a square graph"
    perm = np.random.default_rng(seed).permutation(g.m)          # new label -> old label
    inv = np.empty(g.m, dtype=np.int64)
    inv[perm] = np.arange(g.m)
    rp, col, val = reorder.permute_rows(g.rowptr[: g.m + 1], g.col, perm, g.val)
    col = inv[col]
    rows = np.repeat(np.arange(g.m, dtype=np.int64), np.diff(rp))
    o = np.lexsort((col, rows))
    rowptr = np.concatenate([rp, np.full(g.m_pad - g.m, rp[-1], dtype=np.int32)])
    return graphs.Graph(g.name + "_scrambled", g.m, g.n, rowptr, col[o].astype(np.int32), val[o])


def tca_reorder(g, align_window: int = 0):
    """Row reorder of the reference's optional TCA step (LIBRA_TCA_REORDER=1), or its
    window-aligned variant; returns the reordered graph and the seconds it took."""
    from trspmm import graphs, reorder
    t0 = time.time()
    order = reorder.tca_order(g.rowptr[: g.m + 1], g.col, ncols=g.n, align_window=align_window)
    rp, col, val = reorder.permute_rows(g.rowptr[: g.m + 1], g.col, order, g.val)
    import numpy as np
    rowptr = np.concatenate([rp, np.full(g.m_pad - g.m, rp[-1], dtype=np.int32)])
    return graphs.Graph(g.name + "_tca", g.m, g.n, rowptr, col, val), time.time() - t0


def kernel_ms(plan, B, C, ws, need, iters=10):
    import torch
    from trspmm import _native as nat
    ms = (ctypes.c_float * 3)()
    nat.check(nat.lib().trs_spmm_f16_kernel_ms(plan.handle, B.data_ptr(), B.stride(0), B.shape[1], C.data_ptr(),
                                               C.stride(0), ws.data_ptr() if need else 0, need,
                                               int(torch.cuda.current_stream().cuda_stream), iters, ms),
              "trs_spmm_f16_kernel_ms")
    return list(ms)


def launched(kms, runs):
    """Per-kernel event intervals, None for a kernel the plan does not launch: its interval is
    empty and holds only the cost of the events themselves (~5 us)."""
    return [v if r else None for v, r in zip(kms, runs)]


def dominant(kms) -> int:
    return max((i for i, v in enumerate(kms) if v is not None), key=lambda i: kms[i])


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cold_ms(run, steps: int, flush_mib: int = 1024) -> float:
    """Median time of one step with L2 and MALL flushed first: a write of flush_mib MiB before
    every step, timed on the step alone with events around it."""
    import numpy as np
    import torch
    scratch = torch.empty(flush_mib * (1 << 20) // 4, dtype=torch.float32, device="cuda")
    ts = []
    for _ in range(steps):
        scratch.fill_(1.0)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        run()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    del scratch
    return float(np.median(ts))


def pcie_inclusive_ms(plan, Bh, C, ws, steps: int = 5) -> float:
    """Median time of host-to-host SpMM as the drop-in operators see it: B copied from pinned host
    memory, the SpMM, C copied back to pinned host memory (plan already resident)."""
    import numpy as np
    import torch
    Bp = torch.from_numpy(Bh).pin_memory()
    Cp = torch.empty(C.shape, dtype=C.dtype).pin_memory()
    Bd = torch.empty(Bp.shape, dtype=Bp.dtype, device="cuda")
    ts = []
    for _ in range(steps + 1):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        Bd.copy_(Bp, non_blocking=True)
        plan.spmm(Bd, out=C, workspace=ws)
        Cp.copy_(C, non_blocking=True)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return float(np.median(ts[1:]))


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
                      f"({t * 1e3:.1f} ms/run) on {cpu_model()}"}


def cpu_baseline_sddmm(g, Xh, Yh, flops):
    """torch.sparse.sampled_addmm CSR fp32 on all host cores, same bounds as cpu_baseline."""
    import numpy as np
    import torch
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    nnz = int(g.rowptr[g.m])
    A = torch.sparse_csr_tensor(torch.from_numpy(g.rowptr[: g.m + 1].astype(np.int64)),
                                torch.from_numpy(g.col[:nnz].astype(np.int64)), torch.ones(nnz), size=(g.m, g.n))
    X32 = torch.from_numpy(Xh.astype(np.float32))
    Y32t = torch.from_numpy(Yh.astype(np.float32)).T
    t0 = time.perf_counter()
    torch.sparse.sampled_addmm(A, X32, Y32t, beta=0.0)
    first = time.perf_counter() - t0
    runs = max(1, min(5, int(20.0 / max(first, 1e-3))))
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        torch.sparse.sampled_addmm(A, X32, Y32t, beta=0.0)
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    return {"value": round(flops / t / 1e9, 3), "unit": "GFLOP/s", "cores": cores, "kind": "port",
            "sample": f"full workload, torch.sparse.sampled_addmm CSR fp32, median of {runs} after 1 warm-up "
                      f"({t * 1e3:.1f} ms/run) on {cpu_model()}"}


def calibration_copy(mib: int) -> None:
    """One device copy of `mib` MiB (a known byte count for scaling FETCH_SIZE / WRITE_SIZE in
    rocprofv3 --pmc runs); nothing when mib is 0."""
    if not mib:
        return
    import torch
    src = torch.ones(mib * (1 << 20) // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def build_and_plan(args, g, sddmm, **opts):
    """The format (host builder, or the device builder from a CSR uploaded first) and the plan on
    it, with their wall times: upload_s (CSR to HBM), build_s, plan_s."""
    import numpy as np
    import torch
    import trspmm
    torch.zeros(1, device="cuda")   # HIP runtime start-up stays out of the timings
    torch.cuda.synchronize()
    pre = {"builder": args.builder}
    if args.builder == "device":
        t0 = time.time()
        csr = [torch.from_numpy(np.ascontiguousarray(a, dtype=dt)).cuda()
               for a, dt in ((g.rowptr, np.int32), (g.col, np.int32), (g.val, np.float32))]
        torch.cuda.synchronize()
        pre["upload_s"] = round(time.time() - t0, 4)
        fmt = trspmm.build_format_device(*csr)
        del csr
    else:
        fmt = trspmm.build_format(g.rowptr, g.col, g.val)
    pre["build_s"] = round(fmt.elapsed, 4)
    log(f"[bench] format built ({args.builder}) in {fmt.elapsed:.4f}s")
    t1 = time.time()
    plan = (trspmm.Plan.for_sddmm if sddmm else trspmm.Plan.from_format)(fmt, g.m, g.n, **opts)
    pre["plan_s"] = round(time.time() - t1, 4)
    pre["plan_lowering"] = "device" if plan.stats()["device_lowered"] else "host"
    del fmt
    return plan, pre


def bench_sddmm(args, workload, g, K):
    """Config 4: SDDMM out[e] = X[row_e] . Y[col_e] on the R-MAT pattern (hybrid tiling)."""
    import numpy as np
    import torch
    import trspmm
    from trspmm import _native as nat, graphs
    t0 = time.time()
    plan, pre = build_and_plan(args, g, True, xcd_split=args.xcd_split, host_lowering=args.host_lowering,
                               feature_lanes=args.feature_lanes, hot_rows=args.hot_rows,
                               split_dispatch=int(args.split_dispatch), sddmm_unroll=args.sddmm_unroll,
                               occupancy=args.occupancy)
    st = plan.stats()
    log(f"[bench] sddmm plan {st} ({time.time() - t0:.1f}s)")
    Xh = graphs.dense_operand(g.m, K, seed=4)
    Yh = graphs.dense_operand(g.n, K, seed=5)
    X = torch.from_numpy(Xh).cuda()
    Y = torch.from_numpy(Yh).cuda()
    out = torch.empty(st["nnz"], dtype=torch.float32, device="cuda")
    need = plan.sddmm_workspace_bytes(K)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    calibration_copy(args.calibrate_copy_mib)
    for _ in range(args.warmup):
        plan.sddmm(X, Y, out=out, workspace=ws)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        plan.sddmm(X, Y, out=out, workspace=ws)
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    flops = 2.0 * g.nnz * K
    gflops = flops / (ms_step * 1e-3) / 1e9
    ms = (ctypes.c_float * 2)()
    nat.check(nat.lib().trs_sddmm_f16_kernel_ms(plan.handle, X.data_ptr(), X.stride(0), Y.data_ptr(), Y.stride(0), K,
                                                out.data_ptr(), ws.data_ptr(), need,
                                                int(torch.cuda.current_stream().cuda_stream), 10, ms),
              "trs_sddmm_f16_kernel_ms")
    kms = launched(list(ms), [st["tasks"] > 0, st["mfma_tiles"] > 0])
    ms_cold = cold_ms(lambda: plan.sddmm(X, Y, out=out, workspace=ws), max(5, min(args.steps, 10)))
    names = ["sddmm_tasks", "sddmm_mfma"]
    dom = dominant(kms)
    M, N = g.m, g.n
    # compulsory bytes (column id + fp32 output per entry, row pointers, X and Y once) of the share
    # the dominant kernel computes; the layout's extra bytes are reported apart
    if dom == 0:
        nr = st["csr_nnz"]
        bytes_k = 8 * nr + 4 * (M + 1) + 2 * M * K + 2 * N * K
        impl = (4 * nr if st["mfma_tiles"] else 0) + 16 * st["tasks"]   # output index, task descriptors
        hot_bytes = 2 * K * st["hot_rows"] if need and K >= 128 and K % 8 == 0 else 0
        impl += 2 * hot_bytes                                           # staged hot rows: read + write
        impl += 3 * max(0, need - hot_bytes)                            # split-part merge: index, buffer, output (4 B each)
    else:
        bytes_k = 8 * st["mfma_nnz"] + 2 * M * K + 2 * N * K
        impl = st["mfma_tiles"] * (64 + 1024) - 4 * st["mfma_nnz"]      # column ids, dense output slots
    roof = roofline(bytes_k, impl, kms[dom], names[dom], names, kms, workload)
    roof["whole_step_frac"] = round((8 * g.nnz + 4 * (M + 1) + 2 * M * K + 2 * N * K) / (ms_step * 1e-3) / 1e9
                                    / HBM_PEAK_GBS, 4)
    outj = {"metric": f"SDDMM GFLOP/s (2·nnz·K) + % HBM roofline, R-MAT 2^20 pattern K={K} fp16", "value": round(gflops, 2),
            "unit": "GFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
            "config": {"workload": workload, "m": g.m, "n": g.n, "nnz": g.nnz, "K": K, "mfma_tiles": st["mfma_tiles"],
                       "mfma_nnz": st["mfma_nnz"], "parallelism": "none"},
            "roofline": roof, "preprocess": pre,
            "cold": {"ms_per_step": round(ms_cold, 5), "value": round(flops / (ms_cold * 1e-3) / 1e9, 2),
                     "note": "median step with a 1 GiB write before each (L2 and MALL flushed)"}}
    if not args.no_cpu_baseline:
        outj["cpu_baseline"] = cpu_baseline_sddmm(g, Xh, Yh, flops)
    print(json.dumps(outj), flush=True)


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on `workload` measured in an earlier rocprofv3 --pmc run
    (FETCH_SIZE and WRITE_SIZE, scaled by a device copy of known size) and the file they come from,
    or (None, None) where no counter run is recorded.  Never this run's measurement."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_pmc.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        d = json.load(f)
    src = f"{d.get('source', 'profiles/' + os.path.basename(path))} ({d.get('measured', 'earlier run')}; a separate " \
          "rocprofv3 --pmc run, not this one)"
    return d.get("hbm_bytes_per_launch"), src


def roofline(bytes_k: int, impl: int, ms: float, kernel: str, names, kms, workload: str) -> dict:
    """Roofline object of the dominant kernel: `achieved` = its compulsory bytes per launch over
    its HIP-event duration, `impl_bytes` = what its data layout reads or writes on top (not counted
    as achieved; negative where the layout reads less than the compulsory CSR bytes, as dense tiles
    with 2 bytes per slot and one column id per 16 slots do), `traffic` = measured HBM bytes per launch from the stored counter run named in
    `traffic_source` (null where none is recorded)."""
    achieved = bytes_k / (ms * 1e-3) / 1e9
    traffic, source = load_traffic(kernel, workload)
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": source,
            "alg_bytes": int(bytes_k), "impl_bytes": int(impl), "kernel": kernel, "kernel_ms": round(ms, 4),
            "kernel_ms_all": {n: None if v is None else round(v, 4) for n, v in zip(names, kms)}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 100 untimed steps by default: after the seconds of host-side graph and plan building the GPU
    # clocks need tens of milliseconds of work to ramp up (SDDMM K=64: 0.592 ms per step after 5
    # warm-up steps, 0.499 after 200; R-MAT SpMM K=128 unchanged at 0.969)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=2,
                    help="BASELINE configuration 1-5 (2: the headline); 6: dense 16x16 blocks only (not a "
                         "BASELINE configuration: the MFMA path on its own)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--k", type=int, default=0, help="override the configuration's feature width")
    ap.add_argument("--scramble", type=int, default=None, metavar="SEED",
                    help="relabel the graph's nodes with a random permutation first")
    ap.add_argument("--reorder", choices=["none", "tca", "tca-aligned"], default="none",
                    help="TCA row reorder before the builder (timed, reported under 'preprocess'); "
                         "tca-aligned keeps clusters inside 16-row windows")
    ap.add_argument("--builder", choices=["device", "host"], default="device",
                    help="format builder: on the GPU from the CSR uploaded to HBM (default), or the host "
                         "builder (the reference's CPU algorithm); both give the same format and plan")
    ap.add_argument("--host-lowering", action="store_true",
                    help="build the plan's residual on the host (default: on the device from the input CSR)")
    ap.add_argument("--feature-lanes", type=int, default=None,
                    help="plan option feature_lanes (lanes per lane group; fewer lanes = several feature passes)")
    ap.add_argument("--window-row-cap", type=int, default=None,
                    help="plan option window_row_cap (tiled windows with a longer residual row go back to the "
                         "residual kernel; default 128)")
    ap.add_argument("--xcd-split", type=int, default=None,
                    help="plan option xcd_split (rows of >= N residual entries cut by XCD column ranges; "
                         "-1 off; default: the library's)")
    ap.add_argument("--hot-rows", type=int, default=None,
                    help="plan option hot_rows (B / Y rows of the most gathered columns staged per call; -1 off; "
                         "default: the library's)")
    ap.add_argument("--sddmm-unroll", type=int, default=None,
                    help="plan option sddmm_unroll (SDDMM entries in flight per lane group: 4 or 8)")
    ap.add_argument("--occupancy", type=int, default=None,
                    help="plan option occupancy (residual task kernels held to N waves per SIMD; -1 uncapped)")
    ap.add_argument("--split-dispatch", action="store_true",
                    help="plan option split_dispatch: the XCD split part as its own launch (per-part profiles)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run one device copy of this many MiB first (counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (asked for {args.gpus}): this build has no multi-GPU path; "
              "row windows would shard across GPUs, with B all-gathered once per SpMM", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import trspmm
    from trspmm import graphs

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    t0 = time.time()
    workload, g, K, bseed = make_workload(args.config)
    if args.k:
        K = args.k
        workload = f"{workload.rsplit('_k', 1)[0]}_k{K}" if "_k" in workload else f"{workload}_k{K}"
    log(f"[bench] graph {workload}: m={g.m} nnz={g.nnz} ({time.time() - t0:.1f}s)")
    pre = {}
    if args.scramble is not None:
        g = scramble(g, args.scramble)
        workload += "_scrambled"
    if args.reorder != "none":
        g, pre["reorder_s"] = tca_reorder(g, 16 if args.reorder == "tca-aligned" else 0)
        workload += "_" + args.reorder.replace("-", "_")
        log(f"[bench] TCA reorder {pre['reorder_s']:.2f}s")
    if args.config == 4:
        bench_sddmm(args, workload, g, K)
        return
    t0 = time.time()
    plan, built = build_and_plan(args, g, False, xcd_split=args.xcd_split, host_lowering=args.host_lowering,
                                 window_row_cap=args.window_row_cap, feature_lanes=args.feature_lanes,
                                 hot_rows=args.hot_rows, split_dispatch=int(args.split_dispatch),
                                 occupancy=args.occupancy)
    pre.update(built)
    if "reorder_s" in pre:
        pre["reorder_s"] = round(pre["reorder_s"], 3)
    st = plan.stats()
    log(f"[bench] plan {st} ({time.time() - t0:.1f}s)")
    Bh = graphs.dense_operand(g.n, K, seed=bseed)
    B = torch.from_numpy(Bh).cuda()
    C = torch.empty((g.m, K), dtype=torch.float32, device="cuda")
    need = plan.workspace_bytes(K)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")

    calibration_copy(args.calibrate_copy_mib)
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
    kms = launched(kernel_ms(plan, B, C, ws, need), [st["tasks"] > 0, st["mfma_windows"] > 0, st["split_rows"] > 0])
    names = ["spmm_tasks", "spmm_mfma_win", "spmm_fixup"]
    dom = dominant(kms)
    M, N = g.m, g.n
    rows_w = min(M, 16 * st["mfma_windows"])
    nnz_w = st["window_csr_nnz"]
    # compulsory bytes (fp16 value + int32 column per entry, int32 row pointers, B once, C once) of
    # the share the dominant kernel computes; bytes its data layout adds are reported apart
    if dom == 0:    # residual tasks: entries and rows outside MFMA windows
        nnz_k = st["csr_nnz"] - nnz_w
        rows_k = M - rows_w
        bytes_k = 6 * nnz_k + 4 * (rows_k + 1) + 2 * N * K + 4 * rows_k * K
        impl = 16 * st["tasks"] + 4 * K * st["partial_slots"]          # task descriptors, partial slots
        impl += 4 * K * st["hot_rows"] if K >= 128 and K % 8 == 0 else 0  # staged hot rows: read + write
    elif dom == 1:  # MFMA windows: tile entries + the windows' residual entries, their rows
        bytes_k = 6 * (st["mfma_nnz"] + nnz_w) + 4 * (rows_w + 1) + 2 * N * K + 4 * rows_w * K
        impl = st["mfma_tiles"] * (512 + 64) - 6 * st["mfma_nnz"]      # dense 16x16 tiles + column ids
    else:           # fixup: the split rows it writes
        bytes_k = 4 * st["split_rows"] * K
        impl = 4 * K * st["partial_slots"]
    roof = roofline(bytes_k, impl, kms[dom], names[dom], names, kms, workload)
    roof["whole_step_frac"] = round((6 * g.nnz + 4 * (M + 1) + 2 * N * K + 4 * M * K) / (ms_step * 1e-3) / 1e9
                                    / HBM_PEAK_GBS, 4)
    log(f"[bench] kernels {kms}, roofline {roof}")
    ms_cold = cold_ms(lambda: plan.spmm(B, out=C, workspace=ws), max(5, min(args.steps, 10)))
    log(f"[bench] cold (L2 + MALL flushed) {ms_cold:.4f} ms/step")
    ms_pcie = pcie_inclusive_ms(plan, Bh, C, ws)
    log(f"[bench] host-to-host (B in, C out over PCIe) {ms_pcie:.3f} ms/step")

    metric = METRIC if args.config == 2 and K == 128 else OTHER_METRIC.format(workload=workload)
    out = {"metric": metric, "value": round(gflops, 2), "unit": "GFLOP/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f16", "data": "synthetic",
           "config": {"workload": workload, "m": g.m, "n": g.n, "nnz": g.nnz, "K": K,
                      "mfma_tiles": st["mfma_tiles"], "mfma_nnz": st["mfma_nnz"], "parallelism": "none"},
           "roofline": roof, "preprocess": pre,
           "cold": {"ms_per_step": round(ms_cold, 5), "value": round(flops / (ms_cold * 1e-3) / 1e9, 2),
                    "note": "median step with a 1 GiB write before each (L2 and MALL flushed)"},
           "host_to_host": {"ms_per_step": round(ms_pcie, 4), "value": round(flops / (ms_pcie * 1e-3) / 1e9, 2),
                            "note": "B from pinned host memory, SpMM, C to pinned host memory (not `value`)"}}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(g, Bh, flops)
        log(f"[bench] cpu baseline {out['cpu_baseline']}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
