"""GPU parity of the drop-in operator module Libra6SpMMOnline (reference signatures, CPU tensors
in and out) against the oracle's reading of the same arrays."""
import numpy as np
import pytest
import torch

from oracle import spmm as osp
from trspmm import graphs

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def harness_inputs(g, dimN, seed):
    """What the reference dataset layer hands the operator (mdataset2_online.py:100-167):
    builder tuple with t/c values cast to fp16, rhs fp16 [kOri, dimN]."""
    import Libra5BlockOnline as L5
    out = L5.block_sptc_2to4_online_with_spill(torch.from_numpy(g.rowptr), torch.from_numpy(g.col),
                                               torch.from_numpy(g.val), 32, 32, 3, 8, 16, 16, 0.0, 0.5, 12)
    t = list(out)
    t[3] = t[3].half()
    t[11] = t[11].half()
    t[16] = t[16].half()
    x = torch.from_numpy(graphs.dense_operand(g.n, dimN, seed))
    return t, x


def parallel_call(t, x, g, epoches=3, spill=False):
    import Libra6SpMMOnline as L6
    kw = dict(spill_row=t[30], spill_col=t[31], spill_val=t[32]) if spill else {}
    return L6.forward_fp16_tcu_cuda_sptc_mma_parallel_online(
        t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8], t[9], t[10], t[11], t[12], t[13], t[14], t[15], t[16],
        t[17], t[19], t[20], t[22], t[23], t[25], t[26], t[27], t[28], x,
        t[5].shape[0], t[9].shape[0], 32, t[14].shape[0], 16, x.shape[1], g.m, g.n, epoches, **kw)


def format_reference(t, g, x, with_spill):
    """Oracle reading of the arrays, fp16 values as the operator receives them (t/c already fp16,
    s_value rounded to fp16 as the packed tiles carry it)."""
    arrs = [a.numpy() if a.dtype != torch.float16 else a.float().numpy() for a in t[:29]]
    arrs[19] = arrs[19].astype(np.float16).astype(np.float32)
    spill = (t[30].numpy(), t[31].numpy(), t[32].numpy().astype(np.float16).astype(np.float32)) if with_spill else None
    r, c, v = osp.format_to_coo(arrs, spill)
    return osp.coo_spmm(r, c, v, x.numpy().astype(np.float64), g.m)


@pytest.mark.parametrize("name,gen,dimN", [
    ("er", lambda: graphs.erdos_renyi_gcn(nodes=2048, edges=16384), 64),
    ("sbm", lambda: graphs.sbm(communities=512, seed=2, val_seed=3), 128),
    ("rmat", lambda: graphs.rmat(scale=12, edge_factor=16, seed=3), 128),
])
def test_parallel_operator(name, gen, dimN):
    say("parallel", name)
    g = gen()
    t, x = harness_inputs(g, dimN, seed=1)
    res = parallel_call(t, x, g)
    assert len(res) == 6 and res[0].shape == (g.m, dimN) and res[0].dtype == torch.float32 and not res[0].is_cuda
    assert float(res[1]) > 0
    e = osp.spmm_error(res[0].numpy(), format_reference(t, g, x, False))
    assert e["elementwise_ok"], e
    # with the spill the hybrid result is the full CSR SpMM
    res = parallel_call(t, x, g, spill=True)
    e = osp.spmm_error(res[0].numpy(), osp.csr_spmm(g.rowptr, g.col, g.val, x.numpy(), m=g.m))
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e


def test_sptc_operators():
    import Libra6SpMMOnline as L6
    g = graphs.sbm(communities=256, seed=5, val_seed=6)
    t, x = harness_inputs(g, 64, seed=2)
    w = 16
    ref_groups = osp.coo_spmm(*osp.format_to_coo(
        [np.zeros(1, np.int32)] + [np.zeros(0)] * 6 + [np.zeros(1, np.int32)] + [np.zeros(0)] * 4 +
        [np.zeros(1, np.int32)] + [np.zeros(0)] * 4 + [a.numpy() for a in t[17:29]], None, w),
        x.numpy().astype(np.float64), g.m)
    out, ms = L6.forward_fp16_sptc_online(t[17], t[19], t[20], t[21], x, w, 64, g.m, g.n, 2)
    assert osp.spmm_error(out.numpy(), ref_groups)["elementwise_ok"]
    out, ms = L6.forward_fp16_sptc_mma_online(t[17], t[19], t[20], t[22], x, w, 64, g.m, g.n, 2)
    assert osp.spmm_error(out.numpy(), ref_groups)["elementwise_ok"]
    r, c, v = osp.packed_to_coo(t[25].numpy(), t[26].numpy(), t[27].numpy(), t[28].numpy(), w)
    ref_packed = osp.coo_spmm(r, c, v, x.numpy().astype(np.float64), g.m)
    out, ms = L6.forward_fp16_sptc_mma_packed_online(t[25], t[26], t[27], t[28], x, w, 64, g.m, g.n, 2)
    e = osp.spmm_error(out.numpy(), ref_packed)
    assert e["elementwise_ok"], e
    assert float(ms) > 0


def test_operator_argument_errors():
    import Libra6SpMMOnline as L6
    g = graphs.random_csr(64, 64, 0.1, seed=1)
    t, x = harness_inputs(g, 32, seed=1)
    with pytest.raises(RuntimeError, match="window"):
        L6.forward_fp16_sptc_mma_packed_online(t[25], t[26], t[27], t[28], x, 17, 32, g.m, g.n, 1)
    with pytest.raises(RuntimeError, match="kOri"):
        L6.forward_fp16_sptc_mma_packed_online(t[25], t[26], t[27], t[28], x, 16, 32, g.m, g.n + 1, 1)
    with pytest.raises(RuntimeError, match="dtype"):
        L6.forward_fp16_sptc_online(t[17], t[19].double(), t[20], t[21], x, 16, 32, g.m, g.n, 1)
    with pytest.raises(RuntimeError, match="CPU"):
        L6.forward_fp16_sptc_mma_packed_online(t[25].cuda(), t[26], t[27], t[28], x, 16, 32, g.m, g.n, 1)


def test_reference_harness_flow_through_dataset(tmp_path, monkeypatch):
    """spmm/tr_csr_fp16/test_tr_csr_online.py:77-152 on top of this library: dataset class ->
    parallel operator with the dataset's attributes, checked against the oracle's reading of the
    same arrays, and with the dataset's spill against the full CSR SpMM."""
    import Libra6SpMMOnline as L6
    from tr_csr_fp16.mdataset2_online import GCN_dataset_tcu_sptc_cuda_online
    say("harness flow")
    g = graphs.sbm(communities=300, seed=7, val_seed=8)
    rows = np.repeat(np.arange(g.m_pad), np.diff(g.rowptr))
    (tmp_path / "d").mkdir()
    np.savez(tmp_path / "d" / "sbm.npz", src_li=rows, dst_li=g.col.astype(np.int64),
             num_nodes_src=np.int64(g.m), num_nodes_dst=np.int64(g.n))
    monkeypatch.setenv("TR_DATA_ROOT", str(tmp_path))
    monkeypatch.delenv("TR_FORMAT_CACHE", raising=False)
    monkeypatch.delenv("LIBRA_TCA_REORDER", raising=False)
    torch.manual_seed(3)
    d = GCN_dataset_tcu_sptc_cuda_online("sbm", 64, 8, 32, 32, 3, "d", 16, 16)
    args = (d.t_rowNew_offsetTensor, d.t_blockTensor, d.t_columnTensor, d.t_valueTensor, d.t_window_rowTensor,
            d.t_atomicTensor, d.t_binaryTensor, d.c_row_offsetTensor, d.c_rowTensor, d.c_atomicTensor,
            d.c_colTensor, d.c_valueTensor, d.c_row_offsetTensor_short, d.c_rowTensor_short,
            d.c_atomicTensor_short, d.c_colTensor_short, d.c_valueTensor_short, d.s_columnTensor,
            d.s_valueTensor, d.s_posTensor, d.s_offsetTensor, d.s_tile_windowTensor, d.s_tile_columnTensor,
            d.s_packed_aTensor, d.s_packed_metaTensor, d.s_window_tile_offsetTensor, d.x,
            d.parts_t, d.parts_c, d.partsize_c, d.parts_c_short, d.window, d.x.size(1), d.num_nodes_ori,
            d.num_nodes_dst, 3)
    out, ms, tc, cl, cs, sp = L6.forward_fp16_tcu_cuda_sptc_mma_parallel_online(*args)
    assert out.shape == (g.m, 64) and float(ms) > 0
    # per-path completion times from the common start (mGCNkernel_online.cu:1676-1687), paths in
    # launch order residual -> MFMA windows -> fixups
    tc, cl, cs, sp = float(tc), float(cl), float(cs), float(sp)
    assert 0 < cl <= tc <= cs and sp == tc, (float(ms), tc, cl, cs, sp)
    t = [getattr(d, n) for n in ("t_rowNew_offsetTensor", "t_blockTensor", "t_columnTensor", "t_valueTensor",
                                 "t_window_rowTensor", "t_atomicTensor", "t_binaryTensor", "c_row_offsetTensor",
                                 "c_rowTensor", "c_atomicTensor", "c_colTensor", "c_valueTensor",
                                 "c_row_offsetTensor_short", "c_rowTensor_short", "c_atomicTensor_short",
                                 "c_colTensor_short", "c_valueTensor_short", "s_columnTensor", "s_maskTensor",
                                 "s_valueTensor", "s_posTensor", "s_windowTensor", "s_offsetTensor",
                                 "s_tile_windowTensor", "s_tile_groupTensor", "s_tile_columnTensor",
                                 "s_packed_aTensor", "s_packed_metaTensor", "s_window_tile_offsetTensor")]
    e = osp.spmm_error(out.numpy(), format_reference(t, g, d.x, False))
    assert e["elementwise_ok"], e
    sr, sc, sv = (torch.from_numpy(a) for a in d.spill)
    full = L6.forward_fp16_tcu_cuda_sptc_mma_parallel_online(*args, spill_row=sr, spill_col=sc, spill_val=sv)[0]
    vals16 = d.degrees.numpy().astype(np.float16).astype(np.float32)   # the operator computes in fp16
    e = osp.spmm_error(full.numpy(), osp.csr_spmm(d.row_pointers.numpy(), d.column_index.numpy(), vals16,
                                                  d.x.numpy(), m=g.m))
    assert e["elementwise_ok"] and e["max_rel_to_max"] <= 1e-2, e


def test_skip_tc_kernel_switch(monkeypatch):
    """LIBRA_SKIP_TC_KERNEL=1 leaves the TC share out, as the reference's debug switch skips its TC
    kernel (mGCNkernel_online.cu:1397-1410): the result is the SpMM of every other share."""
    say("skip tc kernel")
    g = graphs.sbm(communities=512, seed=2, val_seed=3)
    t, x = harness_inputs(g, 64, seed=4)
    arrs = [a.numpy() if a.dtype != torch.float16 else a.float().numpy() for a in t[:29]]
    tr, tcol, tv = [], [], []
    osp._tc_to_coo(arrs, tr, tcol, tv)
    assert len(tr) > 0
    full = format_reference(t, g, x, False)
    tc_only = osp.coo_spmm(np.asarray(tr), np.asarray(tcol), np.asarray(tv), x.numpy().astype(np.float64), g.m)
    monkeypatch.setenv("LIBRA_SKIP_TC_KERNEL", "1")
    res = parallel_call(t, x, g)
    e = osp.spmm_error(res[0].numpy(), full - tc_only)
    assert e["elementwise_ok"], e
    monkeypatch.setenv("LIBRA_SKIP_TC_KERNEL", "yes")   # only 1 / true / TRUE switch it on
    res = parallel_call(t, x, g)
    assert osp.spmm_error(res[0].numpy(), full)["elementwise_ok"]
