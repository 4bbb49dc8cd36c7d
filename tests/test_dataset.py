"""Format cache files and the dataset layer (tr_csr_fp16), on the CPU.

The dataset class is the reference harness's caller of the builder
(spmm/tr_csr_fp16/mdataset2_online.py:29-167); its arrays must equal the drop-in builder's output
on the same CSR and values, which the golden fixtures pin to the reference builder.
"""
import os

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import trspmm
from trspmm import graphs, _native as nat
from conftest import same_array, load_golden, golden_files


def _format(seed=3):
    g = graphs.random_csr(700, 650, 0.02, seed=seed)
    return g, trspmm.build_format(g.rowptr, g.col, g.val)


def _same_format(a, b, same_build=True):
    for i in range(32):
        assert same_array(a.slot(i), b.slot(i)), i
    assert (a.window, a.rows, a.canonical) == (b.window, b.rows, b.canonical)
    if same_build:                              # the build time travels with the file
        assert a.elapsed == b.elapsed


def test_format_file_round_trip(tmp_path):
    g, f = _format()
    p = tmp_path / "f.trsf"
    f.save(p)
    _same_format(f, trspmm.Format.load(p))
    assert not os.path.exists(str(p) + ".tmp")


@pytest.mark.parametrize("path", golden_files()[:3], ids=os.path.basename)
def test_format_file_round_trip_golden(path, tmp_path, golden_env):
    rowptr, col, val, params, env, outs = load_golden(path)
    golden_env(env)
    f = trspmm.build_format(rowptr, col, val, **params)
    f.save(tmp_path / "g.trsf")
    h = trspmm.Format.load(tmp_path / "g.trsf")
    for i, (a, b) in enumerate(zip(h.arrays(), outs)):
        assert same_array(a, b), i


def test_format_file_rejects_damage(tmp_path):
    g, f = _format()
    p = tmp_path / "f.trsf"
    f.save(p)
    raw = p.read_bytes()
    cases = {
        "missing": None,
        "truncated": raw[:-9],
        "short": raw[:40],
        "magic": b"X" + raw[1:],
        "flipped": raw[:500] + bytes([raw[500] ^ 1]) + raw[501:],
        "extended": raw + b"\0" * 8,
    }
    for name, data in cases.items():
        q = tmp_path / f"{name}.trsf"
        if data is not None:
            q.write_bytes(data)
        with pytest.raises(nat.TrsError) as e:
            trspmm.Format.load(q)
        assert e.value.code == 6, name          # TRS_EIO


def test_build_format_cached(tmp_path, monkeypatch):
    monkeypatch.delenv("LIBRA_SKIP_TC", raising=False)
    g = graphs.random_csr(500, 480, 0.03, seed=5)
    a = trspmm.build_format_cached(g.rowptr, g.col, g.val, tmp_path, density=4)
    assert a.from_cache is False and len(list(tmp_path.iterdir())) == 1
    b = trspmm.build_format_cached(g.rowptr, g.col, g.val, tmp_path, density=4)
    assert b.from_cache is True
    _same_format(a, b)
    c = trspmm.build_format_cached(g.rowptr, g.col, g.val, tmp_path, density=8)   # other parameters
    assert c.from_cache is False
    monkeypatch.setenv("LIBRA_SKIP_TC", "1")                                       # other environment
    d = trspmm.build_format_cached(g.rowptr, g.col, g.val, tmp_path, density=4)
    assert d.from_cache is False and d.slot(0).shape[0] == 1                       # no TC parts
    val2 = g.val.copy()
    val2[0] += 1.0
    e = trspmm.build_format_cached(g.rowptr, g.col, val2, tmp_path, density=4)     # other values
    assert e.from_cache is False
    # a damaged cache entry is rebuilt and replaced
    monkeypatch.delenv("LIBRA_SKIP_TC")
    key = trspmm.ops.format_cache_key(g.rowptr, g.col, g.val, density=4)[:40]
    path = tmp_path / f"format-{key}.trsf"
    path.write_bytes(path.read_bytes()[:-3])
    f = trspmm.build_format_cached(g.rowptr, g.col, g.val, tmp_path, density=4)
    assert f.from_cache is False
    _same_format(a, trspmm.Format.load(path), same_build=False)


def _write_dataset(tmp_path, nodes=1000, dst_nodes=1000, edges=9000, seed=11):
    rng = np.random.default_rng(seed)
    src = rng.integers(0, nodes, size=edges)
    dst = rng.integers(0, dst_nodes, size=edges)
    # a few dense 16-row blocks so every share of the format is exercised
    blk = np.arange(64)
    src = np.concatenate([src, np.repeat(blk, 16)])
    dst = np.concatenate([dst, np.tile(np.arange(100, 116), 64)])
    d = tmp_path / "graphs"
    d.mkdir(exist_ok=True)
    np.savez(d / "toy.npz", src_li=src, dst_li=dst, num_nodes_src=np.int64(nodes), num_nodes_dst=np.int64(dst_nodes))
    return src, dst


ARGS = dict(dimN=32, density=8, partsize_t=32, partsize_c=32, shortsize=3, window=16, wide=16)


def _dataset(**kw):
    from tr_csr_fp16.mdataset2_online import GCN_dataset_tcu_sptc_cuda_online
    a = dict(ARGS, **kw)
    return GCN_dataset_tcu_sptc_cuda_online("toy", a["dimN"], a["density"], a["partsize_t"], a["partsize_c"],
                                            a["shortsize"], "graphs", a["window"], a["wide"])


def test_dataset_matches_reference_pipeline(tmp_path, monkeypatch):
    import Libra5BlockOnline
    src, dst = _write_dataset(tmp_path, nodes=1000)
    monkeypatch.setenv("TR_DATA_ROOT", str(tmp_path))
    monkeypatch.delenv("TR_FORMAT_CACHE", raising=False)
    monkeypatch.delenv("LIBRA_TCA_REORDER", raising=False)
    torch.manual_seed(0)
    ds = _dataset()
    assert ds.num_nodes_ori == 1000 and ds.num_nodes == 1008 and ds.num_nodes_dst == 1000
    # CSR as the reference builds it: scipy COO -> CSR of the padded shape (duplicates merged)
    ref = sp.coo_matrix((np.ones(len(src)), (src, dst)), shape=(1008, 1000)).tocsr()
    ref.sort_indices()
    assert np.array_equal(ds.row_pointers.numpy(), ref.indptr) and np.array_equal(ds.column_index.numpy(), ref.indices)
    assert ds.degrees.shape == (ref.nnz,) and ds.num_edges == ref.nnz
    out = Libra5BlockOnline.block_sptc_2to4_online(ds.row_pointers, ds.column_index, ds.degrees, 32, 32, 3, 8, 16, 16,
                                                   0.0, 0.5, 12)
    names = ["t_rowNew_offsetTensor", "t_blockTensor", "t_columnTensor", "t_valueTensor", "t_window_rowTensor",
             "t_atomicTensor", "t_binaryTensor", "c_row_offsetTensor", "c_rowTensor", "c_atomicTensor",
             "c_colTensor", "c_valueTensor", "c_row_offsetTensor_short", "c_rowTensor_short",
             "c_atomicTensor_short", "c_colTensor_short", "c_valueTensor_short", "s_columnTensor",
             "s_maskTensor", "s_valueTensor", "s_posTensor", "s_windowTensor", "s_offsetTensor",
             "s_tile_windowTensor", "s_tile_groupTensor", "s_tile_columnTensor", "s_packed_aTensor",
             "s_packed_metaTensor", "s_window_tile_offsetTensor"]
    half = {"t_valueTensor", "c_valueTensor", "c_valueTensor_short"}
    for i, name in enumerate(names):
        got = getattr(ds, name)
        want = out[i].half() if name in half else out[i]
        assert got.dtype == want.dtype and torch.equal(got, want), name
    assert ds.duration.dtype == torch.float64 and ds.duration.dim() == 0
    assert ds.t_valueTensor.numel() > 0 and ds.s_columnTensor.shape[0] > 0
    assert ds.c_colTensor.numel() + ds.c_colTensor_short.numel() > 0
    assert (ds.parts_t, ds.parts_c, ds.parts_c_short) == (out[5].shape[0], out[9].shape[0], out[14].shape[0])
    assert ds.x.shape == (1000, 32) and ds.x.dtype == torch.float16
    assert ds.format_from_cache is False


def test_dataset_format_cache(tmp_path, monkeypatch):
    _write_dataset(tmp_path)
    monkeypatch.setenv("TR_DATA_ROOT", str(tmp_path))
    monkeypatch.setenv("TR_FORMAT_CACHE", str(tmp_path / "cache"))
    monkeypatch.delenv("LIBRA_TCA_REORDER", raising=False)
    torch.manual_seed(1)
    a = _dataset()
    torch.manual_seed(1)
    b = _dataset()
    assert a.format_from_cache is False and b.format_from_cache is True
    for name in ("t_binaryTensor", "c_valueTensor", "s_packed_aTensor", "s_valueTensor", "duration"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    torch.manual_seed(2)                       # other values: another cache entry
    c = _dataset()
    assert c.format_from_cache is False


def test_dataset_paths(tmp_path, monkeypatch):
    from tr_csr_fp16 import tr_paths
    monkeypatch.setenv("TR_DATA_ROOT", str(tmp_path))
    assert tr_paths.dataset_path("graphs", "toy") == (tmp_path / "graphs" / "toy.npz").resolve()
    assert tr_paths.dataset_path(str(tmp_path / "x"), "toy") == (tmp_path / "x" / "toy.npz").resolve()
    with pytest.raises(FileNotFoundError, match="missing"):
        tr_paths.load_graph_npz("graphs", "missing")
    monkeypatch.setenv("TR_RESULTS_DIR", str(tmp_path / "res"))
    p = tr_paths.result_path("a", "b.csv")
    assert p.parent.is_dir() and p.name == "b.csv"


def test_dataset_with_tca_reorder(tmp_path, monkeypatch):
    """LIBRA_TCA_REORDER=1: rows are permuted before the builder (mdataset2_online.py:72-95);
    the padded rows stay last and every row keeps its column set."""
    src, dst = _write_dataset(tmp_path, nodes=1000)
    monkeypatch.setenv("TR_DATA_ROOT", str(tmp_path))
    monkeypatch.delenv("TR_FORMAT_CACHE", raising=False)
    monkeypatch.setenv("LIBRA_TCA_REORDER", "1")
    torch.manual_seed(0)
    ds = _dataset()
    order = ds.reorder_id
    assert order is not None and np.array_equal(np.sort(order), np.arange(1000))
    ref = sp.coo_matrix((np.ones(len(src)), (src, dst)), shape=(1008, 1000)).tocsr()
    ref.sort_indices()
    rp, ci = ds.row_pointers.numpy(), ds.column_index.numpy()
    assert rp.shape == (1009,) and rp[-1] == ref.nnz and np.all(rp[1001:] == rp[1000])
    for k in range(0, 1000, 37):
        assert np.array_equal(ci[rp[k]:rp[k + 1]], ref.indices[ref.indptr[order[k]]:ref.indptr[order[k] + 1]])
    assert ds.edge_index.shape == (2, ref.nnz)
