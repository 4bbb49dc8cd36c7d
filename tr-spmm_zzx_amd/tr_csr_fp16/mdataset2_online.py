"""GCN_dataset_tcu_sptc_cuda_online: the caller of the format builder in the reference harness
(spmm/tr_csr_fp16/mdataset2_online.py:29-167), same constructor, attributes and dtypes.

Steps (reference lines in brackets):
  1. load ``<data_path>/<data>.npz`` (src_li, dst_li, num_nodes_src, num_nodes_dst) [:51, tr_paths]
  2. pad the row count to a multiple of ``window``; CSR of the (deduplicated) edge list [:58-70]
  3. optional row reorder when LIBRA_TCA_REORDER=1 (native TCA clustering, trspmm.reorder) [:72-95]
  4. values ``torch.randn(num_edges)`` (seed torch for reproducible runs) [:98]
  5. builder (trspmm.build_format: bit-exact with block_sptc_2to4_online) -> the 30 attributes,
     part counts, fp16 value tensors [:100-159]
  6. ``x = randn(num_nodes_dst, dimN).half()`` [:165-167]
The reference's Rabbit call (:96) rewrites only ``edge_index``, which nothing downstream reads; it
is omitted.  Addition: when TR_FORMAT_CACHE names a directory, step 5 reads the format from a
cache file keyed by the CSR, its values and the builder parameters, or writes it there
(``self.format_from_cache`` tells which).
"""
from __future__ import annotations

import os

import numpy as np
import torch

import trspmm

from .tr_paths import load_graph_npz

_ATTRS = [
    "t_rowNew_offsetTensor", "t_blockTensor", "t_columnTensor", "t_valueTensor", "t_window_rowTensor",
    "t_atomicTensor", "t_binaryTensor",
    "c_row_offsetTensor", "c_rowTensor", "c_atomicTensor", "c_colTensor", "c_valueTensor",
    "c_row_offsetTensor_short", "c_rowTensor_short", "c_atomicTensor_short", "c_colTensor_short",
    "c_valueTensor_short",
    "s_columnTensor", "s_maskTensor", "s_valueTensor", "s_posTensor", "s_windowTensor", "s_offsetTensor",
    "s_tile_windowTensor", "s_tile_groupTensor", "s_tile_columnTensor", "s_packed_aTensor",
    "s_packed_metaTensor", "s_window_tile_offsetTensor", "duration",
]


def csr_of_edges(src: np.ndarray, dst: np.ndarray, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """Canonical CSR (sorted, duplicates merged) of an edge list, rows x cols; int32 arrays."""
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    if src.shape != dst.shape:
        raise ValueError("src_li and dst_li differ in length")
    if src.size and (src.min() < 0 or src.max() >= rows or dst.min() < 0 or dst.max() >= cols):
        raise ValueError("edge endpoint outside the node range")
    keys = np.unique(src * cols + dst)
    counts = np.bincount(keys // cols, minlength=rows)
    indptr = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    return indptr.astype(np.int32), (keys % cols).astype(np.int32)


class GCN_dataset_tcu_sptc_cuda_online(torch.nn.Module):
    """Hybrid split of a graph: dense TC blocks, 2:4 groups and residual rows, plus features."""

    def __init__(self, data, dimN, density, partsize_t, partsize_c, shortsize, data_path, window, wide,
                 tc_min_util=0.0, sptc_min_util=0.50, sptc_threshold=12):
        super().__init__()
        self.graph = load_graph_npz(data_path, data)
        self.num_features = dimN
        self.window = window
        self.init_edges(density, partsize_t, partsize_c, shortsize, window, wide, tc_min_util, sptc_min_util,
                        sptc_threshold)
        self.init_embedding()

    def init_edges(self, density, partsize_t, partsize_c, shortsize, window, wide, tc_min_util, sptc_min_util,
                   sptc_threshold):
        self.num_nodes_ori = int(self.graph["num_nodes_src"])
        self.num_nodes_dst = int(self.graph["num_nodes_dst"])
        self.num_nodes = self.num_nodes_ori
        if self.num_nodes_ori % window != 0:
            self.num_nodes = self.num_nodes_ori + window - self.num_nodes_ori % window
        src_li = np.asarray(self.graph["src_li"])
        dst_li = np.asarray(self.graph["dst_li"])
        self.edge_index = np.stack([src_li, dst_li])
        indptr, indices = csr_of_edges(src_li, dst_li, self.num_nodes, self.num_nodes_dst)

        self.reorder_id = None
        if os.environ.get("LIBRA_TCA_REORDER", "0") == "1":
            from trspmm import reorder
            new_ptr, new_idx, order = reorder.apply_tca_reorder(indptr, indices, self.num_nodes_ori, thres=16)
            # rows past num_nodes_ori are padding (empty): keep them at the end
            indptr = np.concatenate([new_ptr, np.full(self.num_nodes - self.num_nodes_ori, new_ptr[-1],
                                                      dtype=np.int32)])
            indices = new_idx
            rows = np.repeat(np.arange(self.num_nodes, dtype=np.int64), np.diff(indptr))
            self.edge_index = np.stack([rows, indices.astype(np.int64)])
            self.reorder_id = order
        else:
            print("TCA reorder disabled (LIBRA_TCA_REORDER=0)")

        self.column_index = torch.from_numpy(np.ascontiguousarray(indices, dtype=np.int32))
        self.row_pointers = torch.from_numpy(np.ascontiguousarray(indptr, dtype=np.int32))
        self.num_edges = self.column_index.numel()
        self.degrees = torch.randn(self.num_edges)

        params = dict(part_t=int(partsize_t), part_c=int(partsize_c), short_size=int(shortsize),
                      density=int(density), window=int(window), wide=int(wide), tc_min_util=float(tc_min_util),
                      sptc_min_util=float(sptc_min_util), sptc_threshold=int(sptc_threshold))
        rp, ci, va = self.row_pointers.numpy(), self.column_index.numpy(), self.degrees.numpy()
        cache = os.environ.get("TR_FORMAT_CACHE")
        if cache:
            fmt = trspmm.build_format_cached(rp, ci, va, cache, **params)
            self.format_from_cache = fmt.from_cache
        else:
            fmt = trspmm.build_format(rp, ci, va, **params)
            self.format_from_cache = False
        for name, t in zip(_ATTRS, fmt.tensors()):
            setattr(self, name, t)
        self.spill = fmt.spill()   # entries the 2:4 step drops (not part of the reference output)

        self.parts_t = self.t_atomicTensor.shape[0]
        self.parts_c = self.c_atomicTensor.shape[0]
        self.parts_c_short = self.c_atomicTensor_short.shape[0]
        self.partsize_c = partsize_c

        self.t_valueTensor = self.t_valueTensor.half()
        self.c_valueTensor = self.c_valueTensor.half()
        self.c_valueTensor_short = self.c_valueTensor_short.half()

        tcu_nnz = self.t_valueTensor.numel()
        sptc_nnz = int((self.s_posTensor >= 0).sum().item())
        cuda_nnz = self.c_valueTensor.numel() + self.c_valueTensor_short.numel()
        print(f"tcu: {tcu_nnz};   sptc: {sptc_nnz};   cuda: {cuda_nnz}")
        print(f"parts_t: {self.parts_t};   parts_c: {self.parts_c};   parts_c_short: {self.parts_c_short};   "
              f"sptc_groups: {self.s_columnTensor.shape[0]};   sptc_tiles: {self.s_tile_windowTensor.shape[0]}")

    def init_embedding(self):
        self.x = torch.randn(self.num_nodes_dst, self.num_features).half()
