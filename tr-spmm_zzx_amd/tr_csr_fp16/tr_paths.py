"""Dataset and result locations (interface of spmm/tr_csr_fp16/tr_paths.py:7-59).

Environment: TR_ROOT (project root; default: the repository root), TR_DATA_ROOT (datasets;
default <root>/dgl_dataset), TR_DATA_CSV (dataset index file), TR_RESULTS_DIR (default <root>/res).
A dataset ``data`` under ``data_path`` is the file ``<data_path>/<data>.npz`` holding src_li,
dst_li, num_nodes_src and num_nodes_dst; relative ``data_path`` values resolve under the data root.
"""
from __future__ import annotations

import os
from pathlib import Path

import numpy as np

_REPO = Path(__file__).resolve().parents[2]


def project_root() -> Path:
    return Path(os.environ.get("TR_ROOT", _REPO)).resolve()


def data_root() -> Path:
    return Path(os.environ.get("TR_DATA_ROOT", project_root() / "dgl_dataset")).resolve()


def dataset_path(data_path: str, data: str) -> Path:
    base = Path(data_path)
    if not base.is_absolute():
        base = data_root() / base
    return (base / f"{data}.npz").resolve()


def load_graph_npz(data_path: str, data: str):
    """The dataset's arrays (np.load without pickles). FileNotFoundError names the path tried."""
    path = dataset_path(data_path, data)
    if not path.exists():
        raise FileNotFoundError(f"dataset '{data}' not found at {path} (set TR_DATA_ROOT)")
    return np.load(path, allow_pickle=False)


def index_csv(default_name: str = "data_filter.csv") -> Path:
    explicit = os.environ.get("TR_DATA_CSV")
    if explicit:
        return Path(explicit).resolve()
    root = project_root()
    names = [default_name, "data_filter.csv", "data.csv"]
    for name in names:
        if (root / name).exists():
            return (root / name).resolve()
    return (root / default_name).resolve()


def results_root() -> Path:
    path = Path(os.environ.get("TR_RESULTS_DIR", project_root() / "res")).resolve()
    path.mkdir(parents=True, exist_ok=True)
    return path


def result_path(*parts: str) -> Path:
    path = results_root().joinpath(*parts)
    path.parent.mkdir(parents=True, exist_ok=True)
    return path
