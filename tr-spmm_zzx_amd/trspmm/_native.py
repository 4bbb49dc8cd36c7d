"""Loader and ctypes prototypes for the C ABI in include/trspmm.h (libtrspmm.so).

torch is imported before the library is opened: the HIP runtime torch ships and /opt/rocm's share
the SONAME ``libamdhip64.so.7``, so opening the library after torch binds it to the runtime torch
already loaded (one HIP runtime per process; streams and device pointers are interchangeable).
The library must exist: there is no CPU fallback, a missing build raises ``ImportError``.
"""
from __future__ import annotations

import ctypes
import importlib
import os

import torch  # noqa: F401  (must precede the library, see module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtrspmm.so")

c_i32, c_i64, c_f32, c_f64, c_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_void_p
c_pp = ctypes.POINTER(ctypes.c_void_p)


class BuildParams(ctypes.Structure):
    _fields_ = [("struct_size", c_i32), ("part_size_t", c_i32), ("part_size_c", c_i32), ("short_size", c_i32), ("density", c_i32),
                ("window", c_i32), ("wide", c_i32), ("tc_min_util", c_f32), ("sptc_min_util", c_f32),
                ("sptc_threshold", c_i32), ("skip_tc", c_i32), ("sptc_unit_min_nnz", c_i32),
                ("num_threads", c_i32)]


class PlanOptions(ctypes.Structure):
    _fields_ = [("struct_size", c_i32), ("mfma_tc", c_i32), ("mfma_sptc", c_i32), ("sptc_min_fill", c_f32), ("task_nnz", c_i32),
                ("piece_nnz", c_i32), ("feature_lanes", c_i32), ("streaming", c_i32), ("window_row_cap", c_i32),
                ("xcd_run", c_i32), ("sddmm_unroll", c_i32), ("stage", c_i32),
                ("occupancy", c_i32), ("xcd_split", c_i32), ("host_lowering", c_i32),
                ("sptc_sparse", c_i32), ("hot_rows", c_i32), ("split_dispatch", c_i32)]


class PlanStats(ctypes.Structure):
    _fields_ = [("m", c_i64), ("n", c_i64), ("nnz", c_i64), ("mfma_tiles", c_i64), ("mfma_nnz", c_i64),
                ("csr_nnz", c_i64), ("tasks", c_i64), ("split_rows", c_i64), ("partial_slots", c_i64),
                ("device_bytes", c_i64), ("mfma_windows", c_i64), ("window_csr_nnz", c_i64),
                ("device_lowered", c_i64), ("sparse_tiles", c_i64), ("hot_rows", c_i64), ("hot_entries", c_i64)]


class ReorderParams(ctypes.Structure):
    _fields_ = [("struct_size", c_i32), ("thres", c_i32), ("cluster_thres", c_i32), ("num_perm", c_i32), ("lsh_threshold", ctypes.c_float),
                ("bucket_span", c_i32), ("num_threads", c_i32), ("exhaustive", c_i32), ("align_window", c_i32),
                ("seed", ctypes.c_uint64), ("minhash", c_i32)]


class MatchStats(ctypes.Structure):
    _fields_ = [("total_rows", c_i64), ("total_cols", c_i64), ("total_nnz", c_i64), ("sparsity", c_f64),
                ("num_row_panels", c_i64), ("num_sptc_groups", c_i64), ("num_tc_blocks", c_i64),
                ("num_16x16_blocks", c_i64), ("block_padding_groups", c_i64), ("fine_fallback", c_i64),
                ("coarse_fallback", c_i64), ("fake_zeros", c_i64), ("tc_total_nnz", c_i64),
                ("tc_block_count", c_i64), ("tc_block_max_nnz", c_i64), ("tc_block_min_nnz", c_i64)]


# name -> (restype, argtypes); every symbol declared in include/trspmm.h
PROTOTYPES = {
    "trs_build_params_default": (None, [ctypes.POINTER(BuildParams)]),
    "trs_build_online": (c_i32, [c_p, c_p, c_p, c_i32, c_i64, ctypes.POINTER(BuildParams), c_pp]),
    "trs_format_slot": (c_i32, [c_p, c_i32, c_pp, ctypes.POINTER(c_i64)]),
    "trs_format_elapsed": (c_f64, [c_p]),
    "trs_format_window": (c_i32, [c_p]),
    "trs_format_rows": (c_i32, [c_p]),
    "trs_format_canonical": (c_i32, [c_p]),
    "trs_format_free": (None, [c_p]),
    "trs_format_write": (c_i32, [c_p, ctypes.c_char_p]),
    "trs_reorder_params_default": (None, [ctypes.POINTER(ReorderParams)]),
    "trs_tca_reorder": (c_i32, [c_p, c_p, c_i32, c_i64, c_i32, ctypes.POINTER(ReorderParams), c_p]),
    "trs_lsh_bands": (c_i32, [ctypes.c_float, c_i32, ctypes.POINTER(c_i32), ctypes.POINTER(c_i32)]),
    "trs_minhash_signatures": (c_i32, [c_p, c_p, c_i32, ctypes.POINTER(ReorderParams), c_i32, c_p]),
    "trs_format_read": (c_i32, [ctypes.c_char_p, c_pp]),
    "trs_build_online_device": (c_i32, [c_p, c_p, c_p, c_i32, c_i64, ctypes.POINTER(BuildParams), c_p, c_pp]),
    "trs_dformat_slot": (c_i32, [c_p, c_i32, c_pp, ctypes.POINTER(c_i64)]),
    "trs_dformat_download": (c_i32, [c_p, c_pp]),
    "trs_dformat_elapsed": (c_f64, [c_p]),
    "trs_dformat_rows": (c_i32, [c_p]),
    "trs_dformat_window": (c_i32, [c_p]),
    "trs_dformat_free": (None, [c_p]),
    "trs_match_2to4": (c_i32, [c_p, c_p, c_i32, c_i64, c_i32, c_i32, c_i32, c_i32, ctypes.POINTER(MatchStats)]),
    "trs_plan_options_default": (None, [ctypes.POINTER(PlanOptions)]),
    "trs_plan_create": (c_i32, [c_p, c_i32, c_i32, ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_create_parallel": (c_i32, [c_p, ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_create_sptc": (c_i32, [c_p, c_p, c_p, c_i64, c_p, c_p, c_i64, c_i32, c_i32, c_i32,
                                     ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_create_sptc_packed": (c_i32, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_i32, c_i32, c_i32,
                                            ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_create_csr": (c_i32, [c_p, c_p, c_p, c_i32, c_i32, ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_create_sddmm": (c_i32, [c_p, c_i32, c_i32, ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_create_dformat": (c_i32, [c_p, c_i32, c_i32, ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_create_sddmm_dformat": (c_i32, [c_p, c_i32, c_i32, ctypes.POINTER(PlanOptions), c_pp]),
    "trs_plan_stats_get": (c_i32, [c_p, ctypes.POINTER(PlanStats), c_i64]),
    "trs_plan_free": (None, [c_p]),
    "trs_spmm_workspace_bytes": (c_i64, [c_p, c_i32]),
    "trs_spmm_f16": (c_i32, [c_p, c_p, c_i64, c_i32, c_p, c_i64, c_p, c_i64, c_p]),
    "trs_spmm_f16_noalloc": (c_i32, [c_p, c_p, c_i64, c_i32, c_p, c_i64, c_p]),
    "trs_sddmm_f16": (c_i32, [c_p, c_p, c_i64, c_p, c_i64, c_i32, c_p, c_p]),
    "trs_sddmm_workspace_bytes": (c_i64, [c_p, c_i32]),
    "trs_sddmm_f16_ws": (c_i32, [c_p, c_p, c_i64, c_p, c_i64, c_i32, c_p, c_p, c_i64, c_p]),
    "trs_spmm_f16_timed": (c_i32, [c_p, c_p, c_i64, c_i32, c_p, c_i64, c_p, c_i64, c_p, c_i32, c_i32,
                                   ctypes.POINTER(c_f32)]),
    "trs_spmm_f16_kernel_ms": (c_i32, [c_p, c_p, c_i64, c_i32, c_p, c_i64, c_p, c_i64, c_p, c_i32,
                                       ctypes.POINTER(c_f32)]),
    "trs_sddmm_f16_kernel_ms": (c_i32, [c_p, c_p, c_i64, c_p, c_i64, c_i32, c_p, c_p, c_i64, c_p, c_i32,
                                        ctypes.POINTER(c_f32)]),
    "trs_last_error": (ctypes.c_char_p, []),
    "trs_abi_version": (c_i32, []),
}

_lib = None
_ext = None


class TrsError(RuntimeError):
    """A C-ABI call returned a non-zero trs_status."""

    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where}: {msg} (trs_status {code})")
        self.code = code


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `make -C tr-spmm_zzx_amd` "
                              "(or __graft_entry__.build())")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def check(rc: int, where: str) -> None:
    if rc != 0:
        raise TrsError(rc, where, lib().trs_last_error().decode(errors="replace"))


def ext():
    """The PyTorch extension with the reference operator signatures."""
    global _ext
    if _ext is None:
        lib()
        _ext = importlib.import_module("trspmm._trspmm_ext")
    return _ext
