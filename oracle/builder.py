"""ctypes front-end of the literal builder restatement (builder_oracle.cpp) and of the compiled
reference builder in ``_ref/`` -- TEST INFRASTRUCTURE ONLY (see package docstring).

Pinned by: tests/test_oracle_builder.py compares every array bit-for-bit with the golden fixtures in
tests/golden/ (written by the compiled reference, block_online.cpp) and with ``_ref`` when present.
"""
from __future__ import annotations

import ctypes
import glob
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle_builder.so")

# slot -> (name, numpy dtype); names follow the reference return list (block_online.cpp:844-870)
SLOTS = [
    ("t_rowkNew_offset", np.int32), ("t_blockNew_offset", np.int32), ("t_columnNew", np.int32),
    ("t_valueNew", np.float32), ("t_window_rowNew", np.int32), ("t_atomicNew", np.int32),
    ("t_binaryNew", np.int64),
    ("c_rowNew_offset", np.int32), ("c_rowNew", np.int32), ("c_atomicNew", np.int32),
    ("c_columnNew", np.int32), ("c_valueNew", np.float32),
    ("c_rowNew_offset_residue", np.int32), ("c_rowNew_residue", np.int32),
    ("c_atomicNew_residue", np.int32), ("c_columnNew_residue", np.int32),
    ("c_valueNew_residue", np.float32),
    ("s_columns", np.int32), ("s_masks", np.uint8), ("s_values", np.float32), ("s_pos", np.int8),
    ("s_window", np.int32), ("s_offsets", np.int32), ("s_tile_window", np.int32),
    ("s_tile_group", np.int32), ("s_tile_columns", np.int32), ("s_packed_a", np.int32),
    ("s_packed_meta", np.int32), ("s_window_tile_offset", np.int32),
]
SPILL = [("spill_row", np.int32), ("spill_col", np.int32), ("spill_val", np.float32)]

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.check_call(["make", "-s", "-C", HERE], stdout=sys.stderr)
        lib = ctypes.CDLL(LIB_PATH)
        lib.orc_build.restype = ctypes.c_void_p
        lib.orc_build.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int32] * 6 + [ctypes.c_float] + [ctypes.c_int32] * 2
        lib.orc_len.restype = ctypes.c_int64
        lib.orc_len.argtypes = [ctypes.c_void_p, ctypes.c_int]
        lib.orc_ptr.restype = ctypes.c_void_p
        lib.orc_ptr.argtypes = [ctypes.c_void_p, ctypes.c_int]
        lib.orc_free.argtypes = [ctypes.c_void_p]
        _lib = lib
    return _lib


def shape_slots(arrs: list, window: int) -> list:
    """Apply the reference's tensor shapes (block_online.cpp:789-792, 865-867)."""
    out = list(arrs)
    g = out[21].shape[0]
    out[17] = out[17].reshape(g, 4)
    out[18] = out[18].reshape(g, window)
    out[19] = out[19].reshape(g, window, 2)
    out[20] = out[20].reshape(g, window, 2)
    t = out[23].shape[0]
    out[25] = out[25].reshape(t, 16)
    out[26] = out[26].reshape(t, 8, 4, 2)
    out[27] = out[27].reshape(t, 8)
    return out


def build(rowptr, col, val, part_t=32, part_c=32, short_size=3, density=8, window=16,
          tc_min_util=0.0, skip_tc=False, unit_min_nnz=2):
    """Returns (29 reference arrays, (spill_row, spill_col, spill_val))."""
    lib = _load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    col = np.ascontiguousarray(col, dtype=np.int32)
    val = np.ascontiguousarray(val, dtype=np.float32)
    h = lib.orc_build(rowptr.ctypes.data, col.ctypes.data, val.ctypes.data, rowptr.shape[0] - 1,
                      part_t, part_c, short_size, density, window, float(tc_min_util),
                      int(bool(skip_tc)), unit_min_nnz)
    if not h:
        raise ValueError("oracle builder rejected its parameters")
    try:
        res = []
        for s, (_, dt) in enumerate(SLOTS + SPILL):
            n = lib.orc_len(h, s)
            p = lib.orc_ptr(h, s)
            a = np.empty(n, dtype=dt)
            if n:
                ctypes.memmove(a.ctypes.data, p, n * a.itemsize)
            res.append(a)
    finally:
        lib.orc_free(h)
    return shape_slots(res[:29], window), tuple(res[29:])


_ref_mod = None


def reference_module():
    """The reference builder compiled from /root/reference into _ref/ (None when absent).

    Loaded from its file without entering sys.modules, so ``import Libra5BlockOnline`` elsewhere in
    the process keeps resolving to the product's drop-in module."""
    global _ref_mod
    if _ref_mod is None:
        import importlib.util
        hits = glob.glob(os.path.join(HERE, "_ref", "Libra5BlockOnline*.so"))
        if not hits:
            return None
        spec = importlib.util.spec_from_file_location("Libra5BlockOnline", hits[0])
        _ref_mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(_ref_mod)
    return _ref_mod
