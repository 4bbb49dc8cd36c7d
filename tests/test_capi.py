"""C ABI surface (include/trspmm.h) without a GPU: every declared symbol is exported and bound,
and host-side validation errors come back as status codes with a message."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT
from trspmm import _native as nat

HEADER = os.path.join(ROOT, "include", "trspmm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(trs_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = nat.lib()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(nat.PROTOTYPES), set(names) ^ set(nat.PROTOTYPES)


def test_struct_layouts_match_header():
    assert ctypes.sizeof(nat.BuildParams) == 13 * 4
    assert ctypes.sizeof(nat.PlanOptions) == 18 * 4
    assert ctypes.sizeof(nat.PlanStats) == 16 * 8
    assert ctypes.sizeof(nat.ReorderParams) == 56
    assert ctypes.sizeof(nat.MatchStats) == 16 * 8


def test_abi_version_and_default_struct_sizes():
    lib = nat.lib()
    assert lib.trs_abi_version() == int(re.search(r"#define TRSPMM_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    for cls, fn in ((nat.BuildParams, lib.trs_build_params_default), (nat.PlanOptions, lib.trs_plan_options_default),
                    (nat.ReorderParams, lib.trs_reorder_params_default)):
        p = cls()
        fn(ctypes.byref(p))
        assert p.struct_size == ctypes.sizeof(cls)


class _GuardedBuffer:
    """`size` caller bytes followed by a canary region: a library that reads or writes past the
    caller's struct would touch the canary (writes are checked; reads of it would be of 0xA5 bytes,
    which are no valid struct_size either)."""

    def __init__(self, size: int, fill: bytes):
        self.size = size
        self.buf = ctypes.create_string_buffer(fill.ljust(size, b"\0") + b"\xa5" * 256, size + 256)

    def ptr(self):
        return ctypes.cast(self.buf, ctypes.c_void_p)

    def canary_intact(self) -> bool:
        return self.buf.raw[self.size:] == b"\xa5" * 256


def _v1_plan_options() -> bytes:
    """The 12-field trs_plan_options of ABI version 1 (mfma_tc .. occupancy), defaults."""
    import struct
    return struct.pack("<iifiiiiiiiii", 1, 1, 0.25, 0, 0, 0, -1, 0, 0, 0, 0, 0)


def _v2_plan_options() -> bytes:
    """The 16-field trs_plan_options of ABI version 2 (no struct_size), defaults."""
    import struct
    return struct.pack("<iifiiiiiiiiiiiii", 1, 1, 0.25, 0, 0, 0, -1, 0, 0, 0, 0, 0, 0, 0, 1, 0)


@pytest.mark.parametrize("layout", ["abi_v1", "abi_v2"])
def test_older_plan_options_layouts_are_refused(layout):
    """A caller compiled against an earlier header passes a shorter options struct without
    struct_size: every plan constructor refuses it with TRS_EINVAL (its first field, mfma_tc = 1,
    is no valid size) before reading past that field.  No GPU is touched: the check comes first."""
    lib = nat.lib()
    blob = _v1_plan_options() if layout == "abi_v1" else _v2_plan_options()
    g = _GuardedBuffer(len(blob), blob)
    rowptr = np.array([0, 1], np.int32)
    col = np.array([0], np.int32)
    val = np.zeros(1, np.uint16)
    h = ctypes.c_void_p()
    rc = lib.trs_plan_create_csr(rowptr.ctypes.data, col.ctypes.data, val.ctypes.data, 1, 1,
                                 ctypes.cast(g.ptr(), ctypes.POINTER(nat.PlanOptions)), ctypes.byref(h))
    assert rc == 1 and not h.value
    assert b"struct_size" in lib.trs_last_error()
    assert g.canary_intact()


def test_older_build_and_reorder_params_are_refused():
    import struct
    lib = nat.lib()
    old_build = struct.pack("<iiiiiiffiiii", 32, 32, 3, 8, 16, 16, 0.0, 0.5, 12, -1, -1, 0)   # 12 fields
    g = _GuardedBuffer(len(old_build), old_build)
    rowptr = np.array([0, 1], np.int32)
    col = np.array([0], np.int32)
    val = np.ones(1, np.float32)
    h = ctypes.c_void_p()
    rc = lib.trs_build_online(rowptr.ctypes.data, col.ctypes.data, val.ctypes.data, 1, 1,
                              ctypes.cast(g.ptr(), ctypes.POINTER(nat.BuildParams)), ctypes.byref(h))
    assert rc == 1 and not h.value and b"struct_size" in lib.trs_last_error() and g.canary_intact()
    old_reorder = struct.pack("<iiifiiiiQi", 16, 128, 128, 0.2, 64, 0, 0, 0, 1, 1)   # no struct_size
    g = _GuardedBuffer(len(old_reorder), old_reorder)
    order = np.zeros(1, np.int32)
    rc = lib.trs_tca_reorder(rowptr.ctypes.data, col.ctypes.data, 1, 1, 1,
                             ctypes.cast(g.ptr(), ctypes.POINTER(nat.ReorderParams)), order.ctypes.data)
    assert rc == 1 and b"struct_size" in lib.trs_last_error() and g.canary_intact()


@pytest.mark.parametrize("stats_bytes", [12 * 8, 16 * 8 - 8, 16 * 8 + 8])
def test_plan_stats_of_another_size_are_refused(stats_bytes):
    """trs_plan_stats_get checks the caller's stats size (12 fields in ABI version 1) before
    anything else, so the check is visible without a plan (GPU); with a real plan it is repeated in
    tests/test_gpu_operators.py."""
    lib = nat.lib()
    g = _GuardedBuffer(stats_bytes, b"")
    rc = lib.trs_plan_stats_get(None, ctypes.cast(g.ptr(), ctypes.POINTER(nat.PlanStats)), stats_bytes)
    assert rc == 1 and b"stats_bytes" in lib.trs_last_error() and g.canary_intact()


def _plan_csr(rowptr, col, val, m, n):
    h = ctypes.c_void_p()
    o = nat.PlanOptions()
    nat.lib().trs_plan_options_default(ctypes.byref(o))
    rc = nat.lib().trs_plan_create_csr(rowptr.ctypes.data, col.ctypes.data if col.size else None,
                                       val.ctypes.data if val.size else None, m, n, ctypes.byref(o), ctypes.byref(h))
    return rc, h


def test_plan_rejects_bad_rowptr_and_columns():
    rc, h = _plan_csr(np.array([1, 2], np.int32), np.array([0], np.int32), np.zeros(1, np.uint16), 1, 4)
    assert rc == 1 and not h.value and b"rowptr" in nat.lib().trs_last_error()
    rc, h = _plan_csr(np.array([0, 1], np.int32), np.array([7], np.int32), np.zeros(1, np.uint16), 1, 4)
    assert rc == 5 and b"column" in nat.lib().trs_last_error()


def test_plan_from_noncanonical_format_is_refused():
    import trspmm
    f = trspmm.build_format(np.array([0, 2], np.int32), np.array([3, 1], np.int32), np.ones(2, np.float32))
    h = ctypes.c_void_p()
    rc = nat.lib().trs_plan_create(f.handle, 1, 4, None, ctypes.byref(h))
    assert rc == 4 and b"increasing" in nat.lib().trs_last_error()


def test_null_arguments_are_errors_not_crashes():
    lib = nat.lib()
    assert lib.trs_build_online(None, None, None, 0, 0, None, None) == 1
    assert lib.trs_plan_stats_get(None, None, 0) == 1
    assert lib.trs_spmm_f16(None, None, 0, 1, None, 0, None, 0, None) == 1
    assert lib.trs_spmm_workspace_bytes(None, 8) == 0
    assert lib.trs_sddmm_workspace_bytes(None, 128) == 0
    assert lib.trs_sddmm_f16(None, None, 0, None, 0, 1, None, None) == 1
    assert lib.trs_sddmm_f16_ws(None, None, 0, None, 0, 1, None, None, 0, None) == 1
    assert lib.trs_format_slot(None, 0, None, None) == 1


def test_plan_from_csr_refuses_short_arrays():
    """Plan.from_csr checks the array lengths the C entry point reads (rowptr[0..m], col / val up
    to rowptr[m]) before calling it, so no host read goes out of bounds; no GPU needed."""
    import numpy as np
    import trspmm
    rowptr = np.array([0, 2, 3, 5], np.int32)
    col = np.array([0, 1, 1, 0, 2], np.int32)
    val = np.ones(5, np.float16)
    with pytest.raises(ValueError, match="rowptr"):
        trspmm.Plan.from_csr(rowptr[:-1], col, val, 3, 3)          # shorter than m + 1
    with pytest.raises(ValueError, match="rowptr"):
        trspmm.Plan.from_csr(rowptr, col, val, 2, 3)               # longer than m + 1
    with pytest.raises(ValueError, match="col and val"):
        trspmm.Plan.from_csr(rowptr, col[:4], val, 3, 3)
    with pytest.raises(ValueError, match="col and val"):
        trspmm.Plan.from_csr(rowptr, col, val[:3], 3, 3)
