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
    assert ctypes.sizeof(nat.BuildParams) == 12 * 4
    assert ctypes.sizeof(nat.PlanOptions) == 16 * 4
    assert ctypes.sizeof(nat.PlanStats) == 16 * 8
    assert ctypes.sizeof(nat.ReorderParams) == 48
    assert ctypes.sizeof(nat.MatchStats) == 16 * 8


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
    assert lib.trs_plan_stats_get(None, None) == 1
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
