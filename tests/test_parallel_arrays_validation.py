"""Host-side validation of the reference parallel operator's arrays (trs_plan_create_parallel, the
plan behind Libra6SpMMOnline.forward_fp16_tcu_cuda_sptc_mma_parallel_online; the reference's checks
are TR-source/SpMM/mGCN_online.cpp:858-932).  Runs without a GPU: well-formed arrays pass every
check and only then fail at the device upload (TRS_EDEVICE), malformed ones are refused before it
with TRS_EINVAL / TRS_ERANGE.  With a GPU present the well-formed case builds a plan instead."""
import ctypes

import numpy as np
import pytest

from trspmm import _native as nat
from trspmm import graphs
import trspmm

P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32


class ParallelArrays(ctypes.Structure):
    """Mirror of trs_parallel_arrays (include/trspmm.h)."""
    _fields_ = (
        [(f"{n}", P) if i % 2 == 0 else (f"n_{n}", I64)
         for n in ("t_row_offset", "t_block_offset", "t_column", "t_value", "t_window_row", "t_atomic", "t_binary",
                   "c_row_offsets", "c_row", "c_atomic", "c_column", "c_value",
                   "cs_row_offsets", "cs_row", "cs_atomic", "cs_column", "cs_value")
         for i in (0, 1)]
        + [("s_column", P), ("s_value", P), ("s_pos", P), ("groups", I64), ("s_offsets", P), ("n_s_offsets", I64),
           ("s_tile_column", P), ("s_packed_a", P), ("s_packed_meta", P), ("s_window_tile_offset", P),
           ("tiles", I64), ("n_s_window_tile_offset", I64), ("use_packed_tiles", I32),
           ("spill_row", P), ("spill_col", P), ("spill_val", P), ("spill_count", I64),
           ("parts_t", I32), ("parts_c", I32), ("partsize_c", I32), ("parts_c_short", I32), ("window", I32),
           ("m", I32), ("n", I32)])


def _fixture(g=None):
    default = g is None
    g = g or graphs.sbm(communities=64, seed=3, val_seed=4)   # TC blocks, 2:4 groups, short residual parts
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    arrs = [np.ascontiguousarray(a) for a in f.arrays()]
    assert not default or (arrs[1].size > 1 and arrs[17].shape[0] > 0 and arrs[15].size > 0)
    for i in (3, 11, 16):   # t / c values reach the operator as fp16
        arrs[i] = arrs[i].astype(np.float16).view(np.uint16)
    return g, arrs


def _fill(a, arrs, g, packed):
    keep = []

    def put(name, arr):
        arr = np.ascontiguousarray(arr)
        keep.append(arr)
        setattr(a, name, arr.ctypes.data if arr.size else None)
        if ("n_" + name) in dict(ParallelArrays._fields_):
            setattr(a, "n_" + name, arr.size)

    names = ["t_row_offset", "t_block_offset", "t_column", "t_value", "t_window_row", "t_atomic", "t_binary",
             "c_row_offsets", "c_row", "c_atomic", "c_column", "c_value",
             "cs_row_offsets", "cs_row", "cs_atomic", "cs_column", "cs_value"]
    for i, n in enumerate(names):
        put(n, arrs[i])
    put("s_column", arrs[17])
    put("s_value", arrs[19])
    put("s_pos", arrs[20])
    a.groups = arrs[17].shape[0]
    put("s_offsets", arrs[22])
    a.n_s_offsets = arrs[22].size
    put("s_tile_column", arrs[25])
    put("s_packed_a", arrs[26])
    put("s_packed_meta", arrs[27])
    put("s_window_tile_offset", arrs[28])
    a.n_s_window_tile_offset = arrs[28].size
    a.tiles = arrs[23].shape[0]
    a.use_packed_tiles = int(packed)
    a.spill_count = 0
    a.parts_t, a.parts_c, a.partsize_c, a.parts_c_short = arrs[5].size, arrs[9].size, 32, arrs[14].size
    a.window, a.m, a.n = 16, g.m, g.n
    return keep


def _create(arrs, g, packed=True):
    lib = nat.lib()
    lib.trs_plan_create_parallel.argtypes = [ctypes.POINTER(ParallelArrays), ctypes.POINTER(nat.PlanOptions),
                                             ctypes.POINTER(ctypes.c_void_p)]
    a = ParallelArrays()
    keep = _fill(a, arrs, g, packed)
    h = ctypes.c_void_p()
    rc = lib.trs_plan_create_parallel(ctypes.byref(a), None, ctypes.byref(h))
    del keep
    if rc == 0:
        lib.trs_plan_free(h)
    return rc, lib.trs_last_error().decode()


def test_struct_size_matches_header_layout():
    # sizeof(trs_parallel_arrays) on x86-64 (printed by a C program including the header)
    assert ctypes.sizeof(ParallelArrays) == 440


@pytest.mark.parametrize("packed", [True, False])
def test_wellformed_arrays_pass_validation(packed):
    g, arrs = _fixture()
    rc, msg = _create(arrs, g, packed)
    assert rc in (0, 3), msg           # 0 with a GPU, TRS_EDEVICE (upload) without one


CASES = [
    ("t_row_offset past the sub-blocks", lambda a: a[0].__setitem__(-1, a[1].size + 5), (1,)),
    ("t_row_offset decreasing", lambda a: a[0].__setitem__(1, -1) if a[0].size > 1 else None, (1,)),
    ("residual column beyond n", lambda a: a[15].__setitem__(0, 10 ** 7), (1, 5)),
    ("residual offsets decreasing", lambda a: a[12].__setitem__(1, -3), (1,)),
    ("residual part count beyond its offsets", lambda a: a.__setitem__(12, a[12][:-2].copy()), (1,)),
    ("TC column beyond n", lambda a: a[2].__setitem__(0, 10 ** 7), (1, 5)),
    ("2:4 position outside 0..3", lambda a: a[20].__setitem__((0, 0, 0), 7), (1,)),
    ("s_offsets out of range", lambda a: a[22].__setitem__(-1, a[22][-1] + 9), (1,)),
    ("tile offsets out of range", lambda a: a[28].__setitem__(-1, a[28][-1] + 9), (1,)),
    ("short residual values shorter than columns", lambda a: a.__setitem__(16, a[16][:-1].copy()), (1,)),
]


# Each plan kind validates the arrays it reads: the packed-tile plan reads s_packed_meta and
# s_window_tile_offset (not s_pos or s_offsets), the group plan the reverse.
NOT_READ = {("2:4 position outside 0..3", True), ("s_offsets out of range", True),
            ("tile offsets out of range", False)}
VALIDATION = [(w, m, c, p) for (w, m, c) in CASES for p in (True, False) if (w, p) not in NOT_READ]


@pytest.mark.parametrize("what,mutate,codes,packed", VALIDATION,
                         ids=[f"{c[0]}-{'packed' if c[3] else 'groups'}" for c in VALIDATION])
def test_malformed_arrays_are_refused_before_upload(what, mutate, codes, packed):
    g, arrs = _fixture()
    arrs = [a.copy() for a in arrs]
    mutate(arrs)
    rc, msg = _create(arrs, g, packed)
    assert rc in codes, (what, rc, msg)


@pytest.mark.parametrize("packed", [True, False])
def test_long_residual_values_shorter_than_columns_are_refused(packed):
    # the SBM fixture has no long residual part: give it one of four entries, with a value short
    g, arrs = _fixture()
    arrs = [a.copy() for a in arrs]
    arrs[7] = np.array([0, 4], np.int32)                    # c_row_offsets
    arrs[8] = np.array([0], np.int32)                       # c_row
    arrs[9] = np.array([0], np.int32)                       # c_atomic
    arrs[10] = np.array([0, 1, 2, 3], np.int32)             # c_column
    arrs[11] = np.ones(4, np.float16).view(np.uint16)       # c_value
    rc, msg = _create(arrs, g, packed)
    assert rc in (0, 3), msg                                # well-formed so far
    arrs[11] = arrs[11][:3].copy()
    rc, msg = _create(arrs, g, packed)
    assert rc == 1 and "value" in msg, (rc, msg)
