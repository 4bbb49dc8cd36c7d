"""The libstdc++ introsort restatement the device builder runs (tr-spmm_zzx_amd/csrc/introsort.hpp)
against this compiler's std::sort: the same permutation, element for element, of unit indices
sorted by a key with heavy ties (the builder's nnz-descending unit order, block_online.cpp:358-363),
up to n = 100k; McIlroy-adversary inputs that push it into the heap-sort fallback; and the
list form of the partition step and its batched form (the one a wave runs, a batch of stops per
lane) against the scanning form, and whole sorts built on the batched step (leaves finished by a
stable insertion sort, as the final insertion sort leaves them) against std::sort, and the closed
form for ranges of equal keys against the loop.  No GPU:
tests/native/introsort_check.cpp is compiled with g++ for the host."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT

SRC = os.path.join(ROOT, "tests", "native", "introsort_check.cpp")
INC = os.path.join(ROOT, "tr-spmm_zzx_amd", "csrc")


@pytest.fixture(scope="module")
def chk(tmp_path_factory):
    so = str(tmp_path_factory.mktemp("isort") / "introsort_check.so")
    subprocess.check_call(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-I", INC, SRC, "-o", so])
    lib = ctypes.CDLL(so)
    i64p = ctypes.POINTER(ctypes.c_int64)
    lib.check_random.argtypes = [i64p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint64]
    lib.check_monotone.argtypes = lib.check_random.argtypes
    lib.check_random.restype = lib.check_monotone.restype = ctypes.c_int64
    lib.check_killer.argtypes = [i64p, ctypes.c_int32, ctypes.c_int32]
    lib.check_killer.restype = ctypes.c_int64
    lib.killer_reaches_heap_sort.argtypes = [ctypes.c_int64]
    lib.killer_reaches_heap_sort.restype = ctypes.c_int32
    lib.check_partition_lists.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint64,
                                          ctypes.c_int32]
    lib.check_partition_lists.restype = ctypes.c_int64
    lib.check_partition_batched.argtypes = lib.check_partition_lists.argtypes + [ctypes.c_int32]
    lib.check_partition_batched.restype = ctypes.c_int64
    lib.check_batched_sort.argtypes = [i64p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint64,
                                       ctypes.c_int32]
    lib.check_batched_sort.restype = ctypes.c_int64
    lib.check_tied.argtypes = [ctypes.c_int64]
    lib.check_tied.restype = ctypes.c_int64
    return lib


def _sizes(*n):
    a = np.asarray(n, dtype=np.int64)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), len(n)


SMALL = (0, 1, 2, 3, 15, 16, 17, 18, 31, 32, 33, 47, 64, 100, 257, 1000)
LARGE = (4096, 20000, 65537, 100000)


@pytest.mark.parametrize("alphabet", [1, 2, 3, 5, 14, 33, 1000, 1 << 30])
def test_random_keys_match_std_sort(chk, alphabet):
    keep, p, k = _sizes(*SMALL)
    assert chk.check_random(p, k, alphabet, 40, 1 + alphabet) == 0
    keep, p, k = _sizes(*LARGE)
    assert chk.check_random(p, k, alphabet, 2, 7 + alphabet) == 0


@pytest.mark.parametrize("alphabet", [2, 3, 7, 14, 31])
def test_monotone_keys_match_std_sort(chk, alphabet):
    """Non-increasing keys with long tie runs: the order the builder's units arrive in."""
    keep, p, k = _sizes(*SMALL)
    assert chk.check_monotone(p, k, alphabet, 40, 11 + alphabet) == 0
    keep, p, k = _sizes(*LARGE)
    assert chk.check_monotone(p, k, alphabet, 3, 17 + alphabet) == 0


def test_heap_sort_fallback_matches_std_sort(chk):
    assert chk.killer_reaches_heap_sort(2000) == 1 and chk.killer_reaches_heap_sort(100000) == 1
    keep, p, k = _sizes(100, 1000, 2000, 30000, 100000)
    for tie in (1, 2, 5, 40):
        assert chk.check_killer(p, k, tie) == 0, tie


@pytest.mark.parametrize("alphabet,monotone", [(2, 0), (3, 0), (14, 0), (1000, 0), (2, 1), (5, 1), (14, 1)])
def test_partition_lists_equal_scans(chk, alphabet, monotone):
    assert chk.check_partition_lists(3000, alphabet, 3000, 5 + alphabet, monotone) == 0
    assert chk.check_partition_lists(40, alphabet, 20000, 9 + alphabet, monotone) == 0


@pytest.mark.parametrize("lanes", [1, 2, 3, 4, 8, 64])
@pytest.mark.parametrize("alphabet,monotone", [(2, 0), (3, 0), (1000, 0), (2, 1), (3, 1), (14, 1), (31, 1)])
def test_batched_partition_equals_scans(chk, lanes, alphabet, monotone):
    assert chk.check_partition_batched(2000, alphabet, 1500, 3 + alphabet + lanes, monotone, lanes) == 0
    assert chk.check_partition_batched(200, alphabet, 4000, 7 + alphabet + lanes, monotone, lanes) == 0


@pytest.mark.parametrize("lanes", [2, 5, 64])
@pytest.mark.parametrize("alphabet", [1, 2, 3, 7, 14, 31])
def test_sort_on_batched_partitions_equals_std_sort(chk, lanes, alphabet):
    keep, p, k = _sizes(*SMALL)
    assert chk.check_batched_sort(p, k, alphabet, 20, 21 + alphabet + lanes, lanes) == 0
    keep, p, k = _sizes(4096, 20000, 70000)
    assert chk.check_batched_sort(p, k, alphabet, 2, 23 + alphabet + lanes, lanes) == 0


def test_tied_range_closed_form(chk):
    """The device builder's shortcut for ranges of equal keys (isort::tied_final_offset: each
    element's final offset from its own, no partition passes) against the restated loop and final
    insertion sort, for every length up to 3000 and sampled ones to 100k, at depth limits from one
    too few (the heap-sort case, which tied_depth_ok must recognise) to three more than needed."""
    assert chk.check_tied(100000) == 0
