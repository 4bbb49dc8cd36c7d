"""The C ABI from plain C: tests/native/capi_smoke.c, compiled with gcc as C99 against
include/trspmm.h and linked to libtrspmm.so, builds the format of a CSR and prints every slot's
length; they equal what the same build gives through the Python bindings.  It also checks, from C,
the ABI version, a params struct of another size and a NULL output.  No GPU."""
import os
import subprocess

import numpy as np

from conftest import ROOT
from trspmm import _native as nat
from trspmm import graphs
import trspmm

SRC = os.path.join(ROOT, "tests", "native", "capi_smoke.c")
LIBDIR = os.path.dirname(nat.LIB_PATH)


def test_c_caller_builds_the_same_format(tmp_path):
    exe = str(tmp_path / "capi_smoke")
    subprocess.check_call(["gcc", "-std=c99", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), SRC,
                           "-L", LIBDIR, "-ltrspmm", "-Wl,-rpath," + LIBDIR, "-o", exe])
    g = graphs.sbm(communities=32, seed=5, val_seed=6)
    nnz = int(g.rowptr[-1])
    text = "\n".join([f"{g.rowptr.shape[0] - 1} {nnz}", " ".join(map(str, g.rowptr)), " ".join(map(str, g.col[:nnz])),
                      " ".join(repr(float(v)) for v in g.val[:nnz])])
    r = subprocess.run([exe], input=text, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stderr)
    lengths = [int(x) for x in r.stdout.split()]
    f = trspmm.build_format(g.rowptr, g.col, g.val)
    assert lengths == [f.slot(i).shape[0] for i in range(32)]
    assert lengths[3] > 0 and lengths[17] > 0   # TC values and 2:4 groups: a format with both shares
