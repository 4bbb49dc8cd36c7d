import glob
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "tr-spmm_zzx_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


def golden_files():
    return sorted(glob.glob(os.path.join(GOLDEN, "builder_*.npz")))


def load_golden(path):
    z = np.load(path, allow_pickle=False)
    params = {k[6:]: z[k].item() for k in z.files if k.startswith("param_")}
    env = {k[4:]: str(z[k]) for k in z.files if k.startswith("env_")}
    outs = [z[f"out_{i}"] for i in range(29)]
    return z["rowptr"], z["col"], z["val"], params, env, outs


@pytest.fixture
def golden_env(monkeypatch):
    def apply(env):
        for k in ("LIBRA_SKIP_TC", "LIBRA_SPTC_UNIT_MIN_NNZ"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
    return apply


def same_array(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    return a.dtype == b.dtype and a.shape == b.shape and (a.size == 0 or np.array_equal(a.view(np.uint8), b.view(np.uint8)))
