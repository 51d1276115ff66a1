import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(REPO, "tests", "golden")
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running (full benchmark-size shapes)")


def golden(name):
    """Load a fixture written by tests/golden/make_golden.py (data only)."""
    return np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)


def fixture_config(f):
    from oracle.weights import GPTConfig

    return GPTConfig(*[int(x) for x in f["config"]])


def fixture_weights(f, dtype=None):
    from oracle.weights import make_weights

    from oracle.weights import rope_weights

    cfg = fixture_config(f)
    if dtype is None:
        dtype = np.float16 if str(f["dtype"]) == "float16" else np.float32
    if "rope" in f.files and int(f["rope"]):  # rotary-position fixtures (weights changed in fp32)
        w = rope_weights(make_weights(cfg, seed=int(f["seed"]), dtype=np.float32,
                                      rich=bool(int(f["rich"]))))
        return cfg, {k: v.astype(dtype) for k, v in w.items()}
    return cfg, make_weights(cfg, seed=int(f["seed"]), dtype=dtype, rich=bool(int(f["rich"])))


@pytest.fixture(scope="session")
def gpu():
    """Initialise the HIP runtime; GPU tests fail loudly if the library or GPU is missing."""
    from nimbleml_amd import _native

    _native.ensure_init()
    return _native
