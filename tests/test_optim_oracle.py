"""The optimizer-step oracle (oracle/optim_ref.py) against the reference's own compiled
native kernels (adamw_step, clip_grad_norm from native/src/adamw.cpp, built into
oracle/_ref by `make -C oracle`), and against closed forms. CPU only."""
import glob
import importlib.util
import os

import numpy as np
import pytest

from oracle import optim_ref as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _ref_native():
    so = glob.glob(os.path.join(REPO, "oracle", "_ref", "nimbleml_native*.so"))
    if not so:
        pytest.skip("oracle/_ref not built (make -C oracle) — the reference sources are absent")
    spec = importlib.util.spec_from_file_location("nimbleml_native", so[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _state(n, seed):
    rng = np.random.default_rng(seed)
    p = rng.standard_normal(n).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    v = np.abs(rng.standard_normal(n) * 1e-5).astype(np.float32)
    return p, g, m, v


@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_adamw_matches_reference_native_bit_for_bit(wd):
    native = _ref_native()
    for t in (1, 7):
        args = (1e-3, 0.9, 0.999, 1.0 - 0.9 ** t, 1.0 - 0.999 ** t, 1e-8, wd)
        p, g, m, v = _state(10007, t)
        rp, rg, rm, rv = (a.copy() for a in (p, g, m, v))
        O.adamw_step(p, g, m, v, *args)
        native.adamw_step(rp, rg, rm, rv, *[float(x) for x in args])
        for a, b in ((p, rp), (m, rm), (v, rv)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_adamw_closed_form_first_step():
    """t = 1 from zero moments: the update is lr·g/(|g| + ε) (sign descent), decay first."""
    p = np.array([1.0, -2.0, 0.5], np.float32)
    g = np.array([0.3, -0.1, 2.0], np.float32)
    m, v = np.zeros(3, np.float32), np.zeros(3, np.float32)
    O.adamw_step(p, g, m, v, 0.01, 0.9, 0.999, 0.1, 0.001, 1e-8, 0.1)
    want = np.array([1.0, -2.0, 0.5]) * (1 - 0.01 * 0.1) - 0.01 * np.sign([0.3, -0.1, 2.0])
    assert np.abs(p - want).max() < 1e-6


@pytest.mark.parametrize("max_norm", [0.5, 1e6])
def test_clip_matches_reference_native(max_norm):
    native = _ref_native()
    rng = np.random.default_rng(3)
    grads = [(rng.standard_normal(s) * 0.3).astype(np.float32) for s in (1, 999, 70001, 4096)]
    mine = [g.copy() for g in grads]
    ref = [g.copy() for g in grads]
    n1 = O.clip_grad_norm(mine, max_norm)
    n2 = native.clip_grad_norm(ref, float(max_norm))
    assert np.float32(n1) == np.float32(n2)
    for a, b in zip(mine, ref):
        assert np.array_equal(a, b)
    want = np.sqrt(sum(float(np.sum(g.astype(np.float64) ** 2)) for g in grads))
    assert abs(float(n1) - want) <= 1e-6 * want
