"""Optimizer step on the device against the oracle (oracle/optim_ref.py, itself pinned
bit for bit to the reference's native kernels): AdamW bit-exact over aligned bulk and
ragged tails, with and without weight decay, over several steps; the clip's norm and
scaled gradients within float32 rounding of a float64 sum taken in another order."""
import numpy as np
import pytest

from oracle import optim_ref as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 3, 4, 1001, 1 << 20, (1 << 22) + 7])
@pytest.mark.parametrize("wd", [0.0, 0.05])
def test_adamw_device_bit_exact(gpu, n, wd):
    from nimbleml_amd import _native as N
    from nimbleml_amd import kernels as K

    rng = np.random.default_rng(n)
    p = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    dp, dm, dv = (N.DeviceArray.from_host(a) for a in (p, m, v))
    for t in range(1, 4):
        g = (rng.standard_normal(n) * 10.0 ** -t).astype(np.float32)
        args = (3e-4, 0.9, 0.999, 1.0 - 0.9 ** t, 1.0 - 0.999 ** t, 1e-8, wd)
        K.adamw_step(dp, N.DeviceArray.from_host(g), dm, dv, *args)
        O.adamw_step(p, g, m, v, *args)
    for d, h in ((dp, p), (dm, m), (dv, v)):
        assert np.array_equal(d.numpy().view(np.uint32), h.view(np.uint32))


@pytest.mark.parametrize("max_norm", [0.25, 1e9])
def test_clip_grad_norm_device(gpu, max_norm):
    from nimbleml_amd import _native as N
    from nimbleml_amd import kernels as K

    rng = np.random.default_rng(9)
    sizes = [1, 5, 65536, 65537, 300000, 4096]
    grads = [(rng.standard_normal(s) * 0.01).astype(np.float32) for s in sizes]
    dev = [N.DeviceArray.from_host(g) for g in grads]
    ref = [g.copy() for g in grads]
    got = K.clip_grad_norm(dev, max_norm)
    want = O.clip_grad_norm(ref, max_norm)
    assert abs(got - float(want)) <= 2e-7 * float(want)
    for d, r, g in zip(dev, ref, grads):
        out = d.numpy()
        if max_norm > 1e6:
            assert np.array_equal(out, g)  # below the limit: untouched
        else:
            assert np.abs(out - r).max() <= 2e-7 * np.abs(r).max()
    assert K.clip_grad_norm([], 1.0) == 0.0
