"""The allocation-free tied cross-entropy (nml_tied_ce_forward_device_noalloc) against the
allocating entry point (nml_tied_ce_forward_device), called through the C-ABI.

Two calls in a row, the second smaller, both compared with the allocating entry point
on the same device buffers: the loss within 1e-6 relative (the same per-row arithmetic;
the float64 sum runs over more row chunks, since the fixed scratch holds fewer rows of
logits), float16 and float32, with ignore_index rows. A vocabulary whose one row of logits
exceeds the fixed scratch is refused with an error before anything is launched.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _ce(fn, hidden, weights, labels, ignore):
    from nimbleml_amd import _native as N

    rows, dim = hidden.shape
    loss = ctypes.c_double()
    N.check(fn(hidden.ptr, weights.ptr, labels.ptr, rows, dim, weights.shape[0],
               int(ignore if ignore is not None else 0), int(ignore is not None),
               ctypes.byref(loss), N.np_dtype_code(hidden.dtype)))
    return loss.value


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_noalloc_tied_ce_matches_allocating_entry_point(gpu, dtype):
    from nimbleml_amd import _native as N

    rng = np.random.default_rng(11)
    vocab, dim = 32000, 256
    # rows per chunk of the 32 MiB scratch: 524 (fp16) / 262 (fp32) — several chunks
    for call, (rows, ignore) in enumerate([(1500, None), (300, -100)]):
        h = rng.standard_normal((rows, dim)).astype(dtype)
        w = (0.3 * rng.standard_normal((vocab, dim))).astype(dtype)
        lab = rng.integers(0, vocab, rows).astype(np.int64)
        if ignore is not None:
            lab[::7] = ignore
        hd, wd, ld = (N.DeviceArray.from_host(a) for a in (h, w, lab))
        print(f"call {call}: rows {rows} dtype {np.dtype(dtype).name}", flush=True)
        want = _ce(N.lib.nml_tied_ce_forward_device, hd, wd, ld, ignore)
        got = _ce(N.lib.nml_tied_ce_forward_device_noalloc, hd, wd, ld, ignore)
        assert np.isfinite(want) and want > 0
        assert abs(got - want) <= 1e-6 * abs(want), (call, got, want)


def test_noalloc_tied_ce_refuses_oversized_vocab(gpu):
    from nimbleml_amd import _native as N

    buf = N.DeviceArray((64,), np.float16)
    lab = N.DeviceArray.from_host(np.zeros(1, np.int64))
    loss = ctypes.c_double()
    rc = N.lib.nml_tied_ce_forward_device_noalloc(buf.ptr, buf.ptr, lab.ptr, 1, 8, 20_000_000,
                                                  0, 0, ctypes.byref(loss), 1)
    assert rc != 0
    assert b"scratch" in N.lib.nml_last_error()
