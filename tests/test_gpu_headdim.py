"""Head dims outside the tuned set (8, 16, 32, 64, 128): the reference's CPU attention takes
any head dim (kernels/fused_sdpa.py:71-78) and its device flash kernel any dk ≤ 256
(native/src/sdpa_cuda.cu:237), so ``GPT(768, 8, ...)`` (dk 96) or a dk-256 model must run.

Covered here, each against the oracle (oracle/gpt_ref.py) on the same seeded weights:
  * whole models at dk 40, 96 and 256 — prefill logits, cached decode logits (the
    ``forward_with_cache`` seam of models/generate.py:93-100), greedy tokens of ragged
    rows through ``generate``, and ``compute_loss``;
  * the decode-attention export ``nml_decode_attention_device`` through the C-ABI on
    ragged lengths, against ``R.sdpa`` on each row's cached keys.
Tolerances are the north star's: fp32 logits ≤ 1e-3, fp16 ≤ 3e-2, loss relative ≤ 1e-4.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle.weights import GPTConfig, make_weights, random_ids

pytestmark = pytest.mark.gpu

# (vocab, d_model, heads, layers, max_seq): head dims 40, 96, 256
SHAPES = [(512, 80, 2, 2, 160), (512, 192, 2, 2, 160), (512, 512, 2, 2, 160)]


def _tol(dt):
    return 3e-2 if np.dtype(dt) == np.float16 else 1e-3


def _model(cfg, dt, seed=11):
    import nimbleml_amd as nm

    w = make_weights(cfg, seed=seed, dtype=dt, rich=True)
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=dt)
    return m, w


@pytest.mark.parametrize("dt", [np.float32, np.float16])
@pytest.mark.parametrize("dims", SHAPES, ids=lambda d: f"dk{d[1] // d[2]}")
def test_model_forward_and_cached_decode(gpu, dims, dt):
    cfg = GPTConfig(*dims)
    m, w = _model(cfg, dt)
    ids = random_ids((2, 100), cfg.vocab_size, seed=4)  # two 64-query tiles, ragged end
    lg = m.forward(ids).numpy().astype(np.float64)
    want = R.forward(w, ids, cfg.num_heads, cfg.num_layers).astype(np.float64)
    assert np.abs(lg - want).max() <= _tol(dt)
    # prefill 70 tokens into the cache, then decode 30 one at a time
    a, cache = m.forward_with_cache(ids[:, :70])
    assert np.abs(a.numpy().astype(np.float64) - want[:, :70]).max() <= _tol(dt)
    for t in range(70, 100):
        b, cache = m.forward_with_cache(ids[:, t:t + 1], cache)
        assert np.abs(b.numpy().astype(np.float64)[:, 0] - want[:, t]).max() <= _tol(dt), t


@pytest.mark.parametrize("dims", SHAPES, ids=lambda d: f"dk{d[1] // d[2]}")
def test_model_loss(gpu, dims):
    cfg = GPTConfig(*dims)
    for dt in (np.float32, np.float16):
        m, w = _model(cfg, dt, seed=12)
        ids = random_ids((3, 90), cfg.vocab_size, seed=5)
        labels = random_ids((3 * 90,), cfg.vocab_size, seed=6)
        got = m.compute_loss(ids, labels).item()
        want = R.compute_loss(w, ids, labels, cfg.num_heads, cfg.num_layers)
        rel = 1e-4 if dt == np.float32 else 2 ** -10  # fp16: the reference's fp16 loss
        assert abs(got - want) <= rel * abs(want), (dt, got, want)


@pytest.mark.parametrize("dims", SHAPES, ids=lambda d: f"dk{d[1] // d[2]}")
def test_ragged_greedy_generate_fp32(gpu, dims):
    """Rows of different lengths (packed prefill, then the batched decode step) give the
    oracle's greedy tokens; fp32 logits sit within 1e-3 of the oracle, so every step whose
    reference top-2 margin exceeds that must agree."""
    import nimbleml_amd as nm

    cfg = GPTConfig(*dims)
    m, w = _model(cfg, np.float32, seed=13)
    rng = np.random.default_rng(7)
    rows = [rng.integers(0, cfg.vocab_size, n) for n in (5, 64, 65, 33)]
    new = 16
    out = nm.generate(m, rows, max_new_tokens=new, temperature=0.0)
    compared = 0
    for b, r in enumerate(rows):
        got = np.asarray(out[b])
        kv = R.KVOracle(w, cfg.num_heads, cfg.num_layers)
        lg = kv.step(got[None, :len(r)])[0, -1]
        for t in range(new):
            top2 = np.sort(lg.astype(np.float64))[-2:]
            if top2[1] - top2[0] <= 1e-3:
                break
            assert got[len(r) + t] == int(np.argmax(lg)), (b, t)
            compared += 1
            lg = kv.step(got[None, len(r) + t:len(r) + t + 1])[0, -1]
    assert compared >= 2 * len(rows), compared


@pytest.mark.parametrize("dt", [np.float32, np.float16])
@pytest.mark.parametrize("dk", [8, 40, 64, 96, 128, 256])
def test_decode_attention_device_c_abi(gpu, dk, dt):
    """nml_decode_attention_device through the C-ABI: batch 5 with lengths 1…300 (one to
    five 64-key chunks, ragged), 3 heads, against the float64 softmax attention of each
    row's first lens[b] cached keys (kernels/fused_sdpa.py:71-78)."""
    from nimbleml_amd import _native as N

    rng = np.random.default_rng(dk)
    batch, heads, max_seq = 5, 3, 320
    lens = np.array([1, 64, 65, 300, 129], np.int32)
    q = rng.standard_normal((batch, heads, dk)).astype(dt)
    kc = rng.standard_normal((batch, heads, max_seq, dk)).astype(dt)
    vc = rng.standard_normal((batch, heads, max_seq, dk)).astype(dt)
    dq, dkc, dvc, dl = (N.DeviceArray.from_host(a) for a in (q, kc, vc, lens))
    err = N.DeviceArray.from_host(np.zeros(1, np.int32))
    out = N.DeviceArray((batch, heads * dk), dt)
    scale = float(np.sqrt(dk))
    for rep in range(2):  # the grouped kernel leaves its workspace cleared for the next call
        N.check(N.lib.nml_decode_attention_device(dq.ptr, dkc.ptr, dvc.ptr, dl.ptr, out.ptr, batch,
                                                  heads, max_seq, dk, C.c_float(scale), err.ptr,
                                                  N.np_dtype_code(dt)))
        got = out.numpy().astype(np.float64).reshape(batch, heads, dk)
        assert int(err.numpy()[0]) == 0
        for b in range(batch):
            n = int(lens[b])
            want = R.sdpa(q[b][:, None, :].astype(np.float64), kc[b, :, :n].astype(np.float64),
                          vc[b, :, :n].astype(np.float64), scale, None)[:, 0]
            tol = 4e-3 if dt == np.float16 else 1e-5
            assert np.abs(got[b] - want).max() <= tol, (rep, b)


def test_decode_attention_device_flags_bad_lengths(gpu):
    """A length outside [1, max_seq] is clamped (no key past the cache is read) and
    reported: the Python wrapper raises ValueError."""
    from nimbleml_amd import kernels as K

    rng = np.random.default_rng(0)
    q = rng.standard_normal((2, 1, 64)).astype(np.float32)
    kc = rng.standard_normal((2, 1, 32, 64)).astype(np.float32)
    out = np.asarray(K.decode_attention(q, kc, kc, np.array([3, 32], np.int32), 8.0))
    assert out.shape == (2, 64)
    with pytest.raises(ValueError):
        K.decode_attention(q, kc, kc, np.array([3, 33], np.int32), 8.0)
    with pytest.raises(ValueError):
        K.decode_attention(q, kc, kc, np.array([0, 4], np.int32), 8.0)


def test_head_dim_above_256_is_refused(gpu):
    import nimbleml_amd as nm

    with pytest.raises(RuntimeError, match="head_dim"):
        m = nm.GPT(64, 520, 2, 1, 16)
        m.forward(np.zeros((1, 4), np.int64))
