"""Rotary positions (GPT(use_rope=True), models/gpt.py:46-64 → _fused_arrays.py:95-98)
on the device against the oracle: prefill logits, cached chunks, the loss, and ragged
batched greedy decode. Tolerances as in test_gpu_model.py (fp32 logits 1e-3, fp16
3e-2); tokens are compared while the oracle's top-2 margin exceeds the fp16 tolerance."""
import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle.weights import GPTConfig, make_weights, random_ids

pytestmark = pytest.mark.gpu


def rope_model(cfg, seed, dtype, sharp=True):
    import nimbleml_amd as nm

    w = make_weights(cfg, seed=seed, dtype=np.float32, rich=True)
    w.pop("pos_emb.weights")
    if sharp:  # larger q·k so that positions visibly move the logits
        for i in range(cfg.num_layers):
            for n in ("W_q", "W_k"):
                w[f"blocks.layers.{i}.mha.{n}.weights"] *= 6
    w = {k: v.astype(dtype) for k, v in w.items()}
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=dtype, use_rope=True)
    rope = R.rope_cache(cfg.max_seq_len, cfg.d_model // cfg.num_heads)
    return m, w, rope


@pytest.mark.parametrize("dtype,tol", [(np.float32, 1e-3), (np.float16, 3e-2)])
@pytest.mark.parametrize("dims", [(256, 64, 4, 2, 96), (512, 256, 4, 2, 300)])
def test_rope_forward_matches_oracle(gpu, dtype, tol, dims):
    cfg = GPTConfig(*dims)
    m, w, rope = rope_model(cfg, 11, dtype)
    ids = random_ids((2, min(cfg.max_seq_len, 150)), cfg.vocab_size, seed=4)
    got = m.forward(ids).numpy().astype(np.float64)
    want = R.forward(w, ids, cfg.num_heads, cfg.num_layers, rope).astype(np.float64)
    assert np.abs(got - want).max() <= tol
    # and the positions matter: the same weights without rotation are far off
    plain = R.forward(w, ids, cfg.num_heads, cfg.num_layers,
                      (np.ones_like(rope[0]), np.zeros_like(rope[1])))
    assert np.abs(plain.astype(np.float64) - want).max() > 3 * tol


def test_rope_cached_chunks_and_loss(gpu):
    cfg = GPTConfig(512, 256, 4, 2, 300)
    m, w, rope = rope_model(cfg, 12, np.float32)
    ids = random_ids((2, 180), cfg.vocab_size, seed=6)
    full = m.forward(ids).numpy().astype(np.float64)
    a, cache = m.forward_with_cache(ids[:, :77])
    b, cache = m.forward_with_cache(ids[:, 77:78], cache)
    c, cache = m.forward_with_cache(ids[:, 78:], cache)
    chunks = np.concatenate([a.numpy(), b.numpy(), c.numpy()], axis=1).astype(np.float64)
    assert np.abs(chunks - full).max() <= 1e-3
    labels = random_ids((2, 180), cfg.vocab_size, seed=7)
    got = float(m.compute_loss(ids, labels).numpy())
    want = R.compute_loss(w, ids, labels, cfg.num_heads, cfg.num_layers, rope=rope)
    assert abs(got - want) <= 1e-4 * abs(want)


@pytest.mark.parametrize("lens", [[37], [20, 300, 64, 65, 129, 7, 250, 33, 190, 100, 140, 41]])
def test_rope_ragged_greedy_decode_fp16(gpu, lens):
    """Batch 1 (which would take the persistent step without rotary positions) and 12
    ragged rows (skinny projections, grouped decode attention) at d1024 / 16 heads."""
    import nimbleml_amd as nm

    cfg = GPTConfig(4096, 1024, 16, 2, 1024)
    m, w, rope = rope_model(cfg, 17, np.float16, sharp=False)
    rng = np.random.default_rng(3)
    rows = [rng.integers(0, cfg.vocab_size, n) for n in lens]
    new = 16
    out = nm.generate(m, rows if len(rows) > 1 else rows[0][None, :], max_new_tokens=new,
                      temperature=0.0)
    assert not m.last_decode_persistent()
    w32 = {k: v.astype(np.float32) for k, v in w.items()}
    compared = 0
    for b, r in enumerate(rows):
        got = np.asarray(out[b])
        assert np.array_equal(got[:len(r)], r)
        kv = R.KVOracle(w32, cfg.num_heads, cfg.num_layers, rope)
        lg = kv.step(got[None, :len(r)])[0, -1]
        for t in range(new):
            top2 = np.sort(lg.astype(np.float64))[-2:]
            if top2[1] - top2[0] <= 3e-2:
                break
            assert got[len(r) + t] == int(np.argmax(lg)), (b, t)
            compared += 1
            lg = kv.step(got[None, len(r) + t:len(r) + t + 1])[0, -1]
    assert compared >= 3 * len(rows), compared
