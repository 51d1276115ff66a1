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


@pytest.mark.parametrize("name", ["tiny_rope_fp32", "tiny_rope_fp16"])
def test_rope_reference_fixture(gpu, name):
    """Against the reference's own use_rope=True run (tests/golden/make_golden.py):
    all-position logits within the logit tolerance, the loss, and greedy tokens while
    the oracle's decision margin exceeds that tolerance."""
    import nimbleml_amd as nm
    from conftest import fixture_weights, golden

    f = golden(name)
    cfg, w = fixture_weights(f)
    dt = w["token_emb.weights"].dtype
    tol = 3e-2 if dt == np.float16 else 1e-3
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, ff_mult=cfg.ff_mult, dtype=dt, use_rope=True)
    lg = m.forward(f["greedy"][:, :-1]).numpy().astype(np.float64)
    assert np.abs(lg - f["greedy_logits"].astype(np.float64)).max() <= tol
    got = m.compute_loss(f["loss_ids"], f["loss_labels"]).item()
    assert abs(got - float(f["loss"])) <= (2 ** -8 if dt == np.float16 else 1e-4) * abs(got)
    s0 = f["prompt"].shape[1]
    n = f["greedy"].shape[1] - s0
    out = nm.generate(m, f["prompt"], max_new_tokens=n, temperature=0.0)
    rope = R.rope_cache(cfg.max_seq_len, cfg.d_model // cfg.num_heads)
    kv = R.KVOracle({k: v.astype(np.float32) for k, v in w.items()}, cfg.num_heads,
                    cfg.num_layers, rope)
    ref = f["greedy"]
    lgo = kv.step(ref[:, :s0])[:, -1]
    compared = 0
    alive = np.ones(ref.shape[0], bool)
    for t in range(n):
        top2 = np.sort(lgo.astype(np.float64), axis=-1)[:, -2:]
        alive &= (top2[:, 1] - top2[:, 0]) > tol
        for b in np.nonzero(alive)[0]:
            assert out[b, s0 + t] == ref[b, s0 + t], (b, t)
            compared += 1
        lgo = kv.step(ref[:, s0 + t:s0 + t + 1])[:, -1]
    assert compared >= n, compared
