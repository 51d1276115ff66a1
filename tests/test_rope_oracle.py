"""The oracle's rotary positions (utils/rope.py:12-44) pinned by what the mathematics
fixes, then the host table builder of nimbleml_amd against it. CPU only.

The reference ships no golden vectors for RoPE; these checks are chosen so that the
plausible slips fail one of them: interleaved pairs (2i, 2i+1) instead of the half split
(i, i+half), a flipped sine, the wrong frequency exponent, a position offset ignored in
the incremental path."""
import numpy as np

from oracle import gpt_ref as R
from oracle.weights import GPTConfig, make_weights, random_ids


def test_cache_closed_form():
    cos, sin = R.rope_cache(64, 16, base=10000.0)
    p = np.arange(64, dtype=np.float64)[:, None]
    theta = 10000.0 ** (-np.arange(8, dtype=np.float64) / 8.0)
    want = p * theta
    assert np.abs(cos[:, :8] - np.cos(want)).max() < 4e-6
    assert np.abs(sin[:, :8] - np.sin(want)).max() < 4e-6
    assert np.array_equal(cos[:, :8], cos[:, 8:]) and np.array_equal(sin[:, :8], sin[:, 8:])


def test_unit_vectors_pin_half_split_pairs_and_sign():
    dk, half, p = 16, 8, 5
    cos, sin = R.rope_cache(16, dk)
    for i in range(half):
        e = np.zeros((1, dk), np.float64)
        e[0, i] = 1.0
        x = np.zeros((p + 1, dk), np.float64)
        x[p] = e[0]
        out = R.apply_rope(x, cos, sin)[p]
        want = np.zeros(dk)
        want[i], want[i + half] = cos[p, i], sin[p, i]
        assert np.array_equal(out, want), i
        x[p] = 0.0
        x[p, i + half] = 1.0
        out = R.apply_rope(x, cos, sin)[p]
        want = np.zeros(dk)
        want[i], want[i + half] = -sin[p, i], cos[p, i]
        assert np.array_equal(out, want), i


def test_position_zero_is_identity_and_norms_kept():
    rng = np.random.default_rng(0)
    cos, sin = R.rope_cache(32, 32)
    x = rng.standard_normal((3, 32, 32))
    assert np.array_equal(R.apply_rope(x[:, :1], cos, sin), x[:, :1])
    y = R.apply_rope(x, cos, sin)
    pair = lambda a: a[..., :16] ** 2 + a[..., 16:] ** 2  # noqa: E731
    assert np.abs(pair(y) - pair(x)).max() < 1e-5


def test_scores_depend_on_relative_position_only():
    """<R(m)q, R(n)k> = <R(m-n)q, k>: what makes RoPE a relative encoding."""
    rng = np.random.default_rng(1)
    cos, sin = R.rope_cache(64, 32)
    q, k = rng.standard_normal(32), rng.standard_normal(32)

    def at(v, p):
        x = np.zeros((p + 1, 32))
        x[p] = v
        return R.apply_rope(x, cos, sin)[p]

    for m, n in [(7, 3), (40, 12), (63, 0), (20, 20)]:
        assert abs(at(q, m) @ at(k, n) - at(q, m - n) @ k) < 1e-4 * (1 + abs(q @ k))


def test_offset_rows_equal_full_table_rows():
    rng = np.random.default_rng(2)
    cos, sin = R.rope_cache(40, 8)
    x = rng.standard_normal((2, 40, 8)).astype(np.float32)
    full = R.apply_rope(x, cos, sin)
    assert np.array_equal(R.apply_rope(x[:, 25:31], cos, sin, offset=25), full[:, 25:31])


def test_incremental_oracle_equals_full_forward_with_rope(monkeypatch):
    cfg = GPTConfig(96, 32, 4, 2, 24)
    w = make_weights(cfg, seed=5, rich=True)
    w.pop("pos_emb.weights")
    for i in range(cfg.num_layers):  # sharp attention, so positions move the logits
        for n in ("W_q", "W_k"):
            w[f"blocks.layers.{i}.mha.{n}.weights"] = w[f"blocks.layers.{i}.mha.{n}.weights"] * 25
    rope = R.rope_cache(cfg.max_seq_len, cfg.d_model // cfg.num_heads)
    ids = random_ids((2, 13), cfg.vocab_size, seed=3)
    full = R.forward(w, ids, cfg.num_heads, cfg.num_layers, rope)

    def incremental():
        kv = R.KVOracle(w, cfg.num_heads, cfg.num_layers, rope)
        return np.concatenate([kv.step(ids[:, :6]), kv.step(ids[:, 6:7]), kv.step(ids[:, 7:])], 1)

    assert np.abs(incremental() - full).max() < 1e-4
    # planted slip: every chunk rotated as if it started at position 0
    real = R.apply_rope
    monkeypatch.setattr(R, "apply_rope", lambda x, c, s, offset=0: real(x, c, s, 0))
    assert np.abs(incremental() - full).max() > 1e-2


def test_host_table_builder_matches_oracle_bit_for_bit():
    from nimbleml_amd.rope import build_rope_cache

    for seq, dk in [(2048, 64), (4096, 128), (24, 8)]:
        c1, s1 = build_rope_cache(seq, dk)
        c2, s2 = R.rope_cache(seq, dk)
        assert c1.dtype == np.float32 and np.array_equal(c1, c2) and np.array_equal(s1, s2)


def test_use_rope_model_has_no_position_table():
    import nimbleml_amd as nm

    m = nm.GPT(64, 32, 4, 1, 16, use_rope=True)
    names = {n for n, _ in nm.saveload.named_parameters(m)}
    assert "pos_emb.weights" not in names and "token_emb.weights" in names
    assert m._rope_cos.shape == (16, 8)


def _rope_fixture(name):
    from conftest import fixture_weights, golden

    f = golden(name)
    cfg, w = fixture_weights(f)
    assert int(f["rope"]) == 1 and "pos_emb.weights" not in w
    return f, cfg, w, R.rope_cache(cfg.max_seq_len, cfg.d_model // cfg.num_heads)


def test_oracle_matches_reference_rope_fixtures():
    """The reference's own use_rope=True GPT (tests/golden/make_golden.py): greedy tokens,
    all-position logits, the loss and top-k sampled tokens."""
    for name in ("tiny_rope_fp32", "tiny_rope_fp16"):
        f, cfg, w, rope = _rope_fixture(name)
        H, L = cfg.num_heads, cfg.num_layers
        n = f["greedy"].shape[1] - f["prompt"].shape[1]
        g = R.generate(w, f["prompt"], H, L, max_new_tokens=n, temperature=0.0, rope=rope)
        assert np.array_equal(g, f["greedy"]), name
        lg = R.forward(w, f["greedy"][:, :-1], H, L, rope)
        ref = f["greedy_logits"]
        if ref.dtype == np.float16:
            assert np.array_equal(lg, ref), name  # fp16: bit-exact op-by-op restatement
        else:
            assert np.abs(lg - ref).max() < 1e-5, name
        loss = R.compute_loss(w, f["loss_ids"], f["loss_labels"], H, L, rope=rope)
        rnd = np.float16 if ref.dtype == np.float16 else np.float32
        assert float(rnd(loss)) == float(f["loss"]), name
        toks = R.generate(w, f["prompt"], H, L, max_new_tokens=n, uniforms=f["topk_u"],
                          temperature=0.8, top_k=50, top_p=1.0, rope=rope)
        assert np.array_equal(toks, f["topk_tokens"]), name
