"""The backward oracle (``oracle/grad_ref.py``) pinned by what the mathematics fixes.
CPU only.

``loss_and_grads`` must return the exact gradient of the loss that the forward oracle
(``oracle/gpt_ref.py``, itself pinned bit-exact against the reference's golden vectors)
computes. Central finite differences of that independent forward, in float64, check it
coordinate by coordinate for every parameter kind, with and without ``ignore_index``
and rotary positions. Planted slips (a dropped RMSNorm term, the attention scale
applied twice, a RoPE rotation not inverted) must fail the same check.

The reference's own autograd is not run: its backward is what these checks restate,
and the finite differences fix it without it.
"""
import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle import grad_ref as G
from oracle.weights import GPTConfig, make_weights, random_ids, rope_weights

CFG = GPTConfig(48, 32, 4, 2, 16)  # vocab 48, d 32, 4 heads of 8, 2 layers, 16 positions

KINDS = ["token_emb.weights", "pos_emb.weights", "ln.gamma"] + [
    f"blocks.layers.{i}.{n}" for i in (0, 1) for n in (
        "ln1.gamma", "mha.W_q.weights", "mha.W_q.biases", "mha.W_k.weights", "mha.W_k.biases",
        "mha.W_v.weights", "mha.W_v.biases", "mha.W_o.weights", "mha.W_o.biases", "ln2.gamma",
        "ffn.dense1.weights", "ffn.dense1.biases", "ffn.dense2.weights", "ffn.dense2.biases")]


def _weights(rope=False, scale_qk=1.0):
    w = make_weights(CFG, seed=3, rich=True)
    w = {k: v.astype(np.float64) for k, v in w.items()}
    for k in w:  # larger weights: attention and GELU away from their linear regimes
        if k.endswith(".weights") and "emb" not in k:
            w[k] = w[k] * 12.0
    if rope:
        w = rope_weights(w)
    return w


def _loss(w, ids, labels, ignore=None, rope=None):
    return R.compute_loss(w, ids, labels, CFG.num_heads, CFG.num_layers, ignore_index=ignore,
                          rope=rope)


def _fd_check(w, ids, labels, ignore=None, rope=None, per_kind=3, seed=0, grad_fn=None,
              grad_scale=1.0):
    grad_fn = grad_fn or G.loss_and_grads
    loss, grads = grad_fn(w, ids, labels, CFG.num_heads, CFG.num_layers, ignore_index=ignore,
                          rope=rope, grad_scale=grad_scale)
    assert abs(loss - _loss(w, ids, labels, ignore, rope)) < 1e-12
    rng = np.random.default_rng(seed)
    worst = 0.0
    for name in KINDS:
        if name not in w:
            continue
        a = w[name]
        for _ in range(per_kind):
            idx = tuple(int(rng.integers(0, n)) for n in a.shape)
            if name == "token_emb.weights" and rng.random() < 0.5:
                idx = (int(ids.reshape(-1)[rng.integers(0, ids.size)]), idx[1])
            if name == "pos_emb.weights":
                idx = (int(rng.integers(0, ids.shape[1])), idx[1])
            h = 1e-5
            old = a[idx]
            a[idx] = old + h
            lp = _loss(w, ids, labels, ignore, rope)
            a[idx] = old - h
            lm = _loss(w, ids, labels, ignore, rope)
            a[idx] = old
            fd = grad_scale * (lp - lm) / (2 * h)
            got = grads[name][idx]
            err = abs(got - fd) / max(1e-4, abs(fd))
            worst = max(worst, err)
            assert err < 1e-5, (name, idx, got, fd)
    return loss, grads, worst


def _case(seed, b=2, s=7):
    ids = random_ids((b, s), CFG.vocab_size, seed)
    labels = random_ids((b * s,), CFG.vocab_size, seed + 1)
    return ids, labels


def test_fd_plain():
    ids, labels = _case(1)
    _fd_check(_weights(), ids, labels)


def test_fd_grad_scale_and_single_row():
    ids, labels = _case(2, b=1, s=1)
    _, grads, _ = _fd_check(_weights(), ids, labels, grad_scale=0.37)
    # one position: attention sees only itself, so the scores carry no gradient to W_q/W_k
    assert np.abs(grads["blocks.layers.0.mha.W_q.weights"]).max() < 1e-12
    assert np.abs(grads["blocks.layers.0.mha.W_k.weights"]).max() < 1e-12


def test_fd_ignore_index():
    ids, labels = _case(3, b=2, s=9)
    labels[[0, 4, 5, 11]] = -100
    _, grads, _ = _fd_check(_weights(), ids, labels, ignore=-100)
    # every label ignored: loss 0, no gradient anywhere
    loss, g0 = G.loss_and_grads(_weights(), ids, np.full(labels.shape, -100), CFG.num_heads,
                                CFG.num_layers, ignore_index=-100)
    assert loss == 0.0 and all(not np.any(v) for v in g0.values())


def test_fd_rope():
    ids, labels = _case(4, b=2, s=8)
    cos, sin = R.rope_cache(CFG.max_seq_len, CFG.head_dim)
    w = _weights(rope=True)
    _, grads, _ = _fd_check(w, ids, labels, rope=(cos.astype(np.float64), sin.astype(np.float64)))
    assert "pos_emb.weights" not in grads


def test_position_rows_past_sequence_get_no_gradient():
    ids, labels = _case(5, b=3, s=5)
    _, grads = G.loss_and_grads(_weights(), ids, labels, CFG.num_heads, CFG.num_layers)
    assert not np.any(grads["pos_emb.weights"][5:])
    assert np.any(grads["pos_emb.weights"][:5])
    # vocabulary rows neither in ids nor reached by the head's softmax still get the
    # softmax part of the tied head's gradient: never exactly zero
    assert np.all(np.abs(grads["token_emb.weights"]).sum(axis=1) > 0)


def test_gradients_are_linear_in_grad_scale():
    ids, labels = _case(6)
    w = _weights()
    _, g1 = G.loss_and_grads(w, ids, labels, CFG.num_heads, CFG.num_layers)
    _, g2 = G.loss_and_grads(w, ids, labels, CFG.num_heads, CFG.num_layers, grad_scale=-2.5)
    for k in g1:
        assert np.allclose(g2[k], -2.5 * g1[k], rtol=1e-12, atol=1e-15), k


@pytest.mark.parametrize("slip", ["rms_coef", "double_scale", "rope_forward"])
def test_planted_slips_fail_the_check(monkeypatch, slip):
    ids, labels = _case(7, b=2, s=8)
    rope = None
    w = _weights()
    if slip == "rms_coef":
        def bad(grad, x, g, ms, rms, eps=G.RMS_EPS):
            x_hat = x / rms
            return (grad * g) / rms, np.sum(grad * x_hat, axis=0)
        monkeypatch.setattr(G, "_rms_bwd", bad)
    elif slip == "double_scale":  # the scores gradient divided by sqrt(dk) twice
        orig = G.loss_and_grads

        def bad(w, ids, labels, nh, nl, ignore_index=None, rope=None, grad_scale=1.0):
            loss, g = orig(w, ids, labels, nh, nl, ignore_index, rope, grad_scale)
            for nm in ("W_q", "W_k"):
                for i in range(nl):
                    for suf in (".weights", ".biases"):
                        k = f"blocks.layers.{i}.mha.{nm}{suf}"
                        g[k] = g[k] / (CFG.head_dim ** 0.5)
            return loss, g
        monkeypatch.setattr(G, "loss_and_grads", bad)
    else:
        cos, sin = R.rope_cache(CFG.max_seq_len, CFG.head_dim)
        rope = (cos.astype(np.float64), sin.astype(np.float64))
        w = _weights(rope=True)
        monkeypatch.setattr(G, "_rope_inv", lambda x, c, s: R.apply_rope(x, c, s))
    with pytest.raises(AssertionError):
        _fd_check(w, ids, labels, rope=rope, per_kind=4, grad_fn=G.loss_and_grads)


# ------------------------------------------------------- module-level vector-Jacobian products
# Each VJP oracle is pinned by central differences of the forward oracle (oracle/gpt_ref.py:
# R.block / R.mha / R.ffn / R.rmsnorm): d<dout, f(θ)>/dθ at random coordinates of the input
# and of every parameter the module reads.

def _module_case(seed, b=2, s=6):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, s, CFG.d_model))
    dout = rng.standard_normal((b, s, CFG.d_model))
    return x, dout


def _mixed_mask(s, seed):
    m = np.where(np.random.default_rng(seed).random((s, s)) < 0.3, -np.inf, 0.0)
    np.fill_diagonal(m, 0.0)  # every query keeps one key
    return m + np.random.default_rng(seed + 1).standard_normal((s, s)) * 0.5 * (m == 0)


def _fd_vjp(f, w, x, dout, dx, grads, names, per_kind=3, seed=0):
    """Central differences of <dout, f(w, x)> against dx and grads[name]."""
    rng = np.random.default_rng(seed)

    def obj():
        return float(np.sum(dout * f(w, x)))

    worst = 0.0
    for name in ["x"] + list(names):
        a = x if name == "x" else w[name]
        got_all = dx if name == "x" else grads[name]
        for _ in range(per_kind):
            idx = tuple(int(rng.integers(0, n)) for n in a.shape)
            h = 1e-5
            old = a[idx]
            a[idx] = old + h
            lp = obj()
            a[idx] = old - h
            lm = obj()
            a[idx] = old
            fd = (lp - lm) / (2 * h)
            # the objective is O(100): differences carry ~1e-9 of rounding noise
            err = abs(got_all[idx] - fd) / max(1e-2, abs(fd))
            worst = max(worst, err)
            assert err < 1e-5, (name, idx, got_all[idx], fd)
    return worst


def _block_names(i):
    return [n for n in KINDS if n.startswith(f"blocks.layers.{i}.")]


@pytest.mark.parametrize("mask_kind", ["causal", "none", "mixed"])
def test_fd_block_vjp(mask_kind):
    w = _weights()
    x, dout = _module_case(20)
    s = x.shape[1]
    mask = {"causal": R.causal_mask(s, np.float64), "none": None,
            "mixed": _mixed_mask(s, 3)}[mask_kind]
    out, dx, grads = G.blocks_vjp(w, [1], x, dout, CFG.num_heads, mask)
    assert np.allclose(out, R.block(x, w, 1, CFG.num_heads, mask), rtol=1e-12, atol=1e-12)
    _fd_vjp(lambda w_, x_: R.block(x_, w_, 1, CFG.num_heads, mask), w, x, dout, dx, grads,
            _block_names(1))
    assert not any(np.any(grads[n]) for n in _block_names(0))  # other layers untouched


def test_fd_block_vjp_rope():
    w = _weights(rope=True)
    x, dout = _module_case(21, s=7)
    cos, sin = R.rope_cache(CFG.max_seq_len, CFG.head_dim)
    rc = (cos.astype(np.float64), sin.astype(np.float64))
    mask = R.causal_mask(7, np.float64)
    out, dx, grads = G.blocks_vjp(w, [0], x, dout, CFG.num_heads, mask, rope=rc)
    _fd_vjp(lambda w_, x_: R.block(x_, w_, 0, CFG.num_heads, mask, rc), w, x, dout, dx, grads,
            _block_names(0))


def test_fd_trunk_vjp():
    w = _weights()
    x, dout = _module_case(22)
    mask = R.causal_mask(6, np.float64)
    w["final.gamma"] = 1.0 + 0.3 * np.random.default_rng(9).standard_normal(CFG.d_model)

    def trunk(w_, x_):
        h = x_
        for i in range(CFG.num_layers):
            h = R.block(h, w_, i, CFG.num_heads, mask)
        return R.rmsnorm(h, w_["final.gamma"])

    out, dx, grads = G.blocks_vjp(w, list(range(CFG.num_layers)), x, dout, CFG.num_heads, mask,
                                  final_gamma=w["final.gamma"])
    assert np.allclose(out, trunk(w, x), rtol=1e-12, atol=1e-12)
    _fd_vjp(trunk, w, x, dout, dx, grads,
            _block_names(0) + _block_names(1) + ["final.gamma"])


@pytest.mark.parametrize("mask_kind", ["none", "mixed"])
def test_fd_mha_vjp(mask_kind):
    w = _weights()
    x, dout = _module_case(23, s=5)
    mask = None if mask_kind == "none" else _mixed_mask(5, 4)
    pm = "blocks.layers.0.mha."
    out, dx, grads = G.mha_vjp(w, pm, x, dout, CFG.num_heads, mask)
    assert np.allclose(out, R.mha(x, w, pm, CFG.num_heads, mask), rtol=1e-12, atol=1e-12)
    _fd_vjp(lambda w_, x_: R.mha(x_, w_, pm, CFG.num_heads, mask), w, x, dout, dx, grads,
            [n for n in _block_names(0) if ".mha." in n])


def test_fd_ffn_dense_embedding_vjp():
    w = _weights()
    x, dout = _module_case(24, s=3)
    pf = "blocks.layers.1.ffn."
    out, dx, grads = G.ffn_vjp(w, pf, x, dout)
    assert np.allclose(out, R.ffn(x, w, pf), rtol=1e-12, atol=1e-12)
    _fd_vjp(lambda w_, x_: R.ffn(x_, w_, pf), w, x, dout, dx, grads,
            [n for n in _block_names(1) if ".ffn." in n])
    # Dense: a linear map, so its VJP is fixed by the transposes; checked against
    # differences all the same
    W, bvec = w[pf + "dense1.weights"], w[pf + "dense1.biases"]
    dy = np.random.default_rng(25).standard_normal((2, 3, W.shape[1]))
    out, dx, dW, db = G.dense_vjp(W, bvec, x, dy)
    _fd_vjp(lambda w_, x_: x_ @ w_["W"] + w_["b"], {"W": W, "b": bvec}, x, dy, dx,
            {"W": dW, "b": db}, ["W", "b"])
    # Embedding: each id's rows of dout summed; a repeated id gets both
    ids = np.array([[3, 7, 3], [0, 3, 47]])
    g = G.embedding_vjp(CFG.vocab_size, ids, dout)
    assert np.allclose(g[3], dout[0, 0] + dout[0, 2] + dout[1, 1])
    assert np.allclose(g[47], dout[1, 2]) and not np.any(g[[1, 2, 4]])


def test_planted_mask_slip_fails_the_module_check():
    """A backward that forgets the additive mask (the gradient of the unmasked attention)
    must fail the differences of the masked forward."""
    w = _weights()
    x, dout = _module_case(26, s=5)
    mask = _mixed_mask(5, 8)
    pm = "blocks.layers.0.mha."
    _, dx, grads = G.mha_vjp(w, pm, x, dout, CFG.num_heads, None)
    with pytest.raises(AssertionError):
        _fd_vjp(lambda w_, x_: R.mha(x_, w_, pm, CFG.num_heads, mask), w, x, dout, dx, grads,
                [n for n in _block_names(0) if ".mha." in n])


def test_fd_logits_vjp():
    """GPT.forward's backward for a given d(loss)/d(logits), against differences of the
    forward oracle's <dlogits, logits>."""
    w = _weights()
    ids, _ = _case(27, b=2, s=6)
    dl = np.random.default_rng(28).standard_normal((2, 6, CFG.vocab_size))
    logits, grads = G.logits_vjp(w, ids, dl, CFG.num_heads, CFG.num_layers)
    want = R.forward(w, ids, CFG.num_heads, CFG.num_layers)
    assert np.allclose(logits, want, rtol=1e-12, atol=1e-12)
    rng = np.random.default_rng(29)
    for name in KINDS:
        a = w[name]
        for _ in range(2):
            idx = tuple(int(rng.integers(0, n)) for n in a.shape)
            if name == "pos_emb.weights":
                idx = (int(rng.integers(0, 6)), idx[1])
            h = 1e-5
            old = a[idx]
            a[idx] = old + h
            lp = float(np.sum(dl * R.forward(w, ids, CFG.num_heads, CFG.num_layers)))
            a[idx] = old - h
            lm = float(np.sum(dl * R.forward(w, ids, CFG.num_heads, CFG.num_layers)))
            a[idx] = old
            fd = (lp - lm) / (2 * h)
            assert abs(grads[name][idx] - fd) <= 1e-5 * max(1e-2, abs(fd)), (name, idx)
