"""Module-level autograd on the device: ``out = module(x)`` then ``out.backward(dout)``
(the closures of neural_network/transformer_fused.py:65-78, :128-136,
neural_network/attention.py:103-119, layers/dense.py:81-94, layers/rms_norm.py:76-94,
layers/embedding.py:63-69 and neural_network/feed_forward.py:105-129, run by
Tensor.backward in reverse topological order, utils/tensor.py:286-332).

Every gradient — the input's and each parameter's, in the reference layouts — is compared
with the float64 vector-Jacobian oracles of oracle/grad_ref.py (blocks_vjp, mha_vjp,
ffn_vjp, dense_vjp, embedding_vjp; pinned by finite differences in test_grad_oracle.py)
at the same weights, input and dout.

Tolerances: float32, per tensor, max |device − oracle| ≤ 2e-5 · max |oracle| + 1e-7 (the
backward's float32 sums in another order; a wrong index, transposed operand or dropped
term moves a gradient by O(1) of its size). float16: ≤ 1.5e-2 · max |oracle| (the fp16
rounding of activations and activation gradients, as for the GPT backward)."""
import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle import grad_ref as G
from oracle.weights import GPTConfig, make_weights, rope_weights

pytestmark = pytest.mark.gpu

CFG = GPTConfig(vocab_size=256, d_model=64, num_heads=4, num_layers=2, max_seq_len=64)
RTOL = 2e-5
RTOL16 = 1.5e-2


@pytest.fixture
def dtype_ctx(request, gpu):
    import nimbleml_amd as nm

    old = nm.np_backend.dtype
    nm.set_dtype(np.dtype(request.param).name)
    yield np.dtype(request.param)
    nm.set_dtype(np.dtype(old).name)


def _weights(dt, seed=3, rope=False, scale=4.0):
    w = make_weights(CFG, seed=seed, dtype=np.float32, rich=True)
    for k in w:  # larger weights: attention and GELU away from their linear regimes
        if k.endswith(".weights") and "emb" not in k:
            w[k] = (w[k] * np.float32(scale)).astype(np.float32)
    if rope:
        w = rope_weights(w)
    return {k: v.astype(dt) for k, v in w.items()}


def _gpt(w, dt, **flags):
    import nimbleml_amd as nm

    return nm.GPT.from_arrays(w, CFG.vocab_size, CFG.d_model, CFG.num_heads, CFG.num_layers,
                              CFG.max_seq_len, dtype=dt, **flags)


def _w64(w):
    return {k: v.astype(np.float64) for k, v in w.items()}


def _x(shape, seed, dt, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(dt)


def _check(got, want, dt, name, scale=0.0):
    """``scale``: the gradient scale to measure against when ``want`` is (near) zero."""
    assert got is not None, f"{name}: no gradient"
    g = np.asarray(got, dtype=np.float64).reshape(want.shape)
    err = float(np.abs(g - want).max())
    top = max(float(np.abs(want).max()), scale)
    bound = (RTOL * top + 1e-7) if np.dtype(dt) == np.float32 else RTOL16 * max(top, 1e-3)
    assert err <= bound, (name, err, bound)
    return err / max(top, 1e-30)


def _block_params(blk, i):
    """{oracle name: Tensor} of one FusedTransformerBlock."""
    p = f"blocks.layers.{i}."
    out = {p + "ln1.gamma": blk.ln1.gamma, p + "ln2.gamma": blk.ln2.gamma}
    for n in ("W_q", "W_k", "W_v", "W_o"):
        d = getattr(blk.mha, n)
        out[p + f"mha.{n}.weights"] = d.weights
        out[p + f"mha.{n}.biases"] = d.biases
    for n in ("dense1", "dense2"):
        d = getattr(blk.ffn, n)
        out[p + f"ffn.{n}.weights"] = d.weights
        out[p + f"ffn.{n}.biases"] = d.biases
    return out


def _zero(params):
    for t in params:
        t.grad = None


def _mixed_mask(s, dt, seed=5):
    rng = np.random.default_rng(seed)
    m = np.where(rng.random((s, s)) < 0.3, -np.inf, 0.0)
    np.fill_diagonal(m, 0.0)  # every query keeps one key
    m = m + rng.standard_normal((s, s)) * 0.5 * (m == 0)
    return m.astype(dt)


@pytest.mark.parametrize("dtype_ctx", [np.float32, np.float16], indirect=True)
@pytest.mark.parametrize("mask_kind", ["causal", "mixed", "zeros"])
def test_block_backward(dtype_ctx, mask_kind):
    """FusedTransformerBlock: mask=None (causal, the MFMA backward at dk 16), an arbitrary
    additive mask and an all-zero one (both non-causal: the scalar kernels); s = 37 leaves
    partial tiles."""
    import nimbleml_amd as nm

    dt = dtype_ctx
    w = _weights(dt)
    blk = _gpt(w, dt)._block_list[1]
    b, s = 2, 37
    x = _x((b, s, CFG.d_model), 1, dt)
    dout = _x((b, s, CFG.d_model), 2, dt)
    mask = {"causal": None, "mixed": _mixed_mask(s, dt), "zeros": np.zeros((s, s), dt)}[mask_kind]
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    out = blk(xt, None if mask is None else nm.Tensor(mask, mask.shape))
    out.backward(dout.reshape(-1))
    omask = R.causal_mask(s, np.float64) if mask is None else mask.astype(np.float64)
    want_out, want_dx, want = G.blocks_vjp(_w64(w), [1], x.astype(np.float64),
                                           dout.astype(np.float64), CFG.num_heads, omask)
    worst = _check(out.numpy(), want_out, dt, "out")
    worst = max(worst, _check(xt.grad, want_dx, dt, "x"))
    for name, t in _block_params(blk, 1).items():
        if name.endswith("W_k.biases"):  # exactly 0: softmax ignores a per-row shift
            assert np.abs(np.asarray(t.grad, np.float64)).max() <= 1e-3
            continue
        worst = max(worst, _check(t.grad, want[name], dt, name))
    print(f"block {mask_kind} {dt.name}: worst relative {worst:.3g}")


def test_block_backward_rope_and_single_position(gpu):
    """RoPE tables of a use_rope model (the inverse rotation in the backward), and s = 1."""
    import nimbleml_amd as nm

    w = _weights(np.float32, seed=4, rope=True)
    blk = _gpt(w, np.float32, use_rope=True)._block_list[0]
    cos, sin = R.rope_cache(CFG.max_seq_len, CFG.d_model // CFG.num_heads)
    rc = (cos.astype(np.float64), sin.astype(np.float64))
    for s in (23, 1):
        x = _x((3, s, CFG.d_model), 3 + s, np.float32)
        dout = _x((3, s, CFG.d_model), 4 + s, np.float32)
        xt = nm.Tensor(x, x.shape, requires_grad=True)
        _zero(blk.parameters())
        out = blk(xt)
        out.backward(dout)
        _, want_dx, want = G.blocks_vjp(_w64(w), [0], x.astype(np.float64),
                                        dout.astype(np.float64), CFG.num_heads,
                                        R.causal_mask(s, np.float64), rope=rc)
        _check(xt.grad, want_dx, np.float32, f"x s={s}")
        # one position: the scores carry no gradient, so W_q and W_k get exactly 0 from the
        # oracle and float32 rounding noise from the device, measured at W_v's scale
        vscale = float(np.abs(want["blocks.layers.0.mha.W_v.weights"]).max())
        for name, t in _block_params(blk, 0).items():
            if not name.endswith("W_k.biases"):
                _check(t.grad, want[name], np.float32, f"{name} s={s}", scale=vscale)


def test_trunk_backward_and_embedding_chain(gpu):
    """Embedding → FusedGPTTrunk (every block, then the final RMSNorm) as one graph:
    Tensor.backward runs the trunk's closure, then the embedding's scatter with the
    trunk's input gradient."""
    import nimbleml_amd as nm

    w = _weights(np.float32, seed=6)
    wt = {k.replace("blocks.layers.", "blocks.blocks."): v for k, v in w.items()}
    wt["blocks.ln.gamma"] = w["ln.gamma"]
    m = _gpt(wt, np.float32, fused_trunk=True)
    trunk = m.blocks
    ids = np.random.default_rng(7).integers(0, CFG.vocab_size, (2, 30))
    ids[0, :5] = 9  # repeated ids: their rows add up
    h = m.token_emb(nm.Tensor.from_int64(ids, ids.shape))
    out = trunk(h)
    dout = _x(out.shape, 8, np.float32)
    out.backward(dout)
    x64 = w["token_emb.weights"].astype(np.float64)[ids]
    want_out, want_dx, want = G.blocks_vjp(_w64(w), list(range(CFG.num_layers)), x64,
                                           dout.astype(np.float64), CFG.num_heads,
                                           R.causal_mask(30, np.float64),
                                           final_gamma=w["ln.gamma"].astype(np.float64))
    _check(out.numpy(), want_out, np.float32, "out")
    for i, blk in enumerate(trunk.blocks):
        for name, t in _block_params(blk, i).items():
            if not name.endswith("W_k.biases"):
                _check(t.grad, want[name], np.float32, name)
    _check(trunk.ln.gamma.grad, want["final.gamma"], np.float32, "final norm")
    _check(m.token_emb.weights.grad, G.embedding_vjp(CFG.vocab_size, ids, want_dx),
           np.float32, "token_emb")


@pytest.mark.parametrize("dtype_ctx", [np.float32, np.float16], indirect=True)
@pytest.mark.parametrize("mask_kind", ["none", "causal", "mixed"])
def test_mha_backward(dtype_ctx, mask_kind):
    """MultiHeadAttention: mask=None attends to every key; the causal mask takes the causal
    kernels; an arbitrary mask the scalar ones."""
    import nimbleml_amd as nm

    dt = dtype_ctx
    w = _weights(dt, seed=9)
    mha = _gpt(w, dt)._block_list[0].mha
    s = 29
    x = _x((2, s, CFG.d_model), 10, dt)
    dout = _x((2, s, CFG.d_model), 11, dt)
    mask = {"none": None, "causal": R.causal_mask(s, dt), "mixed": _mixed_mask(s, dt, 6)}[mask_kind]
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    out = mha(xt, None if mask is None else nm.Tensor(mask, mask.shape))
    out.backward(dout)
    pm = "blocks.layers.0.mha."
    want_out, want_dx, want = G.mha_vjp(_w64(w), pm, x.astype(np.float64),
                                        dout.astype(np.float64), CFG.num_heads,
                                        None if mask is None else mask.astype(np.float64))
    _check(out.numpy(), want_out, dt, "out")
    _check(xt.grad, want_dx, dt, "x")
    for n in ("W_q", "W_k", "W_v", "W_o"):
        d = getattr(mha, n)
        _check(d.weights.grad, want[pm + n + ".weights"], dt, n)
        if n != "W_k":
            _check(d.biases.grad, want[pm + n + ".biases"], dt, n + " bias")


@pytest.mark.parametrize("dtype_ctx", [np.float32, np.float16], indirect=True)
def test_dense_ffn_rmsnorm_embedding_backward(dtype_ctx):
    import nimbleml_amd as nm

    dt = dtype_ctx
    w = _weights(dt, seed=12)
    blk = _gpt(w, dt)._block_list[1]
    pf = "blocks.layers.1.ffn."
    x = _x((3, 17, CFG.d_model), 13, dt)
    dout = _x((3, 17, CFG.d_model), 14, dt)
    # FeedForward: the GELU derivative fused into the second projection's backward
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    out = blk.ffn(xt)
    out.backward(dout)
    want_out, want_dx, want = G.ffn_vjp(_w64(w), pf, x.astype(np.float64),
                                        dout.astype(np.float64))
    _check(out.numpy(), want_out, dt, "ffn out")
    _check(xt.grad, want_dx, dt, "ffn x")
    for n in ("dense1", "dense2"):
        d = getattr(blk.ffn, n)
        _check(d.weights.grad, want[pf + n + ".weights"], dt, n)
        _check(d.biases.grad, want[pf + n + ".biases"], dt, n + " bias")
    # Dense on its own: W_o of the attention
    dense = blk.mha.W_o
    _zero(dense.parameters())
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    out = dense(xt)
    out.backward(dout)
    W, bvec = w["blocks.layers.1.mha.W_o.weights"], w["blocks.layers.1.mha.W_o.biases"]
    o64, dx64, dw64, db64 = G.dense_vjp(W.astype(np.float64), bvec.astype(np.float64),
                                        x.astype(np.float64), dout.astype(np.float64))
    _check(xt.grad, dx64, dt, "dense x")
    _check(dense.weights.grad, dw64, dt, "dense W")
    _check(dense.biases.grad, db64, dt, "dense b")
    # RMSNorm
    ln = blk.ln2
    _zero(ln.parameters())
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    out = ln(xt)
    out.backward(dout)
    gx, gg = G.rmsnorm_backward(dout.astype(np.float64), x.astype(np.float64),
                                w["blocks.layers.1.ln2.gamma"].astype(np.float64))
    _check(xt.grad, gx, dt, "rmsnorm x")
    _check(ln.gamma.grad, gg, dt, "rmsnorm gamma")


def test_embedding_backward_and_prefix(gpu):
    """Token rows scatter-added in row order (repeated ids), forward_prefix's rows [0, s)."""
    import nimbleml_amd as nm

    w = _weights(np.float32, seed=15)
    m = _gpt(w, np.float32)
    emb = m.token_emb
    ids = np.array([[3, 7, 3, 3], [0, 255, 7, 1]])
    dout = _x((2, 4, CFG.d_model), 16, np.float32)
    out = emb(nm.Tensor.from_int64(ids, ids.shape))
    out.backward(dout)
    _check(emb.weights.grad, G.embedding_vjp(CFG.vocab_size, ids, dout.astype(np.float64)),
           np.float32, "embedding")
    pos = m.pos_emb
    p = pos.forward_prefix(11)
    g = _x((11, CFG.d_model), 17, np.float32)
    p.backward(g)
    got = np.asarray(pos.weights.grad).reshape(pos.weights.shape)
    assert np.array_equal(got[:11], g) and not np.any(got[11:])


def test_outstanding_graphs_recompute_and_accumulate(gpu):
    """Two forwards of one block before either backward: the first output's backward
    recomputes its saved forward (the device model keeps one); gradients add up over
    backward calls (Tensor._accumulate_grad), and retain_graph keeps the closure."""
    import nimbleml_amd as nm

    w = _weights(np.float32, seed=18)
    blk = _gpt(w, np.float32)._block_list[0]
    x1, x2 = _x((2, 20, CFG.d_model), 19, np.float32), _x((1, 33, CFG.d_model), 20, np.float32)
    d1, d2 = _x((2, 20, CFG.d_model), 21, np.float32), _x((1, 33, CFG.d_model), 22, np.float32)
    t1 = nm.Tensor(x1, x1.shape, requires_grad=True)
    t2 = nm.Tensor(x2, x2.shape, requires_grad=True)
    o1 = blk(t1)
    o2 = blk(t2)
    o1.backward(d1, retain_graph=True)
    o2.backward(d2)
    # the same graph again: backward adds d1 to o1.grad (now 2·d1, utils/tensor.py:307) and the
    # closure reads o1.grad, so o1's gradients count 1 + 2 = 3 times, as in the reference
    o1.backward(d1)
    mask1, mask2 = R.causal_mask(20, np.float64), R.causal_mask(33, np.float64)
    _, dx1, g1 = G.blocks_vjp(_w64(w), [0], x1.astype(np.float64), d1.astype(np.float64),
                              CFG.num_heads, mask1)
    _, dx2, g2 = G.blocks_vjp(_w64(w), [0], x2.astype(np.float64), d2.astype(np.float64),
                              CFG.num_heads, mask2)
    _check(t1.grad, 3 * dx1, np.float32, "x1")
    _check(t2.grad, dx2, np.float32, "x2")
    for name, t in _block_params(blk, 0).items():
        if not name.endswith("W_k.biases"):
            _check(t.grad, 3 * g1[name] + g2[name], np.float32, name)
    assert o1._backward is None and not o1._prev  # released after the last backward


def test_no_grad_and_frozen_parameters(gpu):
    """no_grad: no closure; parameters with requires_grad=False get no gradient while the
    input still does."""
    import nimbleml_amd as nm

    w = _weights(np.float32, seed=23)
    blk = _gpt(w, np.float32)._block_list[0]
    x = _x((1, 9, CFG.d_model), 24, np.float32)
    with nm.no_grad():
        out = blk(nm.Tensor(x, x.shape, requires_grad=True))
    assert not out.requires_grad and out._backward is None
    for p in blk.parameters():
        p.requires_grad = False
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    out = blk(xt)
    assert out.requires_grad and xt in out._prev
    out.backward(np.ones(out.size, np.float32))
    assert all(p.grad is None for p in blk.parameters())
    _, dx, _ = G.blocks_vjp(_w64(w), [0], x.astype(np.float64), np.ones(x.shape),
                            CFG.num_heads, R.causal_mask(9, np.float64))
    _check(xt.grad, dx, np.float32, "x")


@pytest.mark.parametrize("dt", [np.float32, np.float16])
@pytest.mark.parametrize("dims", [(128, 192, 2, 1, 64), (128, 512, 2, 1, 64)],
                         ids=lambda d: f"dk{d[1] // d[2]}")
def test_padded_head_dims_with_masks(gpu, dims, dt):
    """Head dims 96 and 256 (the scalar backward on tiles padded to 128 / 256 columns):
    MultiHeadAttention with an arbitrary mask (non-causal) and the block with its causal
    default, every gradient against the oracle."""
    import nimbleml_amd as nm

    cfg = GPTConfig(*dims)
    old = nm.np_backend.dtype
    nm.set_dtype(np.dtype(dt).name)
    try:
        w = make_weights(cfg, seed=27, dtype=np.float32, rich=True)
        w = {k: v.astype(dt) for k, v in w.items()}
        m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, dtype=dt)
        blk = m._block_list[0]
        s = 21
        x = _x((2, s, cfg.d_model), 28, dt)
        dout = _x((2, s, cfg.d_model), 29, dt)
        mask = _mixed_mask(s, dt, 7)
        xt = nm.Tensor(x, x.shape, requires_grad=True)
        out = blk.mha(xt, nm.Tensor(mask, mask.shape))
        out.backward(dout)
        pm = "blocks.layers.0.mha."
        _, want_dx, want = G.mha_vjp(_w64(w), pm, x.astype(np.float64), dout.astype(np.float64),
                                     cfg.num_heads, mask.astype(np.float64))
        _check(xt.grad, want_dx, dt, "mha x")
        for n in ("W_q", "W_v", "W_o"):
            _check(getattr(blk.mha, n).weights.grad, want[pm + n + ".weights"], dt, n)
        _zero(blk.parameters())
        xt = nm.Tensor(x, x.shape, requires_grad=True)
        out = blk(xt)
        out.backward(dout)
        _, want_dx, want = G.blocks_vjp(_w64(w), [0], x.astype(np.float64),
                                        dout.astype(np.float64), cfg.num_heads,
                                        R.causal_mask(s, np.float64))
        _check(xt.grad, want_dx, dt, "block x")
        for name, t in _block_params(blk, 0).items():
            if not name.endswith("W_k.biases"):
                _check(t.grad, want[name], dt, name)
    finally:
        nm.set_dtype(np.dtype(old).name)


@pytest.mark.parametrize("dt", [np.float32, np.float16])
@pytest.mark.parametrize("rope", [False, True])
def test_gpt_forward_logits_backward(gpu, dt, rope):
    """GPT.forward's logits carry the whole model's backward: logits.backward(dlogits)
    gives every parameter's gradient (the tied embedding gets both the head's and the
    scatter's), against the oracle's logits_vjp; under no_grad the logits carry none."""
    import nimbleml_amd as nm

    w = _weights(dt, seed=30)
    if rope:  # no position table (W_q and W_k at the test's common scale)
        w.pop("pos_emb.weights")
    m = _gpt(w, dt, use_rope=rope)
    ids = np.random.default_rng(31).integers(0, CFG.vocab_size, (2, 33))
    dl = (np.random.default_rng(32).standard_normal((2, 33, CFG.vocab_size)) * 0.1).astype(dt)
    logits = m.forward(ids)
    assert logits.requires_grad
    logits.backward(dl)
    rc = None
    if rope:
        cos, sin = R.rope_cache(CFG.max_seq_len, CFG.d_model // CFG.num_heads)
        rc = (cos.astype(np.float64), sin.astype(np.float64))
    want_logits, want = G.logits_vjp(_w64(w), ids, dl.astype(np.float64), CFG.num_heads,
                                     CFG.num_layers, rope=rc)
    _check(logits.numpy(), want_logits, dt, "logits")
    named = {"token_emb.weights": m.token_emb.weights, "ln.gamma": m.ln.gamma}
    if not rope:
        named["pos_emb.weights"] = m.pos_emb.weights
    for i, blk in enumerate(m._block_list):
        named.update(_block_params(blk, i))
    for name, t in named.items():
        if not name.endswith("W_k.biases"):
            _check(t.grad, want[name], dt, name)
    with nm.no_grad():
        assert not m.forward(ids).requires_grad


def test_backward_after_the_device_copy_was_rebuilt(gpu):
    """A longer sequence rebuilds the block's device model (a larger position capacity)
    between a forward and its backward: the closure keeps the model its forward ran on, so
    the first output's gradients are still right."""
    import nimbleml_amd as nm

    w = _weights(np.float32, seed=33)
    blk = _gpt(w, np.float32)._block_list[1]
    x1 = _x((1, 20, CFG.d_model), 34, np.float32)
    d1 = _x((1, 20, CFG.d_model), 35, np.float32)
    t1 = nm.Tensor(x1, x1.shape, requires_grad=True)
    o1 = blk(t1)
    before = blk.__dict__["_device_copies"]["blocks"][1]
    x2 = _x((1, 64, CFG.d_model), 36, np.float32)  # capacity 64 → this fits; 65 would not
    blk(nm.Tensor(x2, x2.shape))
    assert blk.__dict__["_device_copies"]["blocks"][1] is before
    blk.mha.W_o.weights.data = blk.mha.W_o.weights.data.copy()  # a new buffer: a new key
    blk.mha.W_o.weights._bump_version()
    blk(nm.Tensor(x2, x2.shape))
    assert blk.__dict__["_device_copies"]["blocks"][1] is not before
    o1.backward(d1)
    _, dx1, g1 = G.blocks_vjp(_w64(w), [1], x1.astype(np.float64), d1.astype(np.float64),
                              CFG.num_heads, R.causal_mask(20, np.float64))
    _check(t1.grad, dx1, np.float32, "x1")
    for name, t in _block_params(blk, 1).items():
        if not name.endswith("W_k.biases"):
            _check(t.grad, g1[name], np.float32, name)


def test_recompute_keeps_the_forward_mask(gpu):
    """A masked output whose saved forward was replaced recomputes with its own mask (the
    device copy of the mask stays alive with the output's closure): block and attention."""
    import gc

    import nimbleml_amd as nm

    w = _weights(np.float32, seed=37)
    blk = _gpt(w, np.float32)._block_list[0]
    s = 19
    x1, d1 = _x((2, s, CFG.d_model), 38, np.float32), _x((2, s, CFG.d_model), 39, np.float32)
    mask = _mixed_mask(s, np.float32, 9)
    for mod, vjp in ((blk, "block"), (blk.mha, "mha")):
        _zero(blk.parameters())
        t1 = nm.Tensor(x1, x1.shape, requires_grad=True)
        o1 = mod(t1, nm.Tensor(mask, mask.shape))
        mod(nm.Tensor(x1[:1], (1, s, CFG.d_model)))  # another saving forward, no mask
        gc.collect()
        o1.backward(d1)
        if vjp == "block":
            _, dx, g = G.blocks_vjp(_w64(w), [0], x1.astype(np.float64), d1.astype(np.float64),
                                    CFG.num_heads, mask.astype(np.float64))
            names = _block_params(blk, 0)
        else:
            _, dx, g = G.mha_vjp(_w64(w), "blocks.layers.0.mha.", x1.astype(np.float64),
                                 d1.astype(np.float64), CFG.num_heads, mask.astype(np.float64))
            names = {k: v for k, v in _block_params(blk, 0).items() if ".mha." in k}
        _check(t1.grad, dx, np.float32, f"{vjp} x")
        for name, t in names.items():
            if not name.endswith("W_k.biases"):
                _check(t.grad, g[name], np.float32, f"{vjp} {name}")


@pytest.mark.parametrize("dtype_ctx", [np.float32, np.float16], indirect=True)
def test_sequential_blocks_and_unbiased_dense(dtype_ctx):
    """GPT.blocks as a Sequential of blocks (no fused trunk): one closure per block, run by
    Tensor.backward from the last block to the first; a Dense without bias
    (layers/dense.py:16-25, bias=False) gets only its weight gradient."""
    import nimbleml_amd as nm

    dt = dtype_ctx
    w = _weights(dt, seed=40)
    m = _gpt(w, dt)
    x = _x((2, 26, CFG.d_model), 41, dt)
    dout = _x((2, 26, CFG.d_model), 42, dt)
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    out = m.blocks(xt)
    out.backward(dout)
    want_out, want_dx, want = G.blocks_vjp(_w64(w), list(range(CFG.num_layers)),
                                           x.astype(np.float64), dout.astype(np.float64),
                                           CFG.num_heads, R.causal_mask(26, np.float64))
    _check(out.numpy(), want_out, dt, "out")
    _check(xt.grad, want_dx, dt, "x")
    for i, blk in enumerate(m._block_list):
        for name, t in _block_params(blk, i).items():
            if not name.endswith("W_k.biases"):
                _check(t.grad, want[name], dt, name)
    dense = nm.Dense(CFG.d_model, 40, bias=False)
    xt = nm.Tensor(x, x.shape, requires_grad=True)
    y = dense(xt)
    dy = _x(y.shape, 43, dt)
    y.backward(dy)
    W = np.asarray(dense.weights.data, np.float64).reshape(CFG.d_model, 40)
    _, dx64, dw64, _ = G.dense_vjp(W, None, x.astype(np.float64), dy.astype(np.float64))
    _check(xt.grad, dx64, dt, "dense x")
    _check(dense.weights.grad, dw64, dt, "dense W")
    assert dense.biases is None
