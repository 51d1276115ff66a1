"""Module-level forwards on the GPU against the oracle (row a4 of the drop-in API).

Each module of nimbleml_amd.layers runs its forward through the HIP kernels and is
compared with the CPU restatement of the reference's arithmetic in oracle/gpt_ref.py:
Dense (x·W + b), Embedding / forward_prefix (row gathers: bit-exact), RMSNorm,
FeedForward, MultiHeadAttention (no mask, the causal mask, an arbitrary additive mask),
FusedTransformerBlock (with and without RoPE), FusedGPTTrunk and a Sequential of
blocks, plus fused_sdpa_forward with mask=None and a general mask.

Tolerances, per test below: float32 within 1e-5 of the oracle (1e-6 for the single
ops; the GEMMs sum in another order); float16 within a few float16 ulps at the scale
of the result (2⁻¹⁰·max(1, max|ref|) per ulp): the oracle rounds every intermediate to
float16 as NumPy does, the kernels keep float32 sums and round once.
"""
import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle.weights import GPTConfig, make_weights, rope_weights

pytestmark = pytest.mark.gpu

CFG = GPTConfig(vocab_size=512, d_model=128, num_heads=4, num_layers=3, max_seq_len=96)
DTYPES = [np.float32, np.float16]


def bound(dt, ref, fp32, ulps):
    """fp32: an absolute bound; fp16: `ulps` float16 ulps at the scale of ref."""
    if np.dtype(dt) != np.float16:
        return fp32
    return ulps * 2.0 ** -10 * max(1.0, float(np.abs(ref.astype(np.float64)).max()))


@pytest.fixture
def dtype_ctx(request, gpu):
    import nimbleml_amd as nm

    old = nm.np_backend.dtype
    nm.set_dtype(np.dtype(request.param).name)
    yield np.dtype(request.param)
    nm.set_dtype(np.dtype(old).name)


def gpt_with(w, dt, *, use_rope=False, fused_trunk=False):
    import nimbleml_amd as nm

    m = nm.GPT(CFG.vocab_size, CFG.d_model, CFG.num_heads, CFG.num_layers, CFG.max_seq_len,
               fused_trunk=fused_trunk, use_rope=use_rope)
    nm.load_arrays(m, w)
    return m


def weights(dt, seed=11, rope=False):
    if rope:  # no position table; W_q, W_k scaled up in float32 before the cast
        w = rope_weights(make_weights(CFG, seed=seed, dtype=np.float32, rich=True))
        return {k: v.astype(dt) for k, v in w.items()}
    return make_weights(CFG, seed=seed, dtype=dt, rich=True)


def xin(dt, b=2, s=40, seed=5):
    return (np.random.default_rng(seed).standard_normal((b, s, CFG.d_model)) * 0.7).astype(dt)


def dev(x):
    import nimbleml_amd as nm

    return nm.Tensor(x, x.shape)


def worst(out, ref):
    got = np.asarray(out.data).reshape(out.shape).astype(np.float64)
    assert got.shape == ref.shape
    assert np.all(np.isfinite(got))
    return float(np.abs(got - ref.astype(np.float64)).max())


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_dense_forward(dtype_ctx):
    from nimbleml_amd._native import DeviceArray

    dt = dtype_ctx
    m = gpt_with(weights(dt), dt)
    dense = m._block_list[0].ffn.dense1
    x = xin(dt)
    out = dense(dev(x))
    assert isinstance(out.data, DeviceArray) and out.shape == (2, 40, 4 * CFG.d_model)
    w = np.asarray(dense.weights.data, dt).reshape(dense.weights.shape)
    b = np.asarray(dense.biases.data, dt)
    ref = R._mm(x.reshape(-1, CFG.d_model), w).reshape(2, 40, -1) + b
    err = worst(out, ref)
    print(f"dense {dt.name}: max |d| {err:.3g}")
    assert err <= bound(dt, ref, 1e-6, 1)


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_embedding_forward_and_prefix(dtype_ctx):
    dt = dtype_ctx
    w = weights(dt)
    m = gpt_with(w, dt)
    ids = np.random.default_rng(3).integers(0, CFG.vocab_size, (3, 17))
    out = m.token_emb(ids)
    assert out.shape == (3, 17, CFG.d_model)
    assert np.array_equal(np.asarray(out.data).reshape(out.shape), w["token_emb.weights"][ids])
    flat = m.token_emb(ids.reshape(-1))  # any id shape
    assert np.array_equal(np.asarray(flat.data).reshape(flat.shape),
                          w["token_emb.weights"][ids.reshape(-1)])
    pre = m.pos_emb.forward_prefix(33)
    assert pre.shape == (33, CFG.d_model)
    assert np.array_equal(np.asarray(pre.data).reshape(pre.shape), w["pos_emb.weights"][:33])
    with pytest.raises(ValueError):
        m.token_emb(np.array([[0, CFG.vocab_size]]))
    with pytest.raises(ValueError):
        m.pos_emb.forward_prefix(CFG.max_seq_len + 1)


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_rmsnorm_forward(dtype_ctx):
    dt = dtype_ctx
    w = weights(dt)
    m = gpt_with(w, dt)
    x = xin(dt, seed=8) * dt.type(3)
    out = m.ln(dev(x))
    ref = R.rmsnorm(x, w["ln.gamma"])
    err = worst(out, ref)
    print(f"rmsnorm {dt.name}: max |d| {err:.3g}")
    assert err <= bound(dt, ref, 2e-6, 1)


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_feed_forward(dtype_ctx):
    dt = dtype_ctx
    w = weights(dt)
    m = gpt_with(w, dt)
    x = xin(dt, seed=9)
    out = m._block_list[1].ffn(dev(x))
    ref = R.ffn(x, w, "blocks.layers.1.ffn.")
    err = worst(out, ref)
    print(f"ffn {dt.name}: max |d| {err:.3g}")
    assert err <= bound(dt, ref, 1e-6, 2)


def _mixed_mask(s, dt, seed=4):
    """An additive mask that is neither causal nor empty: finite offsets, −inf at random
    places, every row keeping its diagonal."""
    rng = np.random.default_rng(seed)
    m = (rng.standard_normal((s, s)) * 0.5).astype(dt)
    m[rng.random((s, s)) < 0.3] = -np.inf
    np.fill_diagonal(m, 0)
    return m


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
@pytest.mark.parametrize("mask_kind", ["none", "causal", "mixed"])
def test_multi_head_attention(dtype_ctx, mask_kind):
    import nimbleml_amd as nm

    dt = dtype_ctx
    w = weights(dt)
    m = gpt_with(w, dt)
    s = 37
    x = xin(dt, s=s, seed=10)
    mask = {"none": None, "causal": R.causal_mask(s, dt), "mixed": _mixed_mask(s, dt)}[mask_kind]
    arg = None if mask is None else nm.Tensor(mask, mask.shape)
    out = m._block_list[2].mha(dev(x), arg)
    ref = R.mha(x, w, "blocks.layers.2.mha.", CFG.num_heads, mask)
    err = worst(out, ref)
    print(f"mha {mask_kind} {dt.name}: max |d| {err:.3g}")
    assert err <= bound(dt, ref, 1e-6, 2)


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
@pytest.mark.parametrize("rope", [False, True])
def test_fused_transformer_block(dtype_ctx, rope):
    dt = dtype_ctx
    w = weights(dt, rope=rope)
    m = gpt_with(w, dt, use_rope=rope)
    x = xin(dt, seed=12)
    rc = R.rope_cache(CFG.max_seq_len, CFG.d_model // CFG.num_heads) if rope else None
    for i, blk in enumerate(m._block_list):
        out = blk(dev(x))  # mask=None → causal
        ref = R.block(x, w, i, CFG.num_heads, R.causal_mask(40, dt), rc)
        err = worst(out, ref)
        print(f"block {i} rope={rope} {dt.name}: max |d| {err:.3g}")
        assert err <= bound(dt, ref, 1e-5, 4)


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_fused_gpt_trunk_and_sequential(dtype_ctx):
    dt = dtype_ctx
    w = weights(dt)
    x = xin(dt, seed=13)
    mask = R.causal_mask(40, dt)
    ref = x
    for i in range(CFG.num_layers):
        ref = R.block(ref, w, i, CFG.num_heads, mask)
    # fused_trunk=True names the blocks blocks.blocks.i; the final norm is both ln and
    # blocks.ln
    wt = {k.replace("blocks.layers.", "blocks.blocks."): v for k, v in w.items()}
    wt["blocks.ln.gamma"] = w["ln.gamma"]
    trunk = gpt_with(wt, dt, fused_trunk=True).blocks
    out = trunk(dev(x))
    fin = R.rmsnorm(ref, w["ln.gamma"])
    err = worst(out, fin)
    print(f"trunk {dt.name}: max |d| {err:.3g}")
    assert err <= bound(dt, fin, 1e-5, 8)
    seq = gpt_with(w, dt).blocks  # Sequential of FusedTransformerBlocks
    out = seq(dev(x))
    err = worst(out, ref)
    print(f"sequential {dt.name}: max |d| {err:.3g}")
    assert err <= bound(dt, ref, 1e-5, 8)


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_block_with_explicit_masks(dtype_ctx):
    import nimbleml_amd as nm

    dt = dtype_ctx
    w = weights(dt)
    blk = gpt_with(w, dt)._block_list[0]
    x = xin(dt, s=29, seed=14)
    causal = R.causal_mask(29, dt)
    a = blk(dev(x), nm.Tensor(causal, causal.shape))
    b = blk(dev(x))
    assert np.array_equal(np.asarray(a.data), np.asarray(b.data))
    mixed = _mixed_mask(29, dt, seed=6)
    out = blk(dev(x), mixed)
    ref = R.block(x, w, 0, CFG.num_heads, mixed)
    err = worst(out, ref)
    print(f"block mixed mask {dt.name}: max |d| {err:.3g}")
    assert err <= bound(dt, ref, 1e-5, 4)
    with pytest.raises(ValueError):
        blk(dev(x), np.zeros((28, 28), dt))


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_sdpa_without_and_with_general_mask(dtype_ctx):
    from nimbleml_amd import kernels as K

    dt = dtype_ctx
    rng = np.random.default_rng(15)
    for dk, s in ((16, 50), (64, 70), (128, 33)):
        q, k, v = (rng.standard_normal((3, s, dk)).astype(dt) for _ in range(3))
        scale = float(dk) ** 0.5
        for mask in (None, _mixed_mask(s, dt, seed=dk)):
            out, _ = K.fused_sdpa_forward(q, k, v, scale, mask)
            ref = R.sdpa(q, k, v, scale, mask)
            err = float(np.abs(np.asarray(out).astype(np.float64) - ref).max())
            print(f"sdpa dk={dk} s={s} mask={mask is not None} {dt.name}: {err:.3g}")
            assert err <= bound(dt, ref, 1e-6, 2)


@pytest.mark.parametrize("dtype_ctx", DTYPES, indirect=True)
def test_module_forwards_keep_parameters_resident(dtype_ctx):
    """Each module keeps a device copy of its parameters: a second call with unchanged
    parameters (input already on the device) copies nothing host-to-device and gives the
    same result; load_arrays, and mark_parameters_changed after an in-place edit, make
    the next call upload again, and its result follows the new values."""
    import nimbleml_amd as nm
    from nimbleml_amd import _native as N

    dt = dtype_ctx
    w = weights(dt)
    m = gpt_with(w, dt)
    blk = m._block_list[0]
    xh = xin(dt, seed=16)
    x = nm.Tensor(N.DeviceArray.from_host(xh), xh.shape)
    calls = [lambda: blk(x), lambda: m.blocks(x), lambda: blk.mha(x), lambda: blk.ffn(x),
             lambda: blk.ln1(x), lambda: blk.mha.W_q(x)]
    for call in calls:
        first = np.asarray(call().data)
        before = dict(N.h2d_stats)
        again = np.asarray(call().data)
        assert N.h2d_stats == before, (before, N.h2d_stats)
        assert np.array_equal(first, again)
    ids = np.arange(30, dtype=np.int64).reshape(2, 15)
    m.token_emb(ids)
    before = dict(N.h2d_stats)
    m.token_emb(ids)
    assert N.h2d_stats["bytes"] - before["bytes"] == ids.nbytes  # the ids only
    # new values through load_arrays: uploaded again, and the result is the new block's
    w2 = weights(dt, seed=12)
    before = dict(N.h2d_stats)
    nm.load_arrays(m, w2)
    out = blk(x)
    assert N.h2d_stats["calls"] > before["calls"]
    ref = R.block(xh, w2, 0, CFG.num_heads, R.causal_mask(40, dt))
    assert worst(out, ref) <= bound(dt, ref, 1e-5, 4)
    # an in-place edit declared with mark_parameters_changed
    blk.ln1.gamma.data[...] = (np.asarray(blk.ln1.gamma.data) * 2).astype(dt)
    blk.mark_parameters_changed()
    w3 = dict(w2)
    w3["blocks.layers.0.ln1.gamma"] = (w2["blocks.layers.0.ln1.gamma"] * 2).astype(dt)
    out = blk(x)
    ref = R.block(xh, w3, 0, CFG.num_heads, R.causal_mask(40, dt))
    assert worst(out, ref) <= bound(dt, ref, 1e-5, 4)
