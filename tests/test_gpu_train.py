"""Training on the device: ``compute_loss`` then ``loss.backward()``, float32 and float16 models,
every parameter's gradient against the float64 backward oracle (``oracle/grad_ref.py``,
pinned by finite differences in test_grad_oracle.py).

Tolerance: for each parameter tensor, max |device − oracle| ≤ 2e-5 · max |oracle| + 1e-7
(float32 products and sums in another order; the mistakes this test is for — a wrong
index, transposed operand or dropped term — move a gradient by O(1) of its size).
Head dims 8, 16, 32, 64 and 128 cover every attention-backward tile shape, and 40, 96
and 256 the scalar kernels on padded tiles; sequence lengths that are not tile multiples
cover the partial tiles."""
import ctypes as C

import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle import grad_ref as G
from oracle.weights import GPTConfig, make_weights, random_ids

pytestmark = pytest.mark.gpu

RTOL = 2e-5


def _model(cfg, seed, rope=False, scale=4.0):
    import nimbleml_amd as nm

    w = make_weights(cfg, seed=seed, dtype=np.float32, rich=True)
    for k in w:  # larger weights: attention and GELU away from their linear regimes
        if k.endswith(".weights") and "emb" not in k:
            w[k] = (w[k] * np.float32(scale)).astype(np.float32)
    if rope:
        w.pop("pos_emb.weights")
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float32, use_rope=rope)
    return m, w


def _named_grads(m):
    """The model's parameter grads under the reference names."""
    out = {"token_emb.weights": m.token_emb.weights, "ln.gamma": m.ln.gamma}
    if m.pos_emb is not None:
        out["pos_emb.weights"] = m.pos_emb.weights
    for i, blk in enumerate(m._block_list):
        p = f"blocks.layers.{i}."
        out[p + "ln1.gamma"] = blk.ln1.gamma
        out[p + "ln2.gamma"] = blk.ln2.gamma
        for n in ("W_q", "W_k", "W_v", "W_o"):
            d = getattr(blk.mha, n)
            out[p + f"mha.{n}.weights"] = d.weights
            out[p + f"mha.{n}.biases"] = d.biases
        for n in ("dense1", "dense2"):
            d = getattr(blk.ffn, n)
            out[p + f"ffn.{n}.weights"] = d.weights
            out[p + f"ffn.{n}.biases"] = d.biases
    return {k: (None if t.grad is None else np.asarray(t.grad).reshape(t.shape))
            for k, t in out.items()}


def _compare(got, want, factor=1.0):
    worst = 0.0
    for k, ref in want.items():
        assert k in got and got[k] is not None, k
        g = got[k].astype(np.float64)
        ref = factor * ref
        err = np.abs(g - ref).max()
        bound = RTOL * np.abs(ref).max() + 1e-7
        assert err <= bound, (k, err, bound)
        if not k.endswith("W_k.biases"):  # identically 0: softmax ignores a per-row shift
            worst = max(worst, err / np.abs(ref).max())
    return worst


def _oracle(w, cfg, ids, labels, ignore=None, rope=None, grad_scale=1.0):
    w64 = {k: v.astype(np.float64) for k, v in w.items()}
    if rope is not None:
        rope = (rope[0].astype(np.float64), rope[1].astype(np.float64))
    return G.loss_and_grads(w64, ids, labels, cfg.num_heads, cfg.num_layers, ignore_index=ignore,
                            rope=rope, grad_scale=grad_scale)


CASES = [
    # (vocab, d, heads, layers, max_seq), batch, seq
    ((48, 32, 4, 2, 16), 2, 7),        # dk 8, one partial tile
    ((256, 64, 4, 2, 64), 3, 37),      # dk 16, two tiles, ragged end
    ((512, 128, 4, 2, 96), 2, 96),     # dk 32, three full tiles
    ((512, 128, 2, 2, 128), 2, 70),    # dk 64
    ((1024, 256, 2, 1, 64), 2, 45),    # dk 128 (16-row tiles)
    ((256, 128, 2, 1, 512), 2, 512),   # 1024 rows: weight gradients split over K
    ((256, 80, 2, 1, 64), 2, 50),      # dk 40: tiles padded to 64 columns
    ((256, 192, 2, 1, 64), 2, 45),     # dk 96: padded to 128
    ((256, 512, 2, 1, 48), 2, 20),     # dk 256 (16-row tiles in dynamic LDS)
]


@pytest.mark.parametrize("dims,b,s", CASES)
def test_backward_matches_oracle(gpu, dims, b, s):
    cfg = GPTConfig(*dims)
    m, w = _model(cfg, seed=21)
    ids = random_ids((b, s), cfg.vocab_size, seed=5)
    labels = random_ids((b * s,), cfg.vocab_size, seed=6)
    loss = m.compute_loss(ids, labels)
    assert loss.requires_grad
    want_loss, want = _oracle(w, cfg, ids, labels)
    assert abs(loss.item() - want_loss) <= 1e-5 * abs(want_loss)
    loss.backward()
    got = _named_grads(m)
    print("worst relative gradient error", _compare(got, want))
    # q·(k + b) shifts every score of a row by q·b: the key bias gets no gradient
    for i in range(cfg.num_layers):
        p = f"blocks.layers.{i}.mha."
        assert np.abs(got[p + "W_k.biases"]).max() <= 1e-5 * np.abs(got[p + "W_q.biases"]).max()


def test_ignore_index_grad_scale_and_accumulation(gpu):
    cfg = GPTConfig(256, 64, 4, 2, 64)
    m, w = _model(cfg, seed=22)
    ids = random_ids((2, 33), cfg.vocab_size, seed=7)
    labels = random_ids((66,), cfg.vocab_size, seed=8)
    labels[::3] = -1
    loss = m.compute_loss(ids, labels, ignore_index=-1)
    want_loss, want = _oracle(w, cfg, ids, labels, ignore=-1)
    assert abs(loss.item() - want_loss) <= 1e-5 * abs(want_loss)
    loss.backward(np.array([0.5], np.float32))
    _compare(_named_grads(m), want, factor=0.5)
    # grads accumulate over backward calls (Tensor._accumulate_grad) ...
    loss2 = m.compute_loss(ids, labels, ignore_index=-1)
    loss2.backward()
    _compare(_named_grads(m), want, factor=1.5)
    # ... until zero_grad
    for p in m.parameters():
        p.zero_grad()
    m.compute_loss(ids, labels, ignore_index=-1).backward()
    _compare(_named_grads(m), want)


def test_all_labels_ignored_gives_zero_loss_and_grads(gpu):
    cfg = GPTConfig(48, 32, 4, 2, 16)
    m, _ = _model(cfg, seed=23)
    ids = random_ids((2, 5), cfg.vocab_size, seed=9)
    loss = m.compute_loss(ids, np.full(10, -7), ignore_index=-7)
    assert loss.item() == 0.0
    loss.backward()
    assert all(not np.any(g) for g in _named_grads(m).values())


@pytest.mark.parametrize("dims,b,s", [((256, 64, 4, 2, 64), 2, 40), ((512, 128, 2, 1, 96), 2, 80)])
def test_backward_with_rope(gpu, dims, b, s):
    cfg = GPTConfig(*dims)
    m, w = _model(cfg, seed=24, rope=True)
    ids = random_ids((b, s), cfg.vocab_size, seed=10)
    labels = random_ids((b * s,), cfg.vocab_size, seed=11)
    loss = m.compute_loss(ids, labels)
    rope = R.rope_cache(cfg.max_seq_len, cfg.d_model // cfg.num_heads)
    want_loss, want = _oracle(w, cfg, ids, labels, rope=rope)
    assert abs(loss.item() - want_loss) <= 1e-5 * abs(want_loss)
    loss.backward()
    got = _named_grads(m)
    assert "pos_emb.weights" not in got
    _compare(got, want)


def test_c_abi_backward_accumulates_and_matches_loss(gpu):
    """Through the C-ABI directly: loss_train equals compute_loss's plain loss, two
    nml_model_backward calls double every gradient, zero_grad clears them."""
    from nimbleml_amd import _native as N

    cfg = GPTConfig(256, 64, 4, 2, 64)
    m, w = _model(cfg, seed=25)
    ids = random_ids((2, 30), cfg.vocab_size, seed=12)
    labels = random_ids((60,), cfg.vocab_size, seed=13)
    h = m._device_model()
    dids = N.DeviceArray.from_host(ids)
    dlab = N.DeviceArray.from_host(labels)
    plain, trained = C.c_double(), C.c_double()
    N.check(N.lib.nml_model_loss(h, dids.ptr, dlab.ptr, 2, 30, 0, 0, C.byref(plain)))
    N.check(N.lib.nml_model_zero_grad(h))
    N.check(N.lib.nml_model_loss_train(h, dids.ptr, dlab.ptr, 2, 30, 0, 0, C.byref(trained)))
    assert abs(plain.value - trained.value) <= 1e-6 * abs(plain.value)
    N.check(N.lib.nml_model_backward(h, 1.0))
    one = m._grad_array(N.P_W1, 1, (cfg.d_ff, cfg.d_model))
    N.check(N.lib.nml_model_backward(h, 1.0))
    two = m._grad_array(N.P_W1, 1, (cfg.d_ff, cfg.d_model))
    assert np.abs(two - 2 * one).max() <= 1e-6 * np.abs(one).max()
    _, want = _oracle(w, cfg, ids, labels)
    ref = want["blocks.layers.1.ffn.dense1.weights"].T
    assert np.abs(one - ref).max() <= RTOL * np.abs(ref).max()
    N.check(N.lib.nml_model_zero_grad(h))
    assert not np.any(m._grad_array(N.P_W1, 1, (cfg.d_ff, cfg.d_model)))
    with pytest.raises(RuntimeError):
        N.check(N.lib.nml_model_grad_ptr(h, N.P_ROPE_COS, 0, C.byref(C.c_void_p())))


@pytest.mark.parametrize("dims,b,s", [((256, 64, 4, 2, 64), 2, 40), ((512, 128, 2, 2, 96), 2, 70),
                                      ((512, 256, 2, 1, 64), 2, 33), ((256, 128, 2, 1, 128), 2, 128),
                                      ((256, 192, 2, 1, 64), 2, 45), ((512, 256, 2, 1, 192), 2, 150)])
def test_backward_fp16(gpu, dims, b, s):
    """float16 models: the loss equals the fp16 oracle's (the reference's fp16 rounding),
    and the gradients (kept float32, as under an optimizer's _grad_dtype) match the float64
    gradient at the same fp16 weights within 1.5e-2 of each tensor's largest gradient
    (measured ≤ 9.3e-3): the fp16 rounding of the activations, activation gradients and the
    fp16 P and dS of the attention backward."""
    import nimbleml_amd as nm

    cfg = GPTConfig(*dims)
    w32 = make_weights(cfg, seed=30, dtype=np.float32, rich=True)
    for k in w32:
        if k.endswith(".weights") and "emb" not in k:
            w32[k] = (w32[k] * np.float32(4.0)).astype(np.float32)
    w16 = {k: v.astype(np.float16) for k, v in w32.items()}
    m = nm.GPT.from_arrays(w16, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float16)
    for p in m.parameters():
        p._grad_dtype = np.float32
    ids = random_ids((b, s), cfg.vocab_size, seed=22)
    labels = random_ids((b * s,), cfg.vocab_size, seed=23)
    loss = m.compute_loss(ids, labels)
    want16 = R.compute_loss(w16, ids, labels, cfg.num_heads, cfg.num_layers)
    # the loss Tensor is fp16, as the reference's (losses/cross_entropy.py:158-164)
    assert loss.data.dtype == np.float16
    assert abs(loss.item() - want16) <= 2 ** -10 * abs(want16)
    loss.backward()
    got = _named_grads(m)
    assert all(g.dtype == np.float32 for g in got.values())
    _, want = _oracle(w16, cfg, ids, labels)
    worst = 0.0
    for k, ref in want.items():
        err = np.abs(got[k].astype(np.float64) - ref).max()
        scale = np.abs(ref).max()
        if k.endswith("W_k.biases"):
            # exactly zero (a key bias moves every score of a query alike; softmax ignores
            # it): what the device returns is the fp16 rounding of dS summed over the keys,
            # bounded against the scale of the same layer's W_q bias gradient
            scale = np.abs(want[k.replace("W_k", "W_q")]).max()
        assert err <= 1.5e-2 * scale + 1e-5, (k, err, scale)
        if not k.endswith("W_k.biases"):
            worst = max(worst, err / scale)
    print("worst relative gradient error (fp16)", worst)


def test_backward_fp16_direct_to_lds_path_matches_register_path(gpu, monkeypatch):
    """The float16 backward GEMMs on the direct-to-LDS main loop (operands read across k
    transposed first; split K for the weight gradients, 2048 rows) against the
    register-staged kernel (NIMBLEML_TRAIN_F16_BIG=0) on the same model and batch: the two
    differ only in the fp32 summation order, so every gradient agrees within 2e-3 of the
    tensor's largest."""
    import nimbleml_amd as nm

    cfg = GPTConfig(512, 128, 2, 2, 512)
    w16 = {k: v.astype(np.float16) for k, v in make_weights(cfg, seed=32, rich=True).items()}
    ids = random_ids((4, 512), cfg.vocab_size, seed=26)
    labels = random_ids((4 * 512,), cfg.vocab_size, seed=27)
    grads = []
    for big in ("1", "0"):
        monkeypatch.setenv("NIMBLEML_TRAIN_F16_BIG", big)
        m = nm.GPT.from_arrays(w16, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, dtype=np.float16)
        for p in m.parameters():
            p._grad_dtype = np.float32
        m.compute_loss(ids, labels).backward()
        grads.append(_named_grads(m))
    for k, ref in grads[1].items():
        err = np.abs(grads[0][k].astype(np.float64) - ref).max()
        assert err <= 2e-3 * np.abs(ref).max() + 1e-6, (k, err, np.abs(ref).max())


@pytest.mark.parametrize("dt", ["fp32", "fp16"])
def test_backward_large_vocab(gpu, dt):
    """Vocabularies of 20000 (fp32) and 16384 (fp16): the cross-entropy backward holds each
    logits row in registers (16-byte chunks, 20 and 8 per thread). fp32: every gradient
    within RTOL of the float64 oracle; fp16: the token-embedding and W1 gradients within
    1.5e-2 of the largest, with grad_scale 1024 so that the fp16 logits gradient
    (≈ 1/(rows·V)) stays clear of fp16's subnormal range."""
    from nimbleml_amd import _native as N
    import nimbleml_amd as nm

    if dt == "fp32":
        cfg = GPTConfig(20000, 64, 2, 1, 32)
        m, w = _model(cfg, seed=33)
    else:
        cfg = GPTConfig(16384, 64, 2, 1, 32)
        w = {k: v.astype(np.float16) for k, v in make_weights(cfg, seed=33, rich=True).items()}
        m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, dtype=np.float16)
    ids = random_ids((2, 16), cfg.vocab_size, seed=28)
    labels = random_ids((32,), cfg.vocab_size, seed=29)
    if dt == "fp32":
        m.compute_loss(ids, labels).backward()
        _, want = _oracle(w, cfg, ids, labels)
        _compare(_named_grads(m), want)
        return
    h = m._device_model()
    dids = N.DeviceArray.from_host(ids)
    dlab = N.DeviceArray.from_host(labels)
    loss = C.c_double()
    N.check(N.lib.nml_model_zero_grad(h))
    N.check(N.lib.nml_model_loss_train(h, dids.ptr, dlab.ptr, 2, 16, 0, 0, C.byref(loss)))
    N.check(N.lib.nml_model_backward(h, 1024.0))
    _, want = _oracle(w, cfg, ids, labels, grad_scale=1024.0)
    got = {"token_emb.weights": m._grad_array(N.P_TOKEN_EMB, 0, (cfg.vocab_size, cfg.d_model)),
           "blocks.layers.0.ffn.dense1.weights": m._grad_array(N.P_W1, 0, (cfg.d_ff, cfg.d_model)).T}
    for k, g in got.items():
        ref = want[k]
        err = np.abs(g.astype(np.float64) - ref).max()
        assert err <= 1.5e-2 * np.abs(ref).max(), (k, err, np.abs(ref).max())


def test_model_adamw_step_fp16_masters(gpu):
    """fp16 models: AdamW runs on float32 masters taken from the parameters, and the
    parameters become the masters rounded to fp16 (optimizers/adam.py:75-81, :238-245), bit
    for bit with the reference's float32 adamw_step on the device's gradients."""
    from nimbleml_amd import _native as N
    import nimbleml_amd as nm
    from oracle.optim_ref import adamw_step

    cfg = GPTConfig(256, 64, 4, 1, 64)
    w16 = {k: v.astype(np.float16) for k, v in make_weights(cfg, seed=31, rich=True).items()}
    m = nm.GPT.from_arrays(w16, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float16)
    h = m._device_model()
    ids = N.DeviceArray.from_host(random_ids((2, 16), cfg.vocab_size, seed=24))
    lab = N.DeviceArray.from_host(random_ids((32,), cfg.vocab_size, seed=25))
    slots = _param_slots(cfg, False)

    def ptr(fn, kind, layer):
        p = C.c_void_p()
        N.check(fn(h, kind, layer, C.byref(p)))
        return p

    def dev16(p, shape):
        out = np.empty(shape, np.float16)
        N.check(N.lib.nml_memcpy_d2h(out.ctypes.data, p, out.nbytes))
        return out

    masters = {(k, l): dev16(ptr(N.lib.nml_model_param_ptr, k, l), s).astype(np.float32)
               for k, l, s in slots}
    mom = {key: (np.zeros_like(p), np.zeros_like(p)) for key, p in masters.items()}
    for t in (1, 2):
        loss = C.c_double()
        N.check(N.lib.nml_model_zero_grad(h))
        N.check(N.lib.nml_model_loss_train(h, ids.ptr, lab.ptr, 2, 16, 0, 0, C.byref(loss)))
        N.check(N.lib.nml_model_backward(h, 1.0))
        bc1, bc2 = 1.0 - 0.9 ** t, 1.0 - 0.999 ** t
        for k, l, s in slots:
            g = _dev(N, ptr(N.lib.nml_model_grad_ptr, k, l), s)
            adamw_step(masters[(k, l)], g, *mom[(k, l)], 1e-3, 0.9, 0.999, bc1, bc2, 1e-8, 0.01)
        N.check(N.lib.nml_model_adamw_step(h, 1e-3, 0.9, 0.999, bc1, bc2, 1e-8, 0.01))
        for k, l, s in slots:
            got = dev16(ptr(N.lib.nml_model_param_ptr, k, l), s)
            assert np.array_equal(got, masters[(k, l)].astype(np.float16)), (t, k, l)


def _dev(N, ptr, shape):
    out = np.empty(shape, np.float32)
    N.check(N.lib.nml_memcpy_d2h(out.ctypes.data, ptr, out.nbytes))
    return out


def _param_slots(cfg, rope):
    from nimbleml_amd import _native as N

    d, f = cfg.d_model, cfg.d_ff
    slots = [(N.P_TOKEN_EMB, 0, (cfg.vocab_size, d)), (N.P_LN_F, 0, (d,))]
    if not rope:
        slots.append((N.P_POS_EMB, 0, (cfg.max_seq_len, d)))
    for i in range(cfg.num_layers):
        slots += [(N.P_LN1, i, (d,)), (N.P_WQKV, i, (3 * d, d)), (N.P_BQKV, i, (3 * d,)),
                  (N.P_WO, i, (d, d)), (N.P_BO, i, (d,)), (N.P_LN2, i, (d,)),
                  (N.P_W1, i, (f, d)), (N.P_B1, i, (f,)), (N.P_W2, i, (d, f)), (N.P_B2, i, (d,))]
    return slots


@pytest.mark.parametrize("rope", [False, True])
def test_model_adamw_step_bit_exact(gpu, rope):
    """nml_model_adamw_step over the gradient arena equals the reference's float32
    adamw_step (oracle/optim_ref.py, pinned bit for bit to the compiled reference) applied
    to every parameter with the device's own gradients, over two steps; the rotary tables
    are not touched."""
    from nimbleml_amd import _native as N
    from oracle.optim_ref import adamw_step

    cfg = GPTConfig(256, 64, 4, 2, 64)
    m, _ = _model(cfg, seed=27, rope=rope)
    h = m._device_model()
    ids = N.DeviceArray.from_host(random_ids((2, 24), cfg.vocab_size, seed=16))
    lab = N.DeviceArray.from_host(random_ids((48,), cfg.vocab_size, seed=17))
    slots = _param_slots(cfg, rope)

    def ptr(fn, kind, layer):
        p = C.c_void_p()
        N.check(fn(h, kind, layer, C.byref(p)))
        return p

    if rope:
        cos0 = _dev(N, ptr(N.lib.nml_model_param_ptr, N.P_ROPE_COS, 0), (cfg.max_seq_len, 8))
    params = {(k, l): _dev(N, ptr(N.lib.nml_model_param_ptr, k, l), s) for k, l, s in slots}
    mom = {key: (np.zeros_like(p), np.zeros_like(p)) for key, p in params.items()}
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    for t in (1, 2):
        loss = C.c_double()
        N.check(N.lib.nml_model_zero_grad(h))
        N.check(N.lib.nml_model_loss_train(h, ids.ptr, lab.ptr, 2, 24, 0, 0, C.byref(loss)))
        N.check(N.lib.nml_model_backward(h, 1.0))
        bc1, bc2 = 1.0 - b1 ** t, 1.0 - b2 ** t
        for k, l, s in slots:
            g = _dev(N, ptr(N.lib.nml_model_grad_ptr, k, l), s)
            adamw_step(params[(k, l)], g, *mom[(k, l)], lr, b1, b2, bc1, bc2, eps, wd)
        N.check(N.lib.nml_model_adamw_step(h, lr, b1, b2, bc1, bc2, eps, wd))
        for k, l, s in slots:
            got = _dev(N, ptr(N.lib.nml_model_param_ptr, k, l), s)
            assert np.array_equal(got, params[(k, l)]), (t, k, l)
            m1, m2 = C.c_void_p(), C.c_void_p()
            N.check(N.lib.nml_model_adam_moments(h, k, l, C.byref(m1), C.byref(m2)))
            assert np.array_equal(_dev(N, m1, s), mom[(k, l)][0]), (t, k, l)
            assert np.array_equal(_dev(N, m2, s), mom[(k, l)][1]), (t, k, l)
    if rope:
        assert np.array_equal(_dev(N, ptr(N.lib.nml_model_param_ptr, N.P_ROPE_COS, 0),
                                   (cfg.max_seq_len, 8)), cos0)


def test_device_training_loop_lowers_the_loss(gpu):
    """compute_loss → backward → AdamW on the device for a few steps on one batch: the
    first loss equals the oracle's, and every step lowers the loss."""
    from nimbleml_amd import _native as N

    cfg = GPTConfig(256, 64, 4, 2, 64)
    m, w = _model(cfg, seed=28)
    h = m._device_model()
    ids_h = random_ids((2, 32), cfg.vocab_size, seed=18)
    lab_h = random_ids((64,), cfg.vocab_size, seed=19)
    ids, lab = N.DeviceArray.from_host(ids_h), N.DeviceArray.from_host(lab_h)
    losses = []
    for t in range(1, 7):
        loss = C.c_double()
        N.check(N.lib.nml_model_zero_grad(h))
        N.check(N.lib.nml_model_loss_train(h, ids.ptr, lab.ptr, 2, 32, 0, 0, C.byref(loss)))
        N.check(N.lib.nml_model_backward(h, 1.0))
        N.check(N.lib.nml_model_adamw_step(h, 3e-3, 0.9, 0.999, 1 - 0.9 ** t, 1 - 0.999 ** t,
                                           1e-8, 0.0))
        losses.append(loss.value)
    want0, _ = _oracle(w, cfg, ids_h, lab_h)
    assert abs(losses[0] - want0) <= 1e-5 * want0
    assert all(b < a for a, b in zip(losses, losses[1:])), losses


@pytest.mark.parametrize("flags", [{"fused_trunk": True}, {"gradient_checkpointing": True}])
def test_backward_with_trunk_flags(gpu, flags):
    """fused_trunk (the final RMSNorm inside the trunk module) and gradient_checkpointing
    (a memory/recompute trade in the reference, same gradients) give the oracle's gradients
    under the same parameter names."""
    import nimbleml_amd as nm

    cfg = GPTConfig(256, 64, 4, 2, 64)
    w = make_weights(cfg, seed=29, dtype=np.float32, rich=True)
    arrays = w
    if flags.get("fused_trunk"):  # FusedGPTTrunk's checkpoint names (blocks.blocks.i, blocks.ln)
        arrays = {k.replace("blocks.layers.", "blocks.blocks."): v for k, v in w.items()}
        arrays["blocks.ln.gamma"] = w["ln.gamma"]  # the same RMSNorm under both names
    m = nm.GPT.from_arrays(arrays, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float32, **flags)
    ids = random_ids((2, 20), cfg.vocab_size, seed=20)
    labels = random_ids((40,), cfg.vocab_size, seed=21)
    m.compute_loss(ids, labels).backward()
    _, want = _oracle(w, cfg, ids, labels)
    _compare(_named_grads(m), want)
    assert all(p.grad is not None for p in m.parameters())


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_no_grad_loss_equals_training_loss(gpu, dtype):
    """Under no_grad (utils/grad_mode.py) compute_loss keeps nothing and returns a loss
    without a graph; it is the same number as the loss of the training forward."""
    import nimbleml_amd as nm

    cfg = GPTConfig(256, 64, 4, 2, 64)
    w = {k: v.astype(dtype) for k, v in make_weights(cfg, seed=32, rich=True).items()}
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=dtype)
    ids = random_ids((2, 30), cfg.vocab_size, seed=26)
    labels = random_ids((60,), cfg.vocab_size, seed=27)
    with nm.no_grad():
        plain = m.compute_loss(ids, labels)
        with nm.enable_grad():
            assert nm.is_grad_enabled()
    assert not plain.requires_grad and nm.is_grad_enabled()
    trained = m.compute_loss(ids, labels)
    assert trained.requires_grad
    assert plain.item() == trained.item()


@pytest.mark.parametrize("dims", [(1024, 128, 2, 2, 512), (1024, 256, 2, 2, 512)],
                         ids=["dk64", "dk128"])
def test_fp16_no_grad_loss_stays_near_training_loss(gpu, dims):
    """float16 models at head dims 64/128: without grad the prefill attention keeps its
    scores as fp32 accumulators, while the training forward (whose backward recomputes the
    scores from the saved statistics) rounds them to fp16 as the reference's fp16 path
    does. The two losses (float64 from the C-ABI, before the fp16 Tensor rounding) must
    stay within 1e-5 relative (measured ~1e-6), and each within the fp16 loss rounding of
    the fp16 oracle."""
    import nimbleml_amd as nm
    from nimbleml_amd import _native as N

    cfg = GPTConfig(*dims)
    w = {k: v.astype(np.float16) for k, v in make_weights(cfg, seed=33, rich=True).items()}
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float16)
    b, s = 2, 400
    ids = random_ids((b, s), cfg.vocab_size, seed=28)
    labels = random_ids((b * s,), cfg.vocab_size, seed=29)
    h = m._device_model()
    dids, dlab = N.DeviceArray.from_host(ids), N.DeviceArray.from_host(labels)
    plain, trained = C.c_double(), C.c_double()
    N.check(N.lib.nml_model_loss(h, dids.ptr, dlab.ptr, b, s, 0, 0, C.byref(plain)))
    N.check(N.lib.nml_model_loss_train(h, dids.ptr, dlab.ptr, b, s, 0, 0, C.byref(trained)))
    gap = abs(plain.value - trained.value) / abs(trained.value)
    print(f"no_grad vs training loss: relative gap {gap:.2e}")
    assert gap <= 1e-5, gap
    want = R.compute_loss(w, ids, labels, cfg.num_heads, cfg.num_layers)
    for got in (plain.value, trained.value):
        assert abs(got - want) <= 2 ** -10 * abs(want), (got, want)


def test_interleaved_losses_and_inference_before_backward(gpu):
    """Two losses before one backward: the device keeps one saved forward, so the older
    loss refuses its backward (instead of returning the later batch's gradients); the
    latest one back-propagates correctly. Inference between a loss and its backward
    (forward, no_grad loss, generate) leaves the saved forward intact."""
    import nimbleml_amd as nm

    cfg = GPTConfig(256, 64, 4, 2, 64)
    m, w = _model(cfg, seed=31)
    ids_a = random_ids((2, 20), cfg.vocab_size, seed=1)
    ids_b = random_ids((2, 20), cfg.vocab_size, seed=2)
    lab_a = random_ids((40,), cfg.vocab_size, seed=3)
    lab_b = random_ids((40,), cfg.vocab_size, seed=4)
    loss_a = m.compute_loss(ids_a, lab_a)
    loss_b = m.compute_loss(ids_b, lab_b)
    with pytest.raises(RuntimeError, match="overwritten by a later compute_loss"):
        loss_a.backward()
    # inference in between does not disturb loss_b's saved forward
    m.forward(ids_a)
    with nm.no_grad():
        m.compute_loss(ids_a, lab_a)
    nm.generate(m, ids_a, max_new_tokens=3, temperature=0.0)
    for p in m.parameters():
        p.zero_grad()
    loss_b.backward()
    _, want = _oracle(w, cfg, ids_b, lab_b)
    _compare(_named_grads(m), want)


def test_token_embedding_gradient_is_deterministic_with_repeated_ids(gpu):
    """A 12-token vocabulary over 2 x 300 positions: every id repeats ~50 times, on both
    sides of the 256-row chunk boundaries of the scatter. The token-embedding gradient sums
    an id's rows in ascending row order, as the reference's scatter does, so two backward
    passes give the same bits, and both are within RTOL of the oracle."""
    cfg = GPTConfig(12, 64, 4, 1, 320)
    m, w = _model(cfg, seed=31)
    ids = random_ids((2, 300), cfg.vocab_size, seed=7)
    labels = random_ids((600,), cfg.vocab_size, seed=8)
    assert np.bincount(ids.ravel(), minlength=12).min() >= 20
    grads = []
    for _ in range(2):
        for p in m.parameters():
            p.zero_grad()
        m.compute_loss(ids, labels).backward()
        grads.append(_named_grads(m))
    _, want = _oracle(w, cfg, ids, labels)
    _compare(grads[0], want)
    assert np.array_equal(grads[0]["token_emb.weights"], grads[1]["token_emb.weights"])
