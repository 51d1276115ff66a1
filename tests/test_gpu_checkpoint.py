"""Weight interchange with a device-resident model, and the device Adam/AdamW.

* ``load`` of new weights into a model already on the device: its logits are the new
  weights' oracle logits (and bit-identical to a model built from them directly);
* ``nimbleml_amd.AdamW`` on the device equals the reference's float32 AdamW
  (oracle/optim_ref.adamw_step, pinned bit for bit to the compiled reference) applied to
  the host gradients, bit for bit: the whole-model launch, and per-parameter launches for
  parameter groups with their own lr / weight_decay, a parameter without a gradient
  (skipped, adam.py:97-104) and gradients accumulated over two backward calls;
* after device steps, ``save`` writes the trained weights (``sync_to_host``): loaded into
  a fresh model they give bit-identical logits; ``save_checkpoint`` / ``load_checkpoint``
  carry the step count, moments and float16 masters, and a resumed run continues bit for
  bit like the uninterrupted one (also across ``to_device``, which keeps the state).
"""
import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle.optim_ref import adamw_step
from oracle.weights import GPTConfig, make_weights, random_ids

pytestmark = pytest.mark.gpu

CFG = GPTConfig(256, 64, 4, 2, 64)


def build(dt, seed):
    import nimbleml_amd as nm

    old = nm.np_backend.dtype
    nm.set_dtype(np.dtype(dt).name)
    try:
        m = nm.GPT(CFG.vocab_size, CFG.d_model, CFG.num_heads, CFG.num_layers, CFG.max_seq_len)
    finally:
        nm.set_dtype(np.dtype(old).name)
    w = make_weights(CFG, seed=seed, dtype=dt, rich=True)
    nm.load_arrays(m, w)
    return m, w


def batch(seed):
    return (random_ids((2, 24), CFG.vocab_size, seed=seed),
            random_ids((48,), CFG.vocab_size, seed=seed + 1))


def logits(m, ids):
    return np.asarray(m.forward(ids).data).reshape(ids.shape[0], ids.shape[1], -1)


def host(m):
    from nimbleml_amd.saveload import named_parameters

    return {k: np.asarray(p.data).reshape(p.shape).copy() for k, p in named_parameters(m)}


@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_load_new_weights_into_resident_model(gpu, dt, tmp_path):
    import nimbleml_amd as nm

    m, w1 = build(dt, seed=31)
    ids, _ = batch(3)
    tol = 3e-2 if dt == np.float16 else 1e-3
    assert np.abs(logits(m, ids) - R.forward(w1, ids, CFG.num_heads, CFG.num_layers)).max() <= tol
    w2 = make_weights(CFG, seed=32, dtype=dt, rich=True)
    np.savez(tmp_path / "w2.npz", **w2)
    nm.load(m, str(tmp_path / "w2.npz"))  # the model is resident: this must re-upload
    got = logits(m, ids)
    ref = R.forward(w2, ids, CFG.num_heads, CFG.num_layers)
    print(f"{np.dtype(dt).name}: max |d| after load {np.abs(got - ref).max():.3g}")
    assert np.abs(got - ref).max() <= tol
    fresh, _ = build(dt, seed=32)
    assert np.array_equal(got, logits(fresh, ids))


def _oracle_state(m, opt):
    """Host copies of every parameter (reference layout, float32) and zero moments."""
    params = {id(p): np.asarray(p.data, np.float32).reshape(-1).copy() for p in opt.params}
    mom = {id(p): (np.zeros(p.size, np.float32), np.zeros(p.size, np.float32))
           for p in opt.params}
    return params, mom


def _check(m, opt, params, mom, skipped=()):
    m.sync_to_host()
    ms, vs = opt.m, opt.v
    for i, p in enumerate(opt.params):
        got = np.asarray(p.data).reshape(-1)
        assert np.array_equal(got, params[id(p)]), i
        assert np.array_equal(ms[i], mom[id(p)][0]), i
        assert np.array_equal(vs[i], mom[id(p)][1]), i
    for p in skipped:
        assert not np.any(mom[id(p)][0])


def test_adamw_whole_model_bit_exact(gpu):
    import nimbleml_amd as nm

    m, _ = build(np.float32, seed=33)
    opt = nm.AdamW(m.parameters(), learning_rate=2e-3, weight_decay=0.05)
    params, mom = _oracle_state(m, opt)
    for t in (1, 2, 3):
        ids, lab = batch(10 + t)
        opt.zero_grad(set_to_none=True)
        m.compute_loss(ids, lab).backward()
        bc1, bc2 = 1.0 - 0.9 ** t, 1.0 - 0.999 ** t
        for p in opt.params:
            adamw_step(params[id(p)], np.asarray(p.grad, np.float32), *mom[id(p)], 2e-3, 0.9,
                       0.999, bc1, bc2, 1e-8, 0.05)
        opt.step()
        assert opt.t == t
        _check(m, opt, params, mom)


def test_adamw_groups_missing_grads_and_accumulation(gpu):
    import nimbleml_amd as nm

    m, _ = build(np.float32, seed=34)
    all_p = m.parameters()
    decay = [p for p in all_p if len(p.shape) == 2 and p is not m.token_emb.weights]
    rest = [p for p in all_p if not any(p is q for q in decay)]
    opt = nm.AdamW([{"params": decay, "lr": 3e-3, "weight_decay": 0.1},
                    {"params": rest, "lr": 1e-3, "weight_decay": 0.0}], weight_decay=0.02)
    params, mom = _oracle_state(m, opt)
    frozen = m.pos_emb.weights
    hp = {id(p): (3e-3, 0.1) for p in decay}
    hp.update({id(p): (1e-3, 0.0) for p in rest})
    for t in (1, 2):
        opt.zero_grad(set_to_none=True)
        for mb in range(2):  # two micro-batches: host gradients accumulate
            ids, lab = batch(20 + 2 * t + mb)
            m.compute_loss(ids, lab).backward()
        frozen.grad = None  # no gradient: skipped, moments untouched
        bc1, bc2 = 1.0 - 0.9 ** t, 1.0 - 0.999 ** t
        for p in opt.params:
            if p.grad is None:
                continue
            lr, wd = hp[id(p)]
            adamw_step(params[id(p)], np.asarray(p.grad, np.float32), *mom[id(p)], lr, 0.9,
                       0.999, bc1, bc2, 1e-8, wd)
        opt.step()
        _check(m, opt, params, mom, skipped=(frozen,))


@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_save_after_device_steps_and_resume(gpu, dt, tmp_path):
    import nimbleml_amd as nm

    a, _ = build(dt, seed=35)
    opt_a = nm.AdamW(a.parameters(), learning_rate=1e-3)

    def step(m, opt, t):
        ids, lab = batch(40 + t)
        opt.zero_grad(set_to_none=True)
        loss = m.compute_loss(ids, lab)
        loss.backward()
        opt.step()
        return loss.item()

    for t in (1, 2):
        step(a, opt_a, t)
    before = host(a)
    nm.save(a, str(tmp_path / "w.npz"))
    after = host(a)
    assert any(not np.array_equal(before[k], after[k]) for k in before), "save did not sync"
    ids, _ = batch(7)
    b, _ = build(dt, seed=36)
    nm.load(b, str(tmp_path / "w.npz"))
    assert np.array_equal(logits(b, ids), logits(a, ids))

    nm.save_checkpoint(str(tmp_path / "ck.npz"), a, opt_a, step=2, extra={"tag": "x"})
    with pytest.raises(ValueError):
        nm.load(b, str(tmp_path / "ck.npz"))
    c, _ = build(dt, seed=37)
    opt_c = nm.AdamW(c.parameters(), learning_rate=1e-3)
    meta = nm.load_checkpoint(str(tmp_path / "ck.npz"), c, opt_c)
    assert meta == {"step": 2, "extra": {"tag": "x"}} and opt_c.t == 2
    for x, y in zip(opt_a.m + opt_a.v, opt_c.m + opt_c.v):
        assert np.array_equal(x, y)
    if dt == np.float16:
        for x, y in zip(opt_a.masters, opt_c.masters):
            assert x.dtype == np.float32 and np.array_equal(x, y)
    a.to_device()  # re-upload: the optimizer state carries over
    la, lc = step(a, opt_a, 3), step(c, opt_c, 3)
    assert la == lc
    a.sync_to_host()
    c.sync_to_host()
    assert all(np.array_equal(x, y) for x, y in zip(host(a).values(), host(c).values()))
