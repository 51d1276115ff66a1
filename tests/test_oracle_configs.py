"""Pins of the oracle pieces behind the benchmark-sized fixtures and the native single
ops (CPU only).

* oracle/halfmm.c against NumPy's own float16 matmul: bit-exact on every operand form
  the oracle uses (2-D, batched, transposed views, a folded batch), and the whole fp16
  forward with and without it identical — so the benchmark-sized fixtures
  (tests/golden/make_configs.py) carry the reference's own float16 arithmetic;
* RaggedKVOracle: each row of a lockstep ragged decode equals that row decoded alone;
* sample_flip_tol: no perturbation of the logits within the returned tolerance changes
  the pick (random and adversarial trials), and a planted slip (a tolerance 5x too
  large) is caught by the same trials;
* grad_ref.flash_forward / flash_backward / rmsnorm_backward (the native extension's
  device ops): the forward against the CPU path's softmax attention and the closed forms
  of m and l, the backwards against central finite differences (a planted slip — the
  D term dropped — fails the same check).
"""
import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle import grad_ref as G
from oracle import halfmm
from oracle.weights import GPTConfig, SMALL, TINY, make_weights, random_ids


def test_halfmm_bit_exact_against_numpy():
    rng = np.random.default_rng(0)
    for m, k, n in [(1, 64, 3), (7, 33, 19), (64, 256, 100), (130, 96, 77), (6, 1, 16)]:
        a = rng.standard_normal((m, k)).astype(np.float16)
        b = (rng.standard_normal((k, n)) * 0.05).astype(np.float16)
        assert np.array_equal(halfmm.matmul16(a, b), a @ b)
    q = rng.standard_normal((3, 40, 32)).astype(np.float16)
    kk = rng.standard_normal((3, 40, 32)).astype(np.float16)
    assert np.array_equal(halfmm.matmul16(q, np.swapaxes(kk, -2, -1)),
                          np.matmul(q, np.swapaxes(kk, -2, -1)))
    e = (rng.standard_normal((300, 64)) * 0.02).astype(np.float16)
    h = rng.standard_normal((9, 64)).astype(np.float16)
    assert np.array_equal(halfmm.matmul16(h, np.swapaxes(e, -2, -1)), h @ e.T)
    x = rng.standard_normal((2, 5, 64)).astype(np.float16)
    w = rng.standard_normal((64, 40)).astype(np.float16)
    assert np.array_equal(halfmm.matmul16(x, w), x @ w)
    big = np.full((4, 1000), 60.0, np.float16)  # sums overflow float16: inf like NumPy
    assert np.array_equal(halfmm.matmul16(big, big.T.copy()), big @ big.T)


def test_halfmm_is_in_use():
    assert halfmm.available(), "oracle/halfmm.c did not build (gcc with AVX2/FMA/F16C)"


@pytest.mark.parametrize("cfg", [TINY, GPTConfig(512, 128, 4, 2, 64)])
def test_fp16_forward_same_with_numpy_matmul(cfg, monkeypatch):
    w = make_weights(cfg, seed=2, dtype=np.float16, rich=True)
    ids = random_ids((2, 24), cfg.vocab_size, seed=3)
    fast = R.forward(w, ids, cfg.num_heads, cfg.num_layers)
    monkeypatch.setattr(halfmm, "matmul16", lambda a, b: np.matmul(a, b))
    slow = R.forward(w, ids, cfg.num_heads, cfg.num_layers)
    assert fast.dtype == np.float16 and np.array_equal(fast, slow)


@pytest.mark.parametrize("cfg,dt", [(TINY, np.float16), (GPTConfig(1024, 128, 4, 3, 64), np.float16)])
def test_ragged_oracle_rows_equal_single_rows(cfg, dt):
    w = make_weights(cfg, seed=3, dtype=dt, rich=True)
    rng = np.random.default_rng(0)
    rows = [rng.integers(0, cfg.vocab_size, n) for n in (5, 9, 3)]
    orc = R.RaggedKVOracle(w, cfg.num_heads, cfg.num_layers)
    lg = orc.prefill(rows)
    singles = [R.KVOracle(w, cfg.num_heads, cfg.num_layers) for _ in rows]
    ref = [s.step(r[None])[0, -1] for s, r in zip(singles, rows)]
    for t in range(5):
        for b in range(3):
            assert np.array_equal(lg[b], ref[b]), (t, b)
        tok = np.argmax(lg, axis=-1)
        lg = orc.step(tok)
        ref = [s.step(np.array([[tk]]))[0, -1] for s, tk in zip(singles, tok)]


def _flip_trials(scale_tol):
    """Perturbations of size tol: random ones, the two that push the CDF hardest (every
    logit before the pick up and the rest down, or the reverse), the pick itself down
    and the rest up (it may drop out of the top-k), and the kept set down and the rest
    up (the top-k set changes)."""
    rng = np.random.default_rng(7)
    bad = 0
    for case in range(60):
        x = (rng.standard_normal(400) * 0.6).astype(np.float32)
        u = float(rng.random())
        tok = R.sample_logits(x, temperature=0.8, top_k=50, top_p=1.0, u=u)
        tol = scale_tol * R.sample_flip_tol(x, u, tok, temperature=0.8, top_k=50)
        if tol <= 0:
            continue
        before = np.arange(x.size) < tok
        trials = [rng.uniform(-tol, tol, x.size) for _ in range(20)]
        kept = x >= np.partition(x, -50)[-50]
        trials += [np.where(before, tol, -tol), np.where(before, -tol, tol),
                   np.where(np.arange(x.size) == tok, -tol, tol), np.where(kept, -tol, tol),
                   np.where(kept & before, -tol, np.where(kept, tol, 0.0))]
        for d in trials:
            y = x + d.astype(np.float32)
            if R.sample_logits(y, temperature=0.8, top_k=50, top_p=1.0, u=u) != tok:
                bad += 1
    return bad


def test_sample_flip_tol_is_safe():
    assert _flip_trials(1.0) == 0
    # a planted slip (a tolerance 5x too large) is caught by the same trials
    assert _flip_trials(5.0) > 0
    x = np.asarray([0.0, 1.0, 0.25], np.float32)
    assert R.sample_flip_tol(x, 0.0, 1, temperature=0.0, top_k=0) == 0.375


def test_flash_forward_matches_cpu_attention_and_closed_forms():
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((3, 17, 16)) for _ in range(3))
    scale = 1.0 / np.sqrt(16.0)
    out, m, lsum = G.flash_forward(q, k, v, scale)
    mask = R.causal_mask(17, np.float64)
    want = R.sdpa(q, k, v, np.sqrt(16.0), mask)
    assert np.abs(out - want).max() < 1e-12
    for b in range(3):
        for i in range(17):
            s = [float(q[b, i] @ k[b, j]) * scale for j in range(i + 1)]
            assert abs(m[b, i] - max(s)) < 1e-12
            assert abs(lsum[b, i] - sum(np.exp(np.asarray(s) - max(s)))) < 1e-12


def _fd_check(fn_grads, f, args, idx, eps=1e-6):
    """Central differences of the scalar f(*args) against fn_grads at a few entries."""
    rng = np.random.default_rng(3)
    grads = fn_grads(*args)
    worst = 0.0
    for a_i, g in zip(idx, grads):
        for _ in range(6):
            pos = tuple(rng.integers(0, s) for s in args[a_i].shape)
            up = [a.copy() for a in args]
            dn = [a.copy() for a in args]
            up[a_i][pos] += eps
            dn[a_i][pos] -= eps
            num = (f(*up) - f(*dn)) / (2 * eps)
            worst = max(worst, abs(num - g[pos]) / max(1.0, abs(num)))
    return worst


def test_flash_backward_matches_finite_differences():
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((2, 9, 8)) for _ in range(3))
    go = rng.standard_normal((2, 9, 8))
    scale = 1.0 / np.sqrt(8.0)

    def f(q_, k_, v_):
        return float((G.flash_forward(q_, k_, v_, scale)[0] * go).sum())

    def grads(q_, k_, v_):
        return G.flash_backward(go, q_, k_, v_, scale)

    assert _fd_check(grads, f, (q, k, v), (0, 1, 2)) < 1e-6

    def slip(q_, k_, v_):  # the D term dropped
        out, m, lsum = G.flash_forward(q_, k_, v_, scale)
        s = np.matmul(q_, np.swapaxes(k_, -2, -1)) * scale
        s = np.where(np.tril(np.ones((9, 9), dtype=bool)), s, -np.inf)
        p = np.exp(s - m[..., None]) / lsum[..., None]
        ds = p * np.matmul(go, np.swapaxes(v_, -2, -1))
        return np.matmul(ds, k_) * scale, np.matmul(np.swapaxes(ds, -2, -1), q_) * scale, v_

    assert _fd_check(slip, f, (q, k, v), (0,)) > 1e-3


def test_rmsnorm_backward_matches_finite_differences():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 12))
    gam = 1.0 + 0.1 * rng.standard_normal(12)
    go = rng.standard_normal((5, 12))

    def f(x_, g_):
        return float((G._rms_fwd(x_, g_)[0] * go).sum())

    def grads(x_, g_):
        return G.rmsnorm_backward(go, x_, g_)

    assert _fd_check(grads, f, (x, gam), (0, 1)) < 1e-6
