"""GPU parity of the persistent (one launch per token) batch-1 decode step.

The persistent kernel applies at d_model 1024 / head_dim 64 (the C3 / C4 widths). Its
tokens are checked against the reference's own fixture (c3slice, fp16) and against the
oracle on synthetic weights, greedy and sampled, fp16 and fp32, including contexts
long enough that each head's 16 workgroups loop over several 64-key chunks. Token
ids must be identical wherever the oracle's decision margin exceeds the stated logit
tolerance (fp32 1e-3, fp16 3e-2); the multi-kernel step on the same inputs is the
second reference.
"""
import numpy as np
import pytest

from conftest import fixture_weights, golden
from oracle import gpt_ref as R
from oracle.weights import GPTConfig, make_weights, random_ids

pytestmark = pytest.mark.gpu


def _build(cfg, w, dtype):
    import nimbleml_amd as nm

    return nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                              cfg.max_seq_len, dtype=dtype)


def _greedy_margins(w, cfg, tokens, s0):
    """Top-2 logit gap of the oracle (fp32, KV form) before each generated token."""
    w32 = {k: v.astype(np.float32) for k, v in w.items()}
    kv = R.KVOracle(w32, cfg.num_heads, cfg.num_layers)
    lg = kv.step(tokens[:, :s0])[:, -1]
    out = []
    for t in range(s0, tokens.shape[1]):
        top2 = np.sort(lg.astype(np.float64), axis=-1)[..., -2:]
        out.append(top2[..., 1] - top2[..., 0])
        if t + 1 < tokens.shape[1]:
            lg = kv.step(tokens[:, t:t + 1])[:, -1]
    return out


def _agree_until_tie(ours, ref, s0, margins, tol):
    n = 0
    for t in range(ref.shape[1] - s0):
        if margins[t][0] <= tol:
            break
        assert ours[0, s0 + t] == ref[0, s0 + t], f"step {t}"
        n += 1
    return n


def test_c3slice_fixture_through_persistent_path(gpu):
    """The reference's own d1024/V32000 fp16 tokens, decoded by the persistent kernel."""
    import nimbleml_amd as nm

    f = golden("c3slice_fp16")
    cfg, w = fixture_weights(f)
    m = _build(cfg, w, np.float16)
    s0 = f["prompt"].shape[1]
    n = f["greedy"].shape[1] - s0
    out = nm.generate(m, f["prompt"], max_new_tokens=n, temperature=0.0)
    assert m.last_decode_persistent()
    margins = [np.atleast_1d(np.diff(np.sort(f[f"logits_step{t}"].astype(np.float64), -1)[..., -2:],
                                     axis=-1)[..., 0]) for t in range(n)]
    # every one of the fixture's steps has a top-2 margin above the fp16 tolerance
    assert all(mg[0] > 3e-2 for mg in margins)
    assert _agree_until_tie(out, f["greedy"], s0, margins, 3e-2) == n


@pytest.mark.parametrize("dtype,prompt,new", [(np.float16, 40, 48), (np.float32, 40, 48),
                                               (np.float16, 1000, 40)])
def test_persistent_greedy_matches_oracle(gpu, monkeypatch, dtype, prompt, new):
    import nimbleml_amd as nm

    cfg = GPTConfig(4096, 1024, 16, 2, 2048)
    w = make_weights(cfg, seed=31, dtype=dtype, rich=True)
    m = _build(cfg, w, dtype)
    ids = random_ids((1, prompt), cfg.vocab_size, seed=7)
    out = nm.generate(m, ids, max_new_tokens=new, temperature=0.0)
    assert m.last_decode_persistent()
    monkeypatch.setenv("NIMBLEML_PERSISTENT", "0")
    ref_path = nm.generate(m, ids, max_new_tokens=new, temperature=0.0)
    assert not m.last_decode_persistent()
    tol = 3e-2 if dtype == np.float16 else 1e-3
    margins = _greedy_margins(w, cfg, out, prompt)
    # the oracle's own greedy choice at each step, on our token prefix
    w32 = {k: v.astype(np.float32) for k, v in w.items()}
    kv = R.KVOracle(w32, cfg.num_heads, cfg.num_layers)
    lg = kv.step(out[:, :prompt])[:, -1]
    compared = 0
    for t in range(new):
        if margins[t][0] <= tol:
            break
        assert out[0, prompt + t] == int(np.argmax(lg[0])), f"step {t}"
        assert ref_path[0, prompt + t] == out[0, prompt + t], f"step {t}"
        compared += 1
        lg = kv.step(out[:, prompt + t:prompt + t + 1])[:, -1]
    assert compared >= 8, compared


def test_persistent_logits_match_oracle_fp32(gpu):
    """Sampling mode leaves the step's logits in place: check them directly by driving
    one decode step at a time (max_new_tokens=2: prefill choice + one persistent step)."""
    import nimbleml_amd as nm

    cfg = GPTConfig(4096, 1024, 16, 2, 256)
    w = make_weights(cfg, seed=5, dtype=np.float32, rich=True)
    m = _build(cfg, w, np.float32)
    ids = random_ids((1, 70), cfg.vocab_size, seed=3)
    np.random.seed(0)
    out = nm.generate(m, ids, max_new_tokens=6, temperature=0.7, top_k=40, top_p=1.0)
    assert m.last_decode_persistent()
    u = np.random.RandomState(0).random_sample((6, 1))
    w32 = w
    kv = R.KVOracle(w32, cfg.num_heads, cfg.num_layers)
    lg = kv.step(out[:, :70])[:, -1]
    for t in range(6):
        want = R.sample_logits(lg[0], temperature=0.7, top_k=40, top_p=1.0, u=u[t, 0])
        x = lg[0].astype(np.float64) / 0.7
        th = np.sort(x)[-40]
        near_k = np.sort(np.abs(x - th))[1] < 2e-3
        p = np.exp(x - x.max()) * (x >= th)
        cdf = np.cumsum(p) / p.sum()
        near_u = np.min(np.abs(cdf - u[t, 0])) < 1e-4
        if near_k or near_u:
            break
        assert out[0, 70 + t] == want, t
        lg = kv.step(out[:, 70 + t:71 + t])[:, -1]


def test_persistent_and_multikernel_agree_sampled_fp32(gpu, monkeypatch):
    """Same uniforms through both decode steps give the same tokens. fp32: the two paths
    differ by ~1e-6 in the logits, far below the top-k gaps and CDF distances that a
    draw depends on (in fp16 the 50th/51st logit gap of this model is comparable to the
    fp16 rounding differences, so there the top-k set itself may differ)."""
    import nimbleml_amd as nm

    cfg = GPTConfig(8192, 1024, 16, 2, 512)
    w = make_weights(cfg, seed=9, dtype=np.float32, rich=True)
    m = _build(cfg, w, np.float32)
    ids = random_ids((1, 130), cfg.vocab_size, seed=4)
    np.random.seed(11)
    a = nm.generate(m, ids, max_new_tokens=30, temperature=0.8, top_k=50, top_p=1.0)
    assert m.last_decode_persistent()
    monkeypatch.setenv("NIMBLEML_PERSISTENT", "0")
    np.random.seed(11)
    b = nm.generate(m, ids, max_new_tokens=30, temperature=0.8, top_k=50, top_p=1.0)
    assert not m.last_decode_persistent()
    assert np.array_equal(a, b)
