"""Batched decode at the C3/C4 widths (d_model 1024, head_dim 64): ragged rows through
the multi-kernel step (skinny MFMA projections, split-K attention over the cache).
Each row must generate what it generates alone (the reference runs rows one at a time,
models/generate.py:80-89), checked against the oracle's greedy choice wherever its
top-2 margin exceeds the fp16 logit tolerance."""
import numpy as np
import pytest

from oracle import gpt_ref as R
from oracle.weights import GPTConfig, make_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lens", [[20, 300, 64, 65, 129, 7, 250, 33, 190, 100, 140, 41],
                                  [5 + 13 * i for i in range(40)]])
def test_ragged_batch_rows_match_oracle_fp16(gpu, lens):
    """12 rows (one 16-row MFMA tile) and 40 rows (three tiles, the last partly empty)."""
    import nimbleml_amd as nm

    cfg = GPTConfig(4096, 1024, 16, 2, 1024)
    w = make_weights(cfg, seed=17, dtype=np.float16, rich=True)
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float16)
    rng = np.random.default_rng(3)
    rows = [rng.integers(0, cfg.vocab_size, n) for n in lens]
    new = 20
    out = nm.generate(m, rows, max_new_tokens=new, temperature=0.0)
    assert not m.last_decode_persistent()
    w32 = {k: v.astype(np.float32) for k, v in w.items()}
    compared = 0
    for b, r in enumerate(rows):
        got = np.asarray(out[b])
        assert np.array_equal(got[:len(r)], r)
        kv = R.KVOracle(w32, cfg.num_heads, cfg.num_layers)
        lg = kv.step(got[None, :len(r)])[0, -1]
        for t in range(new):
            top2 = np.sort(lg.astype(np.float64))[-2:]
            if top2[1] - top2[0] <= 3e-2:
                break
            assert got[len(r) + t] == int(np.argmax(lg)), (b, t)
            compared += 1
            lg = kv.step(got[None, len(r) + t:len(r) + t + 1])[0, -1]
    assert compared >= 3 * len(rows), compared


def test_cached_prefill_with_offset_matches_full_forward_fp16(gpu):
    """A prompt chunk appended after a cached prefix (queries start at position 100):
    logits equal those of one full forward over the whole sequence."""
    import nimbleml_amd as nm
    from oracle.weights import random_ids

    cfg = GPTConfig(2048, 1024, 16, 2, 512)
    w = make_weights(cfg, seed=21, dtype=np.float16, rich=True)
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float16)
    ids = random_ids((2, 250), cfg.vocab_size, seed=8)
    full = m.forward(ids).numpy().astype(np.float64)
    a, cache = m.forward_with_cache(ids[:, :100])
    b, cache = m.forward_with_cache(ids[:, 100:], cache)
    assert np.abs(a.numpy().astype(np.float64) - full[:, :100]).max() <= 3e-2
    assert np.abs(b.numpy().astype(np.float64) - full[:, 100:]).max() <= 3e-2
    want = R.forward({k: v.astype(np.float32) for k, v in w.items()}, ids, cfg.num_heads,
                     cfg.num_layers)
    assert np.abs(full - want).max() <= 3e-2


def test_fused_rmsnorm_decode_matches_separate_kernels_fp16(gpu, monkeypatch):
    """The batched decode step with RMSNorm fused into the projections that consume it
    (sums of squares from the residual GEMMs) and with the separate RMSNorm kernels: the
    rounding points are the same, only the fp32 order of the mean's sum differs, so
    the sampled tokens (same uniforms) agree."""
    import nimbleml_amd as nm

    cfg = GPTConfig(4096, 1024, 16, 3, 512)
    w = make_weights(cfg, seed=23, dtype=np.float16, rich=True)
    m = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                           cfg.max_seq_len, dtype=np.float16)
    rng = np.random.default_rng(9)
    rows = [rng.integers(0, cfg.vocab_size, int(n)) for n in rng.integers(30, 200, 24)]
    np.random.seed(4)
    fused = nm.generate(m, rows, max_new_tokens=24, temperature=0.0)
    monkeypatch.setenv("NIMBLEML_FUSE_NORM", "0")
    np.random.seed(4)
    sep = nm.generate(m, rows, max_new_tokens=24, temperature=0.0)
    same = sum(np.array_equal(np.asarray(a), np.asarray(b)) for a, b in zip(fused, sep))
    assert same >= len(rows) - 1, same
