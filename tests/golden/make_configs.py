"""Write the oracle's fixtures for the benchmark-sized configs.

The reference's float16 path at these sizes is out of reach of NumPy's own float16
matmul (no BLAS: hours per prompt), so these fixtures come from the oracle
(oracle/gpt_ref.py), which restates that path op by op in the same NumPy dtypes and
computes its float16 products with oracle/halfmm.c, a bit-exact restatement of
NumPy's float16 matmul loop (tests/test_oracle.py pins both against NumPy itself and
against the reference's own fixtures). Weights and ids are regenerated from seeds by
the tests; the files hold only the decisions and the values the GPU is compared with.

  c3_fp16      C3: V32000 d1024 H16 L24, prompt 512, 64 greedy steps — per step the
               oracle's choice and top-2 gap (greedy on its own tokens), logits at a
               few steps.
  c4_fp16      C4: the same model, 32 prompts of lengths U[128, 1024], 256 sampled
               tokens each (T 0.8, top-k 50, top-p off), row b's draws from
               RandomState(1000 + b) — per row and step the pick and the largest logit
               change that cannot alter it; prefill logits of four rows; every row's
               logits at steps 0, 1, 63 and 255 (teacher-forced on the oracle's tokens).
  c5slice_fp16 C5 widths at two layers: V50304 d2048 H16 (head dim 128), one 4096-token
               sequence, rich weights — compute_loss, and the logits of four positions.

Usage:  python tests/golden/make_configs.py [c3 c4 c5]   (minutes; uses every core)
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import gpt_ref as R  # noqa: E402
from oracle.weights import C3, GPTConfig, c4_rows, make_weights, random_ids, row_uniforms  # noqa: E402

C3_SEED, C3_PROMPT_SEED, C3_PROMPT, C3_STEPS = 41, 42, 512, 64
C3_KEEP = (0, 1, 2, 31, 63)
C4_SEED, C4_ROWS_SEED, C4_ROWS, C4_NEW = 41, 5, 32, 256
C4_T, C4_K, C4_U_SEED = 0.8, 50, 1000
C4_KEEP = (0, 1, 63, 255)
C5SLICE = GPTConfig(50304, 2048, 16, 2, 4096)
C5_SEED, C5_IDS_SEED, C5_S = 43, 44, 4096
C5_KEEP = (0, 1, 2047, 4095)


def make_c3():
    cfg = C3
    w = make_weights(cfg, seed=C3_SEED, dtype=np.float16)
    prompt = random_ids((1, C3_PROMPT), cfg.vocab_size, C3_PROMPT_SEED)
    kv = R.KVOracle(w, cfg.num_heads, cfg.num_layers)
    lg = kv.step(prompt)[0, -1]
    toks, margins, keep = [], [], {}
    for t in range(C3_STEPS):
        if t in C3_KEEP:
            keep[f"logits_step{t}"] = lg.copy()
        tok = R.sample_logits(lg, temperature=0.0, top_k=0, top_p=1.0)
        toks.append(tok)
        margins.append(2.0 * R.sample_flip_tol(lg, 0.0, tok, temperature=0.0, top_k=0))
        if t + 1 < C3_STEPS:
            lg = kv.step(np.asarray([[tok]]))[0, -1]
    return dict(config=np.array([cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                                 cfg.max_seq_len, cfg.ff_mult]),
                seed=np.array(C3_SEED), prompt_seed=np.array(C3_PROMPT_SEED),
                prompt_len=np.array(C3_PROMPT), greedy=np.asarray(toks, dtype=np.int32),
                margins=np.asarray(margins, dtype=np.float32),
                keep_steps=np.asarray(C3_KEEP), **keep)


def make_c4():
    cfg = C3
    w = make_weights(cfg, seed=C4_SEED, dtype=np.float16)
    rows = c4_rows(cfg.vocab_size, C4_ROWS_SEED, C4_ROWS)
    u = row_uniforms(C4_NEW, C4_ROWS, C4_U_SEED)
    orc = R.RaggedKVOracle(w, cfg.num_heads, cfg.num_layers)
    lg = orc.prefill(rows)
    pre = lg[:4].copy()
    keep = {}
    toks = np.zeros((C4_NEW, C4_ROWS), dtype=np.int32)
    flip = np.zeros((C4_NEW, C4_ROWS), dtype=np.float32)
    for t in range(C4_NEW):
        if t in C4_KEEP:  # every row's logits, teacher-forced on the oracle's own tokens
            keep[f"logits_step{t}"] = lg.copy()
        for b in range(C4_ROWS):
            tok = R.sample_logits(lg[b], temperature=C4_T, top_k=C4_K, top_p=1.0, u=u[t, b])
            toks[t, b] = tok
            flip[t, b] = R.sample_flip_tol(lg[b], u[t, b], tok, temperature=C4_T, top_k=C4_K)
        if t + 1 < C4_NEW:
            lg = orc.step(toks[t])
        if t % 32 == 0:
            print(f"  c4 step {t}", flush=True)
    return dict(seed=np.array(C4_SEED), tokens=toks, flip_tol=flip, prefill_logits=pre,
                temperature=np.array(C4_T), top_k=np.array(C4_K),
                keep_steps=np.asarray(C4_KEEP), **keep)


def make_c5():
    cfg = C5SLICE
    w = make_weights(cfg, seed=C5_SEED, dtype=np.float16, rich=True)
    ids = random_ids((1, C5_S), cfg.vocab_size, C5_IDS_SEED)
    labels = random_ids((1, C5_S), cfg.vocab_size, C5_IDS_SEED + 1)
    h = R.hidden_states(w, ids, cfg.num_heads, cfg.num_layers)
    h2d = h.reshape(C5_S, cfg.d_model)
    logits = R._mm(h2d, np.swapaxes(w["token_emb.weights"], -2, -1))
    loss = R.crossentropy(logits, labels.reshape(-1))
    keep = {f"logits_pos{p}": logits[p].copy() for p in C5_KEEP}
    return dict(config=np.array([cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                                 cfg.max_seq_len, cfg.ff_mult]),
                seed=np.array(C5_SEED), ids_seed=np.array(C5_IDS_SEED), loss=np.array(loss),
                keep_pos=np.asarray(C5_KEEP), **keep)


def main(argv):
    which = argv or ["c3", "c4", "c5"]
    for name in which:
        t0 = time.time()
        out = {"c3": make_c3, "c4": make_c4, "c5": make_c5}[name]()
        out["numpy_version"] = np.array(np.__version__)
        fname = {"c3": "c3_fp16", "c4": "c4_fp16", "c5": "c5slice_fp16"}[name]
        np.savez_compressed(os.path.join(HERE, fname + ".npz"), **out)
        print(f"{fname}: {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
