"""Write golden fixtures by running the real reference NimbleML CPU path.

Runs in the build container only (it needs /root/reference and the reference's
own extension, built from its sources by ``make -C oracle`` into oracle/_ref/).
Each case runs in a fresh subprocess because the reference freezes its compute
dtype at import (NimbleML/utils/np_backend.py:157-176).

Weights come from ``oracle.weights.make_weights`` and are injected with the
reference's own ``NimbleML.load`` (NimbleML/utils/saveload.py:273-300), which
casts them to the compute dtype. Sampling runs seed NumPy's global legacy RNG
(the reference draws from it at models/generate.py:57,59); the fixture also
stores the uniforms ``RandomState(seed).random_sample((steps, batch))`` that
those draws consume, in order.

Usage:  python tests/golden/make_golden.py [case ...]
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF_ROOT = os.environ.get("NIMBLEML_REFERENCE", "/root/reference")
REF_EXT = os.path.join(REPO, "oracle", "_ref")

CASES = {
    # name: (config, dtype, rich)
    "tiny_fp32": ("TINY", "float32", False),
    "tiny_fp16": ("TINY", "float16", False),
    "tiny_rich_fp32": ("TINY", "float32", True),
    "tiny_rich_fp16": ("TINY", "float16", True),
    "small_fp32": ("SMALL", "float32", False),
    "small_rich_fp32": ("SMALL", "float32", True),
    "small_ragged_fp32": ("SMALL", "float32", True),
    "c3slice_fp16": ("C3SLICE", "float16", True),
    "tiny_rope_fp32": ("TINY", "float32", True),
    "tiny_rope_fp16": ("TINY", "float16", True),
    "ops_fp32": (None, "float32", False),
    "ops_fp16": (None, "float16", False),
}


def _config(name):
    from oracle.weights import GPTConfig, SMALL, TINY

    if name == "C3SLICE":
        # d1024 / 16 heads / vocab 32000 at two layers: real widths, short depth.
        return GPTConfig(32000, 1024, 16, 2, 64)
    return {"TINY": TINY, "SMALL": SMALL}[name]


def _build_model(cfg, w, use_rope=False):
    import NimbleML

    model = NimbleML.GPT(cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                         cfg.max_seq_len, ff_mult=cfg.ff_mult, fused_blocks=True,
                         use_rope=use_rope)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "w.npz")
        np.savez(path, **w)
        NimbleML.load(model, path)
    return model


def _forward_last(model, seq):
    from NimbleML.utils.tensor import Tensor

    ids = np.asarray(seq, dtype=np.int64)
    t = Tensor.from_int64(ids.ravel(), ids.shape)
    out = model.forward(t)
    return np.asarray(out.data).reshape(out.shape)


def _loss(model, ids, labels, ignore_index=None):
    from NimbleML.utils.tensor import Tensor

    t = Tensor.from_int64(ids.ravel(), ids.shape)
    loss = model.compute_loss(t, labels, ignore_index=ignore_index)
    return float(np.asarray(loss.data).reshape(-1)[0])


def _gen(model, ids, seed, steps, **kw):
    from NimbleML.models.generate import generate

    if seed is not None:
        np.random.seed(seed)
    return np.asarray(generate(model, ids, max_new_tokens=steps, **kw), dtype=np.int64)


def _uniforms(seed, steps, batch):
    return np.random.RandomState(seed).random_sample((steps, batch))


def run_model_case(name, cfg_name, dtype, rich):
    from oracle.weights import make_weights, random_ids

    cfg = _config(cfg_name)
    npdt = np.float16 if dtype == "float16" else np.float32
    seed = {"tiny": 11, "small": 23, "c3slice": 37}[name.split("_")[0]]
    from oracle.weights import rope_weights

    use_rope = "rope" in name
    w = make_weights(cfg, seed=seed, dtype=np.float32, rich=rich)
    if use_rope:
        w = rope_weights(w)
    model = _build_model(cfg, w, use_rope)
    out = {"config": np.array([cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, cfg.ff_mult], dtype=np.int64),
           "seed": np.array(seed), "rich": np.array(int(rich)), "dtype": np.array(dtype),
           "rope": np.array(int(use_rope))}

    if use_rope:
        b, s0, n = 2, 8, 24
        ids = random_ids((b, s0), cfg.vocab_size, seed)
        out["prompt"] = ids
        out["greedy"] = _gen(model, ids, None, n, temperature=0.0)
        out["greedy_logits"] = _forward_last(model, out["greedy"][:, :-1])
        lids = random_ids((2, 32), cfg.vocab_size, seed + 1)
        labels = random_ids((2, 32), cfg.vocab_size, seed + 2)
        out["loss_ids"], out["loss_labels"] = lids, labels
        out["loss"] = np.array(_loss(model, lids, labels))
        out["topk_tokens"] = _gen(model, ids, 123, n, temperature=0.8, top_k=50, top_p=1.0)
        out["topk_u"] = _uniforms(123, n, b)
    elif cfg_name == "TINY":
        b, s0, n = 2, 8, 24
        ids = random_ids((b, s0), cfg.vocab_size, seed)
        out["prompt"] = ids
        out["greedy"] = _gen(model, ids, None, n, temperature=0.0)
        out["greedy_logits"] = _forward_last(model, out["greedy"][:, :-1])
        lids = random_ids((2, 32), cfg.vocab_size, seed + 1)
        labels = random_ids((2, 32), cfg.vocab_size, seed + 2)
        out["loss_ids"], out["loss_labels"] = lids, labels
        out["loss"] = np.array(_loss(model, lids, labels))
        ign = labels.copy()
        ign[:, ::3] = -100
        out["loss_ignore_labels"] = ign
        out["loss_ignore"] = np.array(_loss(model, lids, ign, ignore_index=-100))
        out["loss_all_ignored"] = np.array(
            _loss(model, lids, np.full_like(labels, -100), ignore_index=-100))
        out["topk_tokens"] = _gen(model, ids, 123, n, temperature=0.8, top_k=50, top_p=1.0)
        out["topk_u"] = _uniforms(123, n, b)
        out["topp_tokens"] = _gen(model, ids, 321, n)  # defaults: T=0.8, top_k=0, top_p=0.9
        out["topp_u"] = _uniforms(321, n, b)
        out["reppen_tokens"] = _gen(model, ids, 555, n, temperature=0.8, top_k=20, top_p=1.0,
                                    repetition_penalty=1.3)
        out["reppen_u"] = _uniforms(555, n, b)
        out["greedy_reppen"] = _gen(model, ids, None, n, temperature=0.0,
                                    repetition_penalty=1.5)
    elif name == "small_ragged_fp32":
        lens = [5, 17, 40]
        n = 16
        for r, s0 in enumerate(lens):
            ids = random_ids((1, s0), cfg.vocab_size, seed + 100 + r)
            out[f"row{r}_prompt"] = ids
            out[f"row{r}_tokens"] = _gen(model, ids, 1000 + r, n, temperature=0.8, top_k=50,
                                         top_p=1.0)
            out[f"row{r}_u"] = _uniforms(1000 + r, n, 1)
    elif cfg_name == "SMALL":
        b, s0 = 8, 64
        n = 192 if not rich else 32
        ids = random_ids((b, s0), cfg.vocab_size, seed)
        out["prompt"] = ids
        out["greedy"] = _gen(model, ids, None, n, temperature=0.0)
        steps = [0, n - 1] if not rich else [0, 1, n - 1]
        out["logit_steps"] = np.array(steps)
        for t in steps:
            out[f"logits_step{t}"] = _forward_last(model, out["greedy"][:, :s0 + t])[:, -1]
        lids = random_ids((8, 256), cfg.vocab_size, seed + 1)
        labels = random_ids((8, 256), cfg.vocab_size, seed + 2)
        out["loss_ids"], out["loss_labels"] = lids, labels
        out["loss"] = np.array(_loss(model, lids, labels))
    elif cfg_name == "C3SLICE":
        s0, n = 32, 4
        ids = random_ids((1, s0), cfg.vocab_size, seed)
        out["prompt"] = ids
        out["greedy"] = _gen(model, ids, None, n, temperature=0.0)
        out["logit_steps"] = np.arange(n)
        for t in range(n):
            out[f"logits_step{t}"] = _forward_last(model, out["greedy"][:, :s0 + t])[:, -1]
        lids = random_ids((1, 48), cfg.vocab_size, seed + 1)
        labels = random_ids((1, 48), cfg.vocab_size, seed + 2)
        out["loss_ids"], out["loss_labels"] = lids, labels
        out["loss"] = np.array(_loss(model, lids, labels))
    for k, v in list(out.items()):
        if isinstance(v, np.ndarray) and v.dtype == np.float16 and npdt == np.float16:
            out[k] = v  # fp16 logits are stored exactly
    return out


def run_ops_case(dtype):
    from NimbleML.kernels.embedding_scatter import embedding_lookup
    from NimbleML.kernels.fused_gelu import fused_gelu_forward
    from NimbleML.kernels.fused_rmsnorm import fused_rmsnorm_forward
    from NimbleML.kernels.fused_sdpa import fused_sdpa_forward
    from NimbleML.kernels.fused_tied_crossentropy import fused_tied_crossentropy_forward
    from NimbleML.utils.mask import make_causal_mask

    npdt = np.float16 if dtype == "float16" else np.float32
    rng = np.random.default_rng(4242)
    out = {"dtype": np.array(dtype)}
    x = (rng.standard_normal((37, 96)) * 1.5).astype(npdt)
    g = (1.0 + 0.1 * rng.standard_normal(96)).astype(npdt)
    out["rms_x"], out["rms_g"] = x, g
    out["rms_out"] = np.asarray(fused_rmsnorm_forward(x, g, 1e-5)[0])
    gx = np.concatenate([np.linspace(-8, 8, 4001), rng.standard_normal(3000) * 3]).astype(npdt)
    out["gelu_x"] = gx
    out["gelu_out"] = np.asarray(fused_gelu_forward(gx)[0])
    bh, s, dk = 6, 29, 16
    q = rng.standard_normal((bh, s, dk)).astype(npdt)
    k = rng.standard_normal((bh, s, dk)).astype(npdt)
    v = rng.standard_normal((bh, s, dk)).astype(npdt)
    out["sdpa_q"], out["sdpa_k"], out["sdpa_v"] = q, k, v
    out["sdpa_out"] = np.asarray(fused_sdpa_forward(q, k, v, float(dk) ** 0.5,
                                                    make_causal_mask(s))[0])
    h = rng.standard_normal((45, 64)).astype(npdt)
    e = (0.3 * rng.standard_normal((300, 64))).astype(npdt)
    y = rng.integers(0, 300, size=45, dtype=np.int64)
    out["ce_h"], out["ce_e"], out["ce_y"] = h, e, y
    out["ce_loss"] = np.array(fused_tied_crossentropy_forward(h, e, y)[0])
    tab = rng.standard_normal((50, 24)).astype(npdt)
    ids = rng.integers(0, 50, size=(3, 11), dtype=np.int64)
    out["emb_w"], out["emb_ids"] = tab, ids
    out["emb_out"] = np.asarray(embedding_lookup(tab, ids))
    return out


def child(name):
    sys.path.insert(0, REF_ROOT)
    sys.path.insert(0, REF_EXT)
    sys.path.insert(0, REPO)
    cfg_name, dtype, rich = CASES[name]
    if cfg_name is None:
        out = run_ops_case(dtype)
    else:
        out = run_model_case(name, cfg_name, dtype, rich)
    import numpy
    out["numpy_version"] = np.array(numpy.__version__)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print(f"wrote {name}.npz", flush=True)


def main(argv):
    if len(argv) >= 2 and argv[0] == "--child":
        child(argv[1])
        return 0
    names = argv or list(CASES)
    for name in names:
        dtype = CASES[name][1]
        env = dict(os.environ, NIMBLEML_DEVICE="cpu", NIMBLEML_DTYPE=dtype)
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--child", name], env=env)
        if r.returncode != 0:
            return r.returncode
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
