"""Seeded GPT parameters under the reference's checkpoint names.

Names follow ``named_parameters`` (NimbleML/utils/saveload.py:16-41) applied to
``GPT`` (NimbleML/models/gpt.py:45-71): the token embedding, the learned
position table, ``Sequential`` children as ``blocks.layers.{i}`` with
``ln1/mha/ln2/ffn`` (neural_network/transformer_fused.py:39-42), the four MHA
projections (neural_network/attention.py:131-134), the two FFN denses
(neural_network/feed_forward.py:15-16) and the final RMSNorm ``ln.gamma``.
Layouts follow the layers: ``Dense`` weights ``(in, out)`` with bias ``(out,)``
(layers/dense.py:16-25), ``Embedding`` ``(rows, dim)`` (layers/embedding.py:14-21),
RMSNorm ``gamma`` ``(dim,)`` (layers/rms_norm.py:16-23).

Values: weights ~ N(0, 0.02); biases 0 and gammas 1 (the benchmark configs), or
with ``rich=True`` biases ~ N(0, 0.02) and gammas ~ 1 + N(0, 0.1) so that parity
tests see every bias and gamma. Each tensor draws from its own
``numpy.random.default_rng([seed, index])`` stream so a single layer can be
regenerated without the others.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class GPTConfig:
    vocab_size: int
    d_model: int
    num_heads: int
    num_layers: int
    max_seq_len: int
    ff_mult: int = 4

    @property
    def d_ff(self) -> int:
        return self.ff_mult * self.d_model

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads


TINY = GPTConfig(256, 64, 4, 2, 32)
SMALL = GPTConfig(4096, 256, 8, 6, 256)
C3 = GPTConfig(32000, 1024, 16, 24, 2048)
C5 = GPTConfig(50304, 2048, 16, 24, 4096)


def layer_param_shapes(cfg: GPTConfig):
    d, f = cfg.d_model, cfg.d_ff
    return [
        ("ln1.gamma", (d,)),
        ("mha.W_q.weights", (d, d)),
        ("mha.W_q.biases", (d,)),
        ("mha.W_k.weights", (d, d)),
        ("mha.W_k.biases", (d,)),
        ("mha.W_v.weights", (d, d)),
        ("mha.W_v.biases", (d,)),
        ("mha.W_o.weights", (d, d)),
        ("mha.W_o.biases", (d,)),
        ("ln2.gamma", (d,)),
        ("ffn.dense1.weights", (d, f)),
        ("ffn.dense1.biases", (f,)),
        ("ffn.dense2.weights", (f, d)),
        ("ffn.dense2.biases", (d,)),
    ]


def param_shapes(cfg: GPTConfig):
    """(name, shape) for every parameter, in a fixed order."""
    out = [
        ("token_emb.weights", (cfg.vocab_size, cfg.d_model)),
        ("pos_emb.weights", (cfg.max_seq_len, cfg.d_model)),
    ]
    for i in range(cfg.num_layers):
        out.extend((f"blocks.layers.{i}.{n}", s) for n, s in layer_param_shapes(cfg))
    out.append(("ln.gamma", (cfg.d_model,)))
    return out


def _draw(name: str, shape, seed: int, index: int, rich: bool) -> np.ndarray:
    rng = np.random.default_rng([seed, index])
    if name.endswith(".gamma"):
        if not rich:
            return np.ones(shape, dtype=np.float32)
        return (1.0 + 0.1 * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
    if name.endswith(".biases"):
        if not rich:
            return np.zeros(shape, dtype=np.float32)
    return (0.02 * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)


def make_weights(cfg: GPTConfig, seed: int = 0, dtype=np.float32, rich: bool = False,
                 layers=None) -> dict:
    """All parameters as ``{name: ndarray}`` in ``dtype``.

    ``layers`` restricts block parameters to those layer indices (embeddings and
    the final gamma are always included).
    """
    out = {}
    for index, (name, shape) in enumerate(param_shapes(cfg)):
        if layers is not None and name.startswith("blocks.layers."):
            if int(name.split(".")[2]) not in layers:
                continue
        out[name] = _draw(name, shape, seed, index, rich).astype(dtype)
    return out


def c4_rows(vocab: int, seed: int = 5, batch: int = 32):
    """The C4 prompts: lengths uniform in [128, 1024], ids
    uniform in [0, vocab), from one seeded generator."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 1025, batch)
    return [rng.integers(0, vocab, int(n)).astype(np.int64) for n in lens]


def row_uniforms(steps: int, batch: int, seed0: int = 1000) -> np.ndarray:
    """u[t, b]: the t-th draw of ``RandomState(seed0 + b)``, which is what the reference
    consumes when it generates row b alone after ``np.random.seed(seed0 + b)``
    (models/generate.py:57,59: one draw per row per step)."""
    return np.stack([np.random.RandomState(seed0 + b).random_sample(steps)
                     for b in range(batch)], axis=1)


def random_ids(shape, vocab: int, seed: int) -> np.ndarray:
    """Uniform token ids in [0, vocab) as int64."""
    return np.random.default_rng([seed, 7919]).integers(0, vocab, size=shape, dtype=np.int64)


ROPE_QK_SCALE = 6.0


def rope_weights(w: dict) -> dict:
    """Parameters of a ``use_rope=True`` model from :func:`make_weights` output (apply
    before any cast): no ``pos_emb.weights`` (models/gpt.py:46), and W_q, W_k scaled by
    ROPE_QK_SCALE so that q·k is large enough for rotary positions to move the logits
    visibly (a test choice, not a reference default)."""
    out = {k: v for k, v in w.items() if k != "pos_emb.weights"}
    for k in out:
        if k.endswith("mha.W_q.weights") or k.endswith("mha.W_k.weights"):
            out[k] = out[k] * np.float32(ROPE_QK_SCALE)
    return out
