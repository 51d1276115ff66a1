"""Parameter containers with the reference's attribute names and layouts.

``named_parameters`` (saveload.py) walks these exactly as the reference walks
its modules (NimbleML/utils/saveload.py:16-41), so checkpoints interchange.
  Dense      weights (in, out), biases (out,)          layers/dense.py:16-25
  Embedding  weights (rows, dim)                        layers/embedding.py:14-21
  RMSNorm    gamma (dim,), epsilon 1e-5                 layers/rms_norm.py:16-23
  MultiHeadAttention W_q/W_k/W_v/W_o, scale = sqrt(d_k) neural_network/attention.py:125-137
  FeedForward dense1 (d, ff·d), dense2 (ff·d, d)        neural_network/feed_forward.py:13-16
  FusedTransformerBlock ln1, mha, ln2, ffn              neural_network/transformer_fused.py:35-42
Initial values follow the same distributions (embedding N(0, 0.02), dense
U(−1, 1)/sqrt(in), zero biases, unit gammas) from NumPy's global generator.
The forward passes run in the GPT driver on the GPU (gpt.py).
"""
from __future__ import annotations

import contextlib
from math import sqrt

import numpy as np

from nimbleml_amd import np_backend
from nimbleml_amd.tensor import Tensor

_SKIP_INIT = [False]


@contextlib.contextmanager
def skip_init():
    """Construct parameters uninitialised (for models about to be loaded)."""
    _SKIP_INIT[0] = True
    try:
        yield
    finally:
        _SKIP_INIT[0] = False


def _init(fn, shape):
    if _SKIP_INIT[0]:
        return np.empty(shape, dtype=np_backend.dtype)
    return fn()


class Module:
    training = True

    def forward(self, x):
        raise NotImplementedError("Not implemented yet")

    def parameters(self):
        return []

    def _child_modules(self):
        for name, value in vars(self).items():
            if name.startswith("_"):
                continue
            if isinstance(value, Module):
                yield value
            elif isinstance(value, (list, tuple)):
                for item in value:
                    if isinstance(item, Module):
                        yield item

    def train(self):
        self.training = True
        for child in self._child_modules():
            child.train()

    def eval(self):
        self.training = False
        for child in self._child_modules():
            child.eval()

    def __call__(self, x):
        return self.forward(x)


class Sequential(Module):
    def __init__(self, *layers):
        self.layers = list(layers)

    def __iter__(self):
        return iter(self.layers)

    def parameters(self):
        params = []
        for layer in self.layers:
            if hasattr(layer, "parameters"):
                params.extend(layer.parameters())
        return params


def _param(arr, shape):
    return Tensor(np.asarray(arr, dtype=np_backend.dtype), shape, requires_grad=True)


class Dense(Module):
    def __init__(self, in_features, out_features, bias=True, weight_scale=None):
        self.in_features = in_features
        self.out_features = out_features
        scale = weight_scale if weight_scale is not None else 1.0 / sqrt(max(1, in_features))
        self.weights = _param(_init(lambda: np.random.uniform(-1.0, 1.0, (in_features, out_features))
                                    * scale, (in_features, out_features)),
                              (in_features, out_features))
        self.biases = _param(np.zeros(out_features), (out_features,)) if bias else None

    def parameters(self):
        return [self.weights] + ([self.biases] if self.biases is not None else [])


class Embedding(Module):
    def __init__(self, vocab_size, embed_dim, init_std: float = 0.02):
        self.vocab_size = vocab_size
        self.embed_dim = embed_dim
        self.weights = _param(_init(lambda: np.random.standard_normal((vocab_size, embed_dim))
                                    * init_std, (vocab_size, embed_dim)),
                              (vocab_size, embed_dim))

    def parameters(self):
        return [self.weights]


class RMSNorm(Module):
    def __init__(self, normalized_shape, epsilon=1e-5):
        self.normalized_shape = normalized_shape
        self.epsilon = epsilon
        self.gamma = _param(np.ones(normalized_shape), (normalized_shape,))

    def parameters(self):
        return [self.gamma]


class MultiHeadAttention(Module):
    def __init__(self, d_model, num_heads):
        if d_model % num_heads != 0:
            raise ValueError(f"d_model ({d_model}) must be divisible by num_heads ({num_heads}).")
        self.d_model = d_model
        self.num_heads = num_heads
        self.d_k = d_model // num_heads
        self.W_q = Dense(d_model, d_model)
        self.W_k = Dense(d_model, d_model)
        self.W_v = Dense(d_model, d_model)
        self.W_o = Dense(d_model, d_model)
        self.scale = float(self.d_k) ** 0.5
        self._rope_cache = None

    def parameters(self):
        params = []
        for layer in (self.W_q, self.W_k, self.W_v, self.W_o):
            params.extend(layer.parameters())
        return params


class FeedForward(Module):
    def __init__(self, d_model, ff_mult=4):
        hidden = ff_mult * d_model
        self.dense1 = Dense(d_model, hidden)
        self.dense2 = Dense(hidden, d_model)

    def parameters(self):
        return self.dense1.parameters() + self.dense2.parameters()


class FusedTransformerBlock(Module):
    """Pre-norm block (x + MHA(LN1(x)); x + FFN(LN2(x))). Its forward runs inside
    the GPT driver on the GPU, one launch sequence per block."""

    def __init__(self, d_model, num_heads, ff_mult=4, *, gradient_checkpointing: bool = False):
        self.d_model = d_model
        self.num_heads = num_heads
        self.gradient_checkpointing = bool(gradient_checkpointing)
        self.ln1 = RMSNorm(d_model)
        self.mha = MultiHeadAttention(d_model, num_heads)
        self.ln2 = RMSNorm(d_model)
        self.ffn = FeedForward(d_model, ff_mult=ff_mult)

    def parameters(self):
        params = []
        for layer in (self.ln1, self.mha, self.ln2, self.ffn):
            params.extend(layer.parameters())
        return params


class FusedGPTTrunk(Module):
    """All blocks plus the final RMSNorm as one module (transformer_fused.py:103-144)."""

    def __init__(self, blocks, ln: RMSNorm):
        self.blocks = list(blocks)
        self.ln = ln

    def parameters(self):
        params = []
        for block in self.blocks:
            params.extend(block.parameters())
        params.extend(self.ln.parameters())
        return params
