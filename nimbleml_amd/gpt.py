"""GPT on the MI355X: the reference's model API over a device-resident driver.

``GPT`` keeps NimbleML's constructor, module tree and parameter names
(NimbleML/models/gpt.py:11-71) so checkpoints and user code carry over; its
forward, ``compute_loss``, ``forward_with_cache`` and ``generate`` run on the GPU
through the C-ABI (include/nimbleml_hip.h). Parameters live on the host as the
reference's Tensors and are uploaded once — transposed to (out, in) and with
Q/K/V stacked — into one device allocation, re-uploaded after ``load``.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from nimbleml_amd import _native as N
from nimbleml_amd import np_backend
from nimbleml_amd.grad_mode import is_grad_enabled
from nimbleml_amd.layers import (Embedding, FusedGPTTrunk, FusedTransformerBlock, Module,
                                 RMSNorm, Sequential, block_device_arrays, rope_device_arrays)
from nimbleml_amd.tensor import Tensor


def _ids_array(input_ids) -> np.ndarray:
    if isinstance(input_ids, Tensor):
        return np.asarray(input_ids.data, dtype=np.int64).reshape(input_ids.shape)
    return np.asarray(input_ids, dtype=np.int64)


class KVCache:
    """Per-layer K/V cache on the device (the ``cache`` of ``forward_with_cache``)."""

    def __init__(self, model: "GPT", batch: int):
        self.model = model
        self.batch = int(batch)
        h = C.c_void_p()
        self._model_handle = model._device_model()
        N.check(N.lib.nml_cache_create(self._model_handle, self.batch, C.byref(h)))
        self._h = h
        self._owner = model._dev  # keeps the device model alive while the cache exists

    @property
    def length(self) -> int:
        n = C.c_size_t()
        N.check(N.lib.nml_cache_length(self._h, C.byref(n)))
        return int(n.value)

    def __del__(self):
        try:
            if self._h:
                N.lib.nml_cache_destroy(self._h)
                self._h = None
        except Exception:
            pass


class GPT(Module):
    """Minimal GPT-style autoregressive language model (models/gpt.py:11-211)."""

    def __init__(self, vocab_size, d_model, num_heads, num_layers, max_seq_len, ff_mult=4, *,
                 fused_blocks: bool = True, fused_trunk: bool = False,
                 gradient_checkpointing: bool = False, use_rope: bool = False):
        if d_model % num_heads != 0:
            raise ValueError(f"d_model ({d_model}) must be divisible by num_heads ({num_heads}).")
        if fused_trunk and not fused_blocks:
            raise ValueError("fused_trunk requires fused_blocks=True.")
        if not fused_blocks:
            raise ValueError("nimbleml_amd implements the fused_blocks=True path of GPT.")
        self.vocab_size = vocab_size
        self.d_model = d_model
        self.num_heads = num_heads
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        self.ff_mult = ff_mult
        self.fused_blocks = fused_blocks
        self.fused_trunk = fused_trunk
        self.gradient_checkpointing = bool(gradient_checkpointing)
        self.use_rope = bool(use_rope)
        self.token_emb = Embedding(vocab_size, d_model)
        # rotary positions replace the learned table (models/gpt.py:46-53)
        self.pos_emb = None if self.use_rope else Embedding(max_seq_len, d_model)
        if self.use_rope:
            from nimbleml_amd.rope import build_rope_cache

            self._rope_cos, self._rope_sin = build_rope_cache(max_seq_len, d_model // num_heads)
        else:
            self._rope_cos = self._rope_sin = None
        block_modules = [FusedTransformerBlock(d_model, num_heads, ff_mult,
                                               gradient_checkpointing=gradient_checkpointing)
                         for _ in range(num_layers)]
        if self.use_rope:
            for block in block_modules:
                block.mha._rope_cache = (self._rope_cos, self._rope_sin)
        self.ln = RMSNorm(d_model)
        self.blocks = (FusedGPTTrunk(block_modules, self.ln) if fused_trunk
                       else Sequential(*block_modules))
        self._dtype = np.dtype(np_backend.dtype)
        self._dev = None

    # ------------------------------------------------------------------ params
    @property
    def _block_list(self):
        return self.blocks.blocks if self.fused_trunk else self.blocks.layers

    def parameters(self):
        params = []
        for layer in (self.token_emb, self.blocks):
            params.extend(layer.parameters())
        if self.pos_emb is not None:
            params.extend(self.pos_emb.parameters())
        if not self.fused_trunk:
            params.extend(self.ln.parameters())
        return params

    def _invalidate_device(self):
        self._dev = None  # re-upload on next use (the old handle is freed by __del__ below)

    def _device_arrays(self):
        """(kind, layer, host array in device layout) for every device parameter."""
        dt = self._dtype

        def a(t, shape=None):
            return np.ascontiguousarray(np.asarray(t.data, dtype=dt).reshape(shape or t.shape))

        out = [(N.P_TOKEN_EMB, 0, a(self.token_emb.weights)), (N.P_LN_F, 0, a(self.ln.gamma))]
        if self.use_rope:
            out += rope_device_arrays((self._rope_cos, self._rope_sin),
                                      self.d_model // self.num_heads, dt)
        else:
            out.append((N.P_POS_EMB, 0, a(self.pos_emb.weights)))
        for i, blk in enumerate(self._block_list):
            out += block_device_arrays(blk, i, dt)
        return out

    def _device_model(self):
        if self._dev is not None:
            return self._dev.handle
        N.ensure_init()
        for blk in self._block_list:
            for dense in (blk.mha.W_q, blk.mha.W_k, blk.mha.W_v, blk.mha.W_o,
                          blk.ffn.dense1, blk.ffn.dense2):
                if dense.biases is None:
                    raise ValueError("the HIP path expects Dense layers with biases")
        self._dev = _DeviceModel(self)
        return self._dev.handle

    def to_device(self):
        """Upload (again) the current host parameters."""
        self._dev = None
        self._device_model()
        return self

    # ----------------------------------------------------------------- inputs
    def _check_ids(self, ids: np.ndarray):
        if ids.ndim != 2:
            raise ValueError(f"input_ids must be 2D (batch, seq), got shape {ids.shape}.")
        if ids.shape[1] > self.max_seq_len:
            raise ValueError(f"Sequence length {ids.shape[1]} exceeds maximum sequence length "
                             f"{self.max_seq_len}")
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= self.vocab_size):
            raise ValueError(f"Token ID out of range [0, {self.vocab_size})")

    def _logits_array(self, shape):
        return N.DeviceArray(shape, self._dtype)

    # ---------------------------------------------------------------- forward
    def forward(self, input_ids):
        """All-position logits (batch, seq, vocab) on the device (models/gpt.py:92-121)."""
        ids = _ids_array(input_ids)
        self._check_ids(ids)
        h = self._device_model()
        b, s = ids.shape
        out = self._logits_array((b, s, self.vocab_size))
        dids = N.DeviceArray.from_host(ids)
        N.check(N.lib.nml_model_forward(h, dids.ptr, b, s, out.ptr, 0))
        return Tensor(out, (b, s, self.vocab_size))

    def forward_last(self, input_ids):
        """Logits of the last position only, (batch, vocab)."""
        ids = _ids_array(input_ids)
        self._check_ids(ids)
        h = self._device_model()
        b, s = ids.shape
        out = self._logits_array((b, self.vocab_size))
        dids = N.DeviceArray.from_host(ids)
        N.check(N.lib.nml_model_forward(h, dids.ptr, b, s, out.ptr, 1))
        return Tensor(out, (b, self.vocab_size))

    def forward_with_cache(self, input_ids, cache=None):
        """Append ``input_ids`` (batch, s) to the KV cache and return their logits
        (batch, s, vocab) — the hook models/generate.py:93-100 looks for."""
        ids = _ids_array(input_ids)
        if ids.ndim != 2:
            raise ValueError(f"input_ids must be 2D (batch, seq), got shape {ids.shape}.")
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= self.vocab_size):
            raise ValueError(f"Token ID out of range [0, {self.vocab_size})")
        h = self._device_model()
        b, s = ids.shape
        if cache is None:
            cache = KVCache(self, b)
        if cache.model is not self or cache.batch != b:
            raise ValueError("cache was created for another model or batch size")
        if cache._model_handle is not h:
            raise ValueError("parameters were reloaded since this cache was created; start a "
                             "new cache")
        if cache.length + s > self.max_seq_len:
            raise ValueError(f"Sequence length {cache.length + s} exceeds maximum sequence "
                             f"length {self.max_seq_len}")
        out = self._logits_array((b, s, self.vocab_size))
        dids = N.DeviceArray.from_host(ids)
        N.check(N.lib.nml_model_forward_cached(h, cache._h, dids.ptr, b, s, out.ptr, 0))
        return Tensor(out, (b, s, self.vocab_size)), cache

    def compute_loss(self, input_ids, labels, ignore_index=None):
        """Mean tied-head cross-entropy (models/gpt.py:123-137); logits are formed in
        row chunks on the device and never all at once.

        When gradients are enabled (``grad_mode``) and the parameters require them, the
        device keeps what the backward needs, and
        ``loss.backward()`` adds every parameter's gradient to its ``grad``
        (losses/cross_entropy.py:166-191 and the array-level backward of
        neural_network/_fused_arrays.py): in the compute dtype, or float32 where an optimizer
        pinned ``_grad_dtype`` (optimizers/optimizer.py:33-38).
        """
        ids = _ids_array(input_ids)
        self._check_ids(ids)
        b, s = ids.shape
        lab = np_backend.as_label_indices(labels, batch_size=b * s)
        h = self._device_model()
        dids = N.DeviceArray.from_host(ids)
        dlab = N.DeviceArray.from_host(lab)
        loss = C.c_double()
        has_ign = ignore_index is not None
        train = is_grad_enabled() and any(p.requires_grad for p in self.parameters())
        fn = N.lib.nml_model_loss_train if train else N.lib.nml_model_loss
        N.check(fn(h, dids.ptr, dlab.ptr, b, s, int(ignore_index) if has_ign else 0,
                   int(has_ign), C.byref(loss)))
        # The reference wraps the loss in a compute-dtype Tensor (losses/cross_entropy.py:158-164).
        out = Tensor([0.0], (), requires_grad=train)
        out.data = np.asarray([loss.value], dtype=self._dtype)
        if train:
            dev = self._dev
            gen = self._saved_generation()

            def _backward():
                if self._dev is not dev:
                    raise RuntimeError("parameters were re-uploaded since this loss was "
                                       "computed; compute the loss again")
                if self._saved_generation() != gen:
                    raise RuntimeError("activations were overwritten by a later compute_loss; "
                                       "compute this loss again before its backward()")
                N.check(N.lib.nml_model_zero_grad(h))
                N.check(N.lib.nml_model_backward(h, float(out.grad[0])))
                self._pull_grads()

            out._backward = _backward
        return out

    def _saved_generation(self) -> int:
        g = C.c_ulonglong()
        N.check(N.lib.nml_model_saved_generation(self._dev.handle, C.byref(g)))
        return int(g.value)

    def _grad_array(self, kind, layer, shape):
        """Device gradient of parameter (kind, layer) as a host float32 array."""
        ptr = C.c_void_p()
        N.check(N.lib.nml_model_grad_ptr(self._dev.handle, kind, layer, C.byref(ptr)))
        out = np.empty(shape, dtype=np.float32)
        N.check(N.lib.nml_memcpy_d2h(out.ctypes.data, ptr, out.nbytes))
        return out

    def _pull_grads(self):
        """Add the device gradients of one backward to the parameters' ``grad``, in the
        reference layouts ((in, out) weights, Q/K/V split)."""
        d, f = self.d_model, self.ff_mult * self.d_model
        g = self._grad_array
        self.token_emb.weights._accumulate_grad(g(N.P_TOKEN_EMB, 0, (self.vocab_size, d)))
        if self.pos_emb is not None:
            self.pos_emb.weights._accumulate_grad(g(N.P_POS_EMB, 0, (self.max_seq_len, d)))
        self.ln.gamma._accumulate_grad(g(N.P_LN_F, 0, (d,)))
        for i, blk in enumerate(self._block_list):
            m = blk.mha
            wqkv = g(N.P_WQKV, i, (3 * d, d))
            bqkv = g(N.P_BQKV, i, (3 * d,))
            for j, dense in enumerate((m.W_q, m.W_k, m.W_v)):
                dense.weights._accumulate_grad(wqkv[j * d:(j + 1) * d].T)
                dense.biases._accumulate_grad(bqkv[j * d:(j + 1) * d])
            m.W_o.weights._accumulate_grad(g(N.P_WO, i, (d, d)).T)
            m.W_o.biases._accumulate_grad(g(N.P_BO, i, (d,)))
            blk.ln1.gamma._accumulate_grad(g(N.P_LN1, i, (d,)))
            blk.ln2.gamma._accumulate_grad(g(N.P_LN2, i, (d,)))
            blk.ffn.dense1.weights._accumulate_grad(g(N.P_W1, i, (f, d)).T)
            blk.ffn.dense1.biases._accumulate_grad(g(N.P_B1, i, (f,)))
            blk.ffn.dense2.weights._accumulate_grad(g(N.P_W2, i, (d, f)).T)
            blk.ffn.dense2.biases._accumulate_grad(g(N.P_B2, i, (d,)))

    @classmethod
    def from_arrays(cls, arrays, vocab_size, d_model, num_heads, num_layers, max_seq_len,
                    ff_mult=4, dtype=None, **kwargs):
        """Build a model directly from ``{name: array}`` (reference checkpoint names)
        without drawing random initial weights first."""
        from nimbleml_amd import layers
        from nimbleml_amd.saveload import load_arrays

        old = np_backend.dtype
        if dtype is not None:
            np_backend.set_dtype(np.dtype(dtype).name)
        try:
            with layers.skip_init():
                m = cls(vocab_size, d_model, num_heads, num_layers, max_seq_len, ff_mult, **kwargs)
        finally:
            np_backend.set_dtype(np.dtype(old).name)
        return load_arrays(m, arrays)

    def generate(self, input_ids, **kwargs):
        """Autoregressive generation (see ``nimbleml_amd.generate.generate``)."""
        from nimbleml_amd.generate import generate as _generate

        return _generate(self, input_ids, **kwargs)

    def last_decode_ms(self) -> float:
        """Average device time of one decode step in the last generate() call."""
        ms = C.c_float()
        N.check(N.lib.nml_model_last_decode_ms(self._device_model(), C.byref(ms)))
        return float(ms.value)

    def last_decode_persistent(self) -> bool:
        """Whether the last generate() ran the persistent one-launch-per-token step."""
        v = C.c_int()
        N.check(N.lib.nml_model_last_decode_path(self._device_model(), C.byref(v)))
        return bool(v.value)

    def __del__(self):
        self._dev = None


class _DeviceModel:
    """Owns the C model handle."""

    def __init__(self, model: GPT):
        h = C.c_void_p()
        N.check(N.lib.nml_model_create(model.vocab_size, model.d_model, model.num_heads,
                                       model.num_layers, model.max_seq_len,
                                       model.ff_mult * model.d_model,
                                       N.np_dtype_code(model._dtype), C.byref(h)))
        self.handle = h
        try:
            for kind, layer, arr in model._device_arrays():
                N.check(N.lib.nml_model_set_param(h, kind, layer, arr.ctypes.data, arr.nbytes))
        except Exception:
            N.lib.nml_model_destroy(h)
            self.handle = None
            raise

    def __del__(self):
        try:
            if self.handle:
                N.lib.nml_model_destroy(self.handle)
                self.handle = None
        except Exception:
            pass
