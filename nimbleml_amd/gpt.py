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
import weakref

import numpy as np

from nimbleml_amd import _native as N
from nimbleml_amd import np_backend
from nimbleml_amd.grad_mode import is_grad_enabled
from nimbleml_amd.layers import (Embedding, FusedGPTTrunk, FusedTransformerBlock, Module,
                                 RMSNorm, Sequential, TransformerBlock, block_device_arrays,
                                 rope_device_arrays)
from nimbleml_amd.tensor import Tensor

# Every live GPT, so that an optimizer given ``model.parameters()`` finds its model.
_MODELS = weakref.WeakSet()


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
        self.lengths = None  # per-row lengths of a ragged prefill (None: all rows alike)

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
        if use_rope and not fused_blocks:  # models/gpt.py:44-45
            raise ValueError("use_rope requires fused_blocks=True (RoPE is applied in the "
                             "fused MHA path).")
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
        if fused_blocks:
            block_modules = [FusedTransformerBlock(d_model, num_heads, ff_mult,
                                                   gradient_checkpointing=gradient_checkpointing)
                             for _ in range(num_layers)]
        else:  # models/gpt.py:66-67: the unfused block, the same function and parameters
            block_modules = [TransformerBlock(d_model, num_heads, ff_mult)
                             for _ in range(num_layers)]
        if self.use_rope:
            for block in block_modules:
                block.mha._rope_cache = (self._rope_cos, self._rope_sin)
        self.ln = RMSNorm(d_model)
        self.blocks = (FusedGPTTrunk(block_modules, self.ln) if fused_trunk
                       else Sequential(*block_modules))
        self._dtype = np.dtype(np_backend.dtype)
        self._dev = None
        self._host_stale = False   # device parameters changed since the host Tensors
        self._arena_grads = None   # (device model, {id(param): grad}) when they agree
        self._adam_stash = None    # optimizer state kept across a device re-upload
        _MODELS.add(self)

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
        """The host parameters changed (``load``): re-upload them on next use. The AdamW state
        of the old device copy (moments, fp16 masters) moves to the new one, as the
        reference's optimizer keeps its state across a ``load``."""
        self._stash_adam()
        self._dev = None  # the old handle is freed by _DeviceModel.__del__
        self._host_stale = False
        self._arena_grads = None

    # ---------------------------------------------------------- device layout
    def _device_shape(self, kind):
        d, f = self.d_model, self.ff_mult * self.d_model
        return {N.P_TOKEN_EMB: (self.vocab_size, d), N.P_POS_EMB: (self.max_seq_len, d),
                N.P_LN_F: (d,), N.P_LN1: (d,), N.P_LN2: (d,), N.P_WQKV: (3 * d, d),
                N.P_BQKV: (3 * d,), N.P_WO: (d, d), N.P_BO: (d,), N.P_W1: (f, d), N.P_B1: (f,),
                N.P_W2: (d, f), N.P_B2: (d,)}[kind]

    def _param_layout(self):
        """Where each parameter lives in the device layout: (Tensor, kind, layer, first row,
        rows, transposed). Weights are stored (out, in), the reference's transpose; W_q,
        W_k, W_v are the row blocks of the stacked (3d, d) weight, their biases the thirds
        of the stacked bias."""
        d = self.d_model
        out = [(self.token_emb.weights, N.P_TOKEN_EMB, 0, 0, None, False)]
        if self.pos_emb is not None:
            out.append((self.pos_emb.weights, N.P_POS_EMB, 0, 0, None, False))
        out.append((self.ln.gamma, N.P_LN_F, 0, 0, None, False))
        for i, blk in enumerate(self._block_list):
            m = blk.mha
            out.append((blk.ln1.gamma, N.P_LN1, i, 0, None, False))
            for j, dense in enumerate((m.W_q, m.W_k, m.W_v)):
                out.append((dense.weights, N.P_WQKV, i, j * d, d, True))
                out.append((dense.biases, N.P_BQKV, i, j * d, d, False))
            out += [(m.W_o.weights, N.P_WO, i, 0, None, True),
                    (m.W_o.biases, N.P_BO, i, 0, None, False),
                    (blk.ln2.gamma, N.P_LN2, i, 0, None, False),
                    (blk.ffn.dense1.weights, N.P_W1, i, 0, None, True),
                    (blk.ffn.dense1.biases, N.P_B1, i, 0, None, False),
                    (blk.ffn.dense2.weights, N.P_W2, i, 0, None, True),
                    (blk.ffn.dense2.biases, N.P_B2, i, 0, None, False)]
        return out

    def _param_ranges(self):
        """{id(param): (kind, layer, first element, elements)} in the device layout."""
        out = {}
        for t, kind, layer, r0, rows, _tr in self._param_layout():
            shape = self._device_shape(kind)
            row = int(np.prod(shape[1:], dtype=np.int64)) if len(shape) > 1 else 1
            n = (rows if rows is not None else shape[0]) * row
            out[id(t)] = (kind, layer, r0 * row, n)
        return out

    def _read_device(self, ptr_of, dtype, params=None):
        """{id(param): array in the reference's layout} read from the device arrays that
        ``ptr_of(kind, layer)`` points to (parameters, gradients, moments, masters)."""
        want = None if params is None else {id(p) for p in params}
        blocks, out = {}, {}
        for t, kind, layer, r0, rows, tr in self._param_layout():
            if want is not None and id(t) not in want:
                continue
            if (kind, layer) not in blocks:
                a = np.empty(self._device_shape(kind), dtype=dtype)
                N.check(N.lib.nml_memcpy_d2h(a.ctypes.data, ptr_of(kind, layer), a.nbytes))
                blocks[(kind, layer)] = a
            a = blocks[(kind, layer)]
            v = a if rows is None else a[r0:r0 + rows]
            out[id(t)] = np.ascontiguousarray(v.T if tr else v).reshape(t.shape)
        return out

    def _write_device(self, ptr_of, dtype, values):
        """Write {id(param): array in the reference's layout} into the device arrays that
        ``ptr_of(kind, layer)`` points to; rows of a stacked block without a value keep
        theirs."""
        groups = {}
        for t, kind, layer, r0, rows, tr in self._param_layout():
            if id(t) in values:
                groups.setdefault((kind, layer), []).append((t, r0, rows, tr))
        for (kind, layer), items in groups.items():
            shape = self._device_shape(kind)
            whole = len(items) == 1 and items[0][2] is None
            a = np.empty(shape, dtype=dtype)
            if not whole and sum(it[2] for it in items) != shape[0]:
                N.check(N.lib.nml_memcpy_d2h(a.ctypes.data, ptr_of(kind, layer), a.nbytes))
            for t, r0, rows, tr in items:
                v = np.asarray(values[id(t)], dtype=dtype)
                if tr:
                    v = v.reshape(t.shape).T
                tgt = a if rows is None else a[r0:r0 + rows]
                tgt[...] = v.reshape(tgt.shape)
            N.check(N.lib.nml_memcpy_h2d(ptr_of(kind, layer), a.ctypes.data, a.nbytes))

    def _ptr(self, fn, kind, layer, which=0):
        if fn is N.lib.nml_model_adam_moments:
            a, b = C.c_void_p(), C.c_void_p()
            N.check(fn(self._dev.handle, kind, layer, C.byref(a), C.byref(b)))
            return (a, b)[which]
        p = C.c_void_p()
        N.check(fn(self._dev.handle, kind, layer, C.byref(p)))
        return p

    # ------------------------------------------------------------ host sync
    def sync_to_host(self):
        """Copy the device parameters into the host Tensors (after optimizer steps on the
        device), in the reference's layouts, so ``save``, ``named_parameters`` and reads of
        ``param.data`` see the trained values. A no-op when the host is current."""
        if self._dev is None or not self._host_stale:
            return self
        vals = self._read_device(lambda k, l: self._ptr(N.lib.nml_model_param_ptr, k, l),
                                 self._dtype)
        for t, *_ in self._param_layout():
            t.data[...] = vals[id(t)].ravel()
            t._bump_version()
        self._host_stale = False
        return self

    def _push_grads(self, params):
        """Put the host ``grad`` of ``params`` (zeros where it is None) into the device
        gradient arena, unless the arena already holds exactly those arrays (one backward
        since the gradients were cleared)."""
        rec = self._arena_grads
        if rec is not None and rec[0] is self._dev and all(
                p.grad is rec[1].get(id(p)) for p in params):
            return
        vals = {id(p): (p.grad if p.grad is not None else np.zeros(p.size, np.float32))
                for p in params}
        self._write_device(lambda k, l: self._ptr(N.lib.nml_model_grad_ptr, k, l), np.float32,
                           vals)
        self._arena_grads = None

    # ------------------------------------------------------ optimizer state
    def _adam_pointers(self, which):
        if which == "master":
            return lambda k, l: self._ptr(N.lib.nml_model_adam_master, k, l)
        i = 0 if which == "m" else 1
        return lambda k, l: self._ptr(N.lib.nml_model_adam_moments, k, l, i)

    def _adam_read(self, which, params=None):
        return self._read_device(self._adam_pointers(which), np.float32, params)

    def _adam_write(self, which, values):
        self._write_device(self._adam_pointers(which), np.float32, values)

    def _stash_adam(self):
        if self._dev is None or not getattr(self._dev, "adam", False):
            return
        st = {w: self._adam_read(w) for w in ("m", "v")}
        if self._dtype == np.float16:
            st["master"] = self._adam_read("master")
        self._adam_stash = st

    def _adam_state_ready(self):
        """Allocate the device AdamW state (restoring one carried over a re-upload)."""
        h = self._device_model()
        if getattr(self._dev, "adam", False):
            return h
        N.check(N.lib.nml_model_adam_state_init(h))
        self._dev.adam = True
        if self._adam_stash is not None:
            for which, vals in self._adam_stash.items():
                self._adam_write(which, vals)
            self._adam_stash = None
        return h

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
        """Upload (again) the current host parameters (after changing them in place). The
        device optimizer state carries over. Parameters trained on the device and not yet
        copied back (``sync_to_host``) are replaced by the host values."""
        self._invalidate_device()
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
        """All-position logits (batch, seq, vocab) on the device (models/gpt.py:92-121).

        With gradients wanted (grad mode on and a parameter requiring them) the logits carry
        the backward of the whole forward: ``logits.backward(dlogits)`` recomputes the
        forward keeping its activations (the recompute of gradient checkpointing,
        transformer_fused.py:69-73) and adds every parameter's gradient
        (``nml_model_logits_backward``)."""
        ids = _ids_array(input_ids)
        self._check_ids(ids)
        h = self._device_model()
        b, s = ids.shape
        out = self._logits_array((b, s, self.vocab_size))
        dids = N.DeviceArray.from_host(ids)
        N.check(N.lib.nml_model_forward(h, dids.ptr, b, s, out.ptr, 0))
        params = self.parameters()
        needs = is_grad_enabled() and any(p.requires_grad for p in params)
        logits = Tensor(out, (b, s, self.vocab_size), requires_grad=needs)
        if needs:
            dev = self._dev

            def _backward():
                if logits.grad is None:
                    return
                if self._dev is not dev:
                    raise RuntimeError("parameters were re-uploaded since these logits were "
                                       "computed; run the forward again")
                g = np.ascontiguousarray(np.asarray(logits.grad).reshape(logits.shape),
                                         dtype=self._dtype)
                dg = N.DeviceArray.from_host(g)
                N.check(N.lib.nml_model_zero_grad(h))
                N.check(N.lib.nml_model_logits_backward(h, dids.ptr, b, s, dg.ptr))
                self._pull_grads()

            logits._backward = _backward
        return logits

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
        longest = int(cache.lengths.max()) if cache.lengths is not None else cache.length
        if longest + s > self.max_seq_len:
            raise ValueError(f"Sequence length {longest + s} exceeds maximum sequence "
                             f"length {self.max_seq_len}")
        out = self._logits_array((b, s, self.vocab_size))
        dids = N.DeviceArray.from_host(ids)
        N.check(N.lib.nml_model_forward_cached(h, cache._h, dids.ptr, b, s, out.ptr, 0))
        if cache.lengths is not None:
            cache.lengths = cache.lengths + s
        return Tensor(out, (b, s, self.vocab_size)), cache

    def prefill_ragged(self, rows):
        """Prefill a new KV cache with rows of different lengths (a list of 1-D id arrays)
        in one packed pass, as ``generate`` does for a ragged batch; returns each row's
        last-position logits (batch, vocab) and the cache. Each row continues at its own
        position: ``forward_with_cache(ids (batch, 1), cache)`` then runs one step of the
        batched decode loop. (The reference runs such rows one at a time,
        models/generate.py:80-89.)"""
        rows = [np.asarray(r, dtype=np.int64).reshape(-1) for r in rows]
        if not rows or any(r.size == 0 for r in rows):
            raise ValueError("prompts must not be empty")
        for r in rows:
            if int(r.min()) < 0 or int(r.max()) >= self.vocab_size:
                raise ValueError(f"Token ID out of range [0, {self.vocab_size})")
            if r.size > self.max_seq_len:
                raise ValueError(f"Sequence length {r.size} exceeds maximum sequence length "
                                 f"{self.max_seq_len}")
        b = len(rows)
        plen = np.asarray([r.size for r in rows], dtype=np.int32)
        stride = int(plen.max())
        prompts = np.zeros((b, stride), dtype=np.int64)
        for i, r in enumerate(rows):
            prompts[i, :r.size] = r
        h = self._device_model()
        cache = KVCache(self, b)
        out = self._logits_array((b, self.vocab_size))
        dp = N.DeviceArray.from_host(prompts)
        N.check(N.lib.nml_model_prefill_ragged(h, cache._h, dp.ptr, stride,
                                               plen.ctypes.data_as(N.PI32), b, out.ptr))
        cache.lengths = plen.astype(np.int64)
        return Tensor(out, (b, self.vocab_size)), cache

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
        out = np.empty(shape, dtype=np.float32)
        N.check(N.lib.nml_memcpy_d2h(out.ctypes.data, self._ptr(N.lib.nml_model_grad_ptr, kind,
                                                                 layer), out.nbytes))
        return out

    def _pull_grads(self):
        """Add the device gradients of one backward to the parameters' ``grad``, in the
        reference layouts ((in, out) weights, Q/K/V split)."""
        params = [t for t, *_ in self._param_layout()]
        fresh = all(p.grad is None for p in params)
        g = self._read_device(lambda k, l: self._ptr(N.lib.nml_model_grad_ptr, k, l), np.float32)
        for p in params:
            p._accumulate_grad(g[id(p)])
        # the arena equals the host gradients when each was empty before and is float32
        self._arena_grads = (self._dev, {id(p): p.grad for p in params}) if fresh and all(
            p.grad.dtype == np.float32 for p in params) else None

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
        self.adam = False  # AdamW state allocated on the device
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
