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

Every module's ``forward`` runs on the GPU and returns a Tensor over a ``DeviceArray``:
  Dense.forward               layers/dense.py:27-70        x·W + b (nml_linear_device)
  Embedding.forward / _prefix layers/embedding.py:23-118   gather (nml_embedding_gather_device)
  RMSNorm.forward             layers/rms_norm.py:25-95     (nml_rmsnorm_forward_device)
  FeedForward.forward         neural_network/feed_forward.py   two GEMMs, GELU fused
  MultiHeadAttention.forward  neural_network/attention.py:139-168  (nml_model_mha_forward)
  FusedTransformerBlock.forward  neural_network/transformer_fused.py:44-95
  FusedGPTTrunk.forward          transformer_fused.py:103-144 (nml_model_blocks_forward)
  Sequential.forward          neural_network/module.py:54-65
Each module keeps a device copy of its parameters (a device model for the block, trunk
and attention modules; transposed weights for Dense and FeedForward), keyed on the
parameters' versions: ``load``/``load_arrays`` and ``GPT.sync_to_host`` bump them, and
code that edits ``param.data`` in place by other means calls
``module.mark_parameters_changed()``. A second call with unchanged parameters uploads
nothing. Masks follow
the reference: an additive (seq, seq) array or Tensor; ``None`` is causal for the
fused block and trunk and no mask for MultiHeadAttention.

Autograd: with gradients wanted (``is_grad_enabled()`` and the input or a parameter
requiring them), each output carries the closure its reference module attaches, run on
the device by ``Tensor.backward`` in reverse topological order:
  Dense                 layers/dense.py:81-94          nml_linear_backward_device
  Embedding / _prefix   layers/embedding.py:63-69, :111-117  nml_embedding_backward_device
  RMSNorm               layers/rms_norm.py:76-94       nml_rmsnorm_backward_typed_device
  FeedForward           neural_network/feed_forward.py:105-129  two linear backwards, the
                        GELU derivative fused into the second
  MultiHeadAttention    neural_network/attention.py:103-119 (its SDPA) with the projections
                        nml_model_mha_forward_train / nml_model_mha_backward
  FusedTransformerBlock transformer_fused.py:65-78     nml_model_blocks_forward_train /
  FusedGPTTrunk         transformer_fused.py:128-136   nml_model_blocks_backward
Parameter gradients are added to each parameter's ``grad`` (Tensor._accumulate_grad) in the
reference layouts; the input's gradient goes to the input Tensor. The device models keep
one saved forward each: a backward whose forward was replaced by a later saving forward
of the same module recomputes it from the kept input first (the reference's
``gradient_checkpointing`` recompute, transformer_fused.py:69-73), so any number of
outstanding graphs give the same gradients.
"""
from __future__ import annotations

import contextlib
import ctypes as C
from math import prod, sqrt

import numpy as np

from nimbleml_amd import _native as N
from nimbleml_amd import np_backend
from nimbleml_amd.grad_mode import is_grad_enabled
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

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def mark_parameters_changed(self):
        """Declare that parameter values were edited in place: the device copies are
        rebuilt at the next call (load/load_arrays do this themselves)."""
        for p in self.parameters():
            p._bump_version()


# ------------------------------------------------------------------ resident copies
def _params_key(params, dt, *extra):
    """What a device copy depends on: each parameter's identity, version and buffer."""
    def buf(p):
        return p.data.ctypes.data if isinstance(p.data, np.ndarray) else id(p.data)

    return (np.dtype(dt).str, extra, tuple((id(p), p._version, buf(p)) for p in params))


def _resident(module, name, key, build):
    """The device copy ``name`` of ``module`` for ``key``, built when the key changed. The
    previous copy is dropped from the module; it is freed when nothing else holds it (an
    output's autograd closure keeps the copy its forward ran on until its backward)."""
    cache = module.__dict__.setdefault("_device_copies", {})
    hit = cache.get(name)
    if hit is not None and hit[0] == key:
        return hit[1]
    cache.pop(name, None)
    value = build()
    cache[name] = (key, value)
    return value


def _seq_capacity(s):
    """Positions a cached device model is built for: at least 64, a power of two ≥ s."""
    p = 64
    while p < s:
        p *= 2
    return p


# ------------------------------------------------------------------ device plumbing
def _compute_dtype():
    return np.dtype(np_backend.dtype)


def _device_input(x, dt):
    """``x`` (Tensor, DeviceArray or array) as a DeviceArray of its own shape in ``dt``."""
    data, shape = (x.data, x.shape) if isinstance(x, Tensor) else (x, np.shape(x))
    if isinstance(data, N.DeviceArray):
        if data.dtype != dt:
            raise TypeError(f"expected a {dt} input, got {data.dtype}")
        return data.reshape(shape)
    return N.DeviceArray.from_host(np.asarray(data, dtype=dt).reshape(shape))


def _host(t, shape, dt):
    return np.ascontiguousarray(np.asarray(t.data, dtype=dt).reshape(shape))


def _needs_grad(x, params):
    return is_grad_enabled() and (getattr(x, "requires_grad", False)
                                  or any(p.requires_grad for p in params))


def _output(arr, shape, x, params, op, backward=None):
    """The module's result Tensor. With gradients wanted, ``backward(out)`` becomes its
    autograd closure and the input Tensor ``x`` its child (the edge Tensor.backward
    walks)."""
    needs = _needs_grad(x, params)
    kids = (x,) if needs and isinstance(x, Tensor) else ()
    out = Tensor(arr, shape, requires_grad=needs, _children=kids, _op=op)
    if needs and backward is not None:
        out._backward = lambda: backward(out)
    return out


# ------------------------------------------------------------------ backward helpers
def _dy(out, dt):
    """``out.grad`` on the device in the compute dtype and out's shape (None when unset)."""
    if out.grad is None:
        return None
    g = np.asarray(out.grad).reshape(out.shape)
    return N.DeviceArray.from_host(np.ascontiguousarray(g, dtype=dt))


def _f32_zeros(shape, wanted):
    """A zeroed float32 device gradient buffer, or None when not wanted."""
    return N.DeviceArray.from_host(np.zeros(shape, np.float32)) if wanted else None


def _wants(t):
    return isinstance(t, Tensor) and t.requires_grad


def _to_input(x, dx):
    """Hand the input gradient (a DeviceArray) to the input Tensor."""
    if dx is not None and _wants(x):
        x._accumulate_grad(dx.numpy().reshape(-1))


def _model_grad(model, kind, layer, shape):
    """The float32 gradient of a device model's parameter (kind, layer) on the host."""
    p = C.c_void_p()
    N.check(N.lib.nml_model_grad_ptr(model.handle, kind, layer, C.byref(p)))
    out = np.empty(shape, np.float32)
    N.check(N.lib.nml_memcpy_d2h(out.ctypes.data, p.value, out.nbytes))
    return out


def _saved_generation(model):
    g = C.c_ulonglong()
    N.check(N.lib.nml_model_saved_generation(model.handle, C.byref(g)))
    return int(g.value)


def _saved_forward(model, state, rerun):
    """Make the device model's saved activations those of this output's forward:
    ``state[0]`` is the generation it saved; a later saving forward replaced it, so run
    ``rerun`` (the same forward on the kept input) again."""
    if model.handle is None:
        raise RuntimeError("the device model of this output's forward was closed; run the "
                           "forward again before backward()")
    if _saved_generation(model) != state[0]:
        rerun()
        state[0] = _saved_generation(model)


def _add_dense_grads(dense, w_t_grad, b_grad):
    """Device-layout (out, in) weight gradient and bias gradient into a Dense's ``grad``."""
    if w_t_grad is not None:
        dense.weights._accumulate_grad(np.ascontiguousarray(w_t_grad.T))
    if b_grad is not None and dense.biases is not None:
        dense.biases._accumulate_grad(b_grad)


def _mha_grads(model, mha, layer):
    d = mha.d_model
    wqkv = _model_grad(model, N.P_WQKV, layer, (3 * d, d))
    bqkv = _model_grad(model, N.P_BQKV, layer, (3 * d,))
    for j, dense in enumerate((mha.W_q, mha.W_k, mha.W_v)):
        _add_dense_grads(dense, wqkv[j * d:(j + 1) * d], bqkv[j * d:(j + 1) * d])
    _add_dense_grads(mha.W_o, _model_grad(model, N.P_WO, layer, (d, d)),
                     _model_grad(model, N.P_BO, layer, (d,)))


def _block_grads(model, blk, layer):
    d = blk.d_model
    f1, f2 = blk.ffn.dense1, blk.ffn.dense2
    blk.ln1.gamma._accumulate_grad(_model_grad(model, N.P_LN1, layer, (d,)))
    _mha_grads(model, blk.mha, layer)
    blk.ln2.gamma._accumulate_grad(_model_grad(model, N.P_LN2, layer, (d,)))
    _add_dense_grads(f1, _model_grad(model, N.P_W1, layer, (f1.out_features, d)),
                     _model_grad(model, N.P_B1, layer, (f1.out_features,)))
    _add_dense_grads(f2, _model_grad(model, N.P_W2, layer, (d, f2.in_features)),
                     _model_grad(model, N.P_B2, layer, (d,)))


def _mask_mode(mask, seq, dt, *, none_is_causal):
    """``(causal, DeviceArray | None)`` for a mask argument: a mask equal to the causal
    mask (utils/mask.py:8-13: −inf above the diagonal, 0 elsewhere) takes the causal
    kernels; any other (seq, seq) mask is added to the scores as given."""
    if mask is None:
        return (1, None) if none_is_causal else (0, None)
    arr = np.asarray(mask.data if isinstance(mask, Tensor) else mask)
    if isinstance(mask, Tensor):
        arr = arr.reshape(mask.shape)
    if arr.shape != (seq, seq):
        raise ValueError(f"mask must be ({seq}, {seq}), got {arr.shape}")
    arr = np.ascontiguousarray(arr.astype(dt, copy=False))
    if np.array_equal(arr, np.triu(np.full((seq, seq), -np.inf, dtype=dt), k=1)):
        return 1, None
    return 0, N.DeviceArray.from_host(arr)


def _dense_bias(dense, dt):
    if dense.biases is None:
        return np.zeros(dense.out_features, dtype=dt)
    return _host(dense.biases, (dense.out_features,), dt)


def mha_device_arrays(mha, layer, dt):
    """(kind, layer, array) of one attention module in the device layout: W_q | W_k | W_v
    stacked and transposed to (3d, d), W_o transposed to (d, d)."""
    d = mha.d_model
    w = [_host(x.weights, (d, d), dt) for x in (mha.W_q, mha.W_k, mha.W_v)]
    b = [_dense_bias(x, dt) for x in (mha.W_q, mha.W_k, mha.W_v)]
    return [(N.P_WQKV, layer, np.ascontiguousarray(np.concatenate(w, axis=1).T)),
            (N.P_BQKV, layer, np.concatenate(b)),
            (N.P_WO, layer, np.ascontiguousarray(_host(mha.W_o.weights, (d, d), dt).T)),
            (N.P_BO, layer, _dense_bias(mha.W_o, dt))]


def block_device_arrays(blk, layer, dt):
    """(kind, layer, array) of one FusedTransformerBlock in the device layout."""
    d = blk.d_model
    f1, f2 = blk.ffn.dense1, blk.ffn.dense2
    return ([(N.P_LN1, layer, _host(blk.ln1.gamma, (d,), dt))]
            + mha_device_arrays(blk.mha, layer, dt)
            + [(N.P_LN2, layer, _host(blk.ln2.gamma, (d,), dt)),
               (N.P_W1, layer, np.ascontiguousarray(_host(f1.weights, (d, f1.out_features),
                                                          dt).T)),
               (N.P_B1, layer, _dense_bias(f1, dt)),
               (N.P_W2, layer, np.ascontiguousarray(_host(f2.weights, (f2.in_features, d),
                                                          dt).T)),
               (N.P_B2, layer, _dense_bias(f2, dt))])


def rope_device_arrays(rope_cache, head_dim, dt):
    """The first half of each RoPE table row in the compute dtype, as apply_rope_flat casts
    it (utils/rope.py:36-38)."""
    cos, sin = rope_cache
    half = head_dim // 2
    return [(N.P_ROPE_COS, 0, np.ascontiguousarray(np.asarray(cos)[:, :half].astype(dt))),
            (N.P_ROPE_SIN, 0, np.ascontiguousarray(np.asarray(sin)[:, :half].astype(dt)))]


class _CallModel:
    """A device model of a module's parameters: only the arrays given are uploaded (the
    token and position tables stay unused); kept by the module while its parameters are
    unchanged, freed with the object."""

    def __init__(self, d_model, num_heads, num_layers, max_seq_len, d_ff, dt, arrays):
        N.ensure_init()
        h = C.c_void_p()
        N.check(N.lib.nml_model_create(1, d_model, num_heads, num_layers, max_seq_len, d_ff,
                                       N.np_dtype_code(dt), C.byref(h)))
        self.handle = h
        self.max_seq_len = max_seq_len
        try:
            for kind, layer, arr in arrays:
                N.check(N.lib.nml_model_set_param(h, kind, layer, arr.ctypes.data, arr.nbytes))
                N.count_h2d(arr.nbytes)
        except Exception:
            self.close()
            raise

    def close(self):
        if self.handle:
            N.lib.nml_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _blocks_forward(owner, blocks, ln, x, mask, op, params):
    """FusedTransformerBlock / FusedGPTTrunk forward over a (batch, seq, d) input, on the
    device model ``owner`` keeps of its parameters."""
    blocks = list(blocks)
    if len(x.shape) != 3:
        raise ValueError(f"expected (batch, seq, d_model), got {x.shape}")
    b, s, d = x.shape
    blk0 = blocks[0]
    if d != blk0.d_model:
        raise ValueError(f"Expected d_model {blk0.d_model}, got {d}")
    dt = _compute_dtype()
    causal, mdev = _mask_mode(mask, s, dt, none_is_causal=True)
    dk = d // blk0.num_heads
    rope = blk0.mha._rope_cache
    if rope is not None:  # _fused_arrays.py:95-98: positions 0..seq-1 of the block's table
        p = int(np.asarray(rope[0]).shape[0])
        if s > p:
            raise ValueError(f"Sequence length {s} exceeds the RoPE table ({p} positions)")
    else:
        p = _seq_capacity(s)
        hit = owner.__dict__.get("_device_copies", {}).get("blocks")
        if hit is not None and hit[1].max_seq_len >= s:
            p = hit[1].max_seq_len  # the cached model covers this length
    rope_key = (id(rope[0]), id(rope[1])) if rope is not None else None

    def build():
        arrays = []
        for i, blk in enumerate(blocks):
            arrays += block_device_arrays(blk, i, dt)
        arrays.append((N.P_LN_F, 0, _host(ln.gamma, (d,), dt) if ln is not None
                       else np.ones(d, dtype=dt)))
        if rope is not None:
            arrays += rope_device_arrays(rope, dk, dt)
        return _CallModel(d, blk0.num_heads, len(blocks), p, blk0.ffn.dense1.out_features, dt,
                          arrays)

    model = _resident(owner, "blocks", _params_key(params, dt, p, rope_key), build)
    xd = _device_input(x, dt)
    out = N.DeviceArray((b, s, d), dt)
    args = (b, s, int(ln is not None), causal, N.ptr(mdev))
    if not _needs_grad(x, params):
        N.check(N.lib.nml_model_blocks_forward(model.handle, xd.ptr, out.ptr, *args))
        N.check(N.lib.nml_synchronize())
        return _output(out, (b, s, d), x, params, op)
    N.check(N.lib.nml_model_blocks_forward_train(model.handle, xd.ptr, out.ptr, *args))
    N.check(N.lib.nml_synchronize())
    state = [_saved_generation(model)]

    def rerun():  # the mask's device copy is referenced here, so it outlives the forward
        tmp = N.DeviceArray((b, s, d), dt)
        N.check(N.lib.nml_model_blocks_forward_train(model.handle, xd.ptr, tmp.ptr, b, s,
                                                     int(ln is not None), causal, N.ptr(mdev)))

    def backward(o):
        dy = _dy(o, dt)
        if dy is None:
            return
        _saved_forward(model, state, rerun)
        N.check(N.lib.nml_model_zero_grad(model.handle))
        dx = N.DeviceArray((b, s, d), dt) if _wants(x) else None
        N.check(N.lib.nml_model_blocks_backward(model.handle, dy.ptr, N.ptr(dx)))
        for i, blk in enumerate(blocks):
            _block_grads(model, blk, i)
        if ln is not None:
            ln.gamma._accumulate_grad(_model_grad(model, N.P_LN_F, 0, (d,)))
        _to_input(x, dx)

    return _output(out, (b, s, d), x, params, op, backward)


class Sequential(Module):
    def __init__(self, *layers):
        self.layers = list(layers)

    def __iter__(self):
        return iter(self.layers)

    def forward(self, data):
        """neural_network/module.py:54-65: each layer in order."""
        for layer in self.layers:
            data = layer(data)
        return data

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

    def forward(self, inputs):
        """layers/dense.py:27-70: ``x·W + b`` over the last dimension."""
        if inputs.shape[-1] != self.in_features:
            raise ValueError(f"Expected last dim {self.in_features}, got {inputs.shape[-1]}")
        from nimbleml_amd import kernels as K

        dt = _compute_dtype()
        shape = (*inputs.shape[:-1], self.out_features)
        x = _device_input(inputs, dt)
        w_t, b = self._device_weights(dt)
        out = K.linear_t(x, w_t, b)
        rows = prod(shape[:-1])

        def backward(o):  # layers/dense.py:81-94
            dy = _dy(o, dt)
            if dy is None:
                return
            dx = N.DeviceArray((rows, self.in_features), dt) if _wants(inputs) else None
            dw = _f32_zeros((self.out_features, self.in_features), self.weights.requires_grad)
            db = _f32_zeros((self.out_features,), _wants(self.biases))
            N.check(N.lib.nml_linear_backward_device(
                dy.ptr, x.ptr, w_t.ptr, N.ptr(dx), N.ptr(dw), N.ptr(db), rows, self.in_features,
                self.out_features, None, N.np_dtype_code(dt)))
            _add_dense_grads(self, None if dw is None else dw.numpy(),
                             None if db is None else db.numpy())
            _to_input(inputs, dx)

        return _output(out.reshape(shape), shape, inputs, self.parameters(), "dense", backward)

    def _device_weights(self, dt):
        """(W transposed to (out, in), bias or None) on the device, kept while unchanged."""
        def build():
            w = np.ascontiguousarray(_host(self.weights, (self.in_features, self.out_features),
                                           dt).T)
            b = None if self.biases is None else _host(self.biases, (self.out_features,), dt)
            return (N.DeviceArray.from_host(w),
                    None if b is None else N.DeviceArray.from_host(b))

        return _resident(self, "linear", _params_key(self.parameters(), dt), build)

    def parameters(self):
        return [self.weights] + ([self.biases] if self.biases is not None else [])


class Embedding(Module):
    def __init__(self, vocab_size, embed_dim, init_std: float = 0.02):
        self.vocab_size = vocab_size
        self.embed_dim = embed_dim
        self.weights = _param(_init(lambda: np.random.standard_normal((vocab_size, embed_dim))
                                    * init_std, (vocab_size, embed_dim)),
                              (vocab_size, embed_dim))

    def forward(self, inputs):
        """layers/embedding.py:23-70: rows of the table for integer ids of any shape."""
        from nimbleml_amd import kernels as K

        if isinstance(inputs, Tensor):
            ids = np.asarray(inputs.data, dtype=np.int64).reshape(inputs.shape)
        else:
            ids = np.asarray(inputs, dtype=np.int64)
        dt = _compute_dtype()
        w = self._device_table(dt)
        shape = (*ids.shape, self.embed_dim)
        if ids.size == 0:
            return _output(N.DeviceArray(shape, dt), shape, None, self.parameters(), "embedding")
        out = K.embedding_lookup(w, ids)

        def backward(o):  # layers/embedding.py:63-69: scatter-add into the rows used
            dy = _dy(o, dt)
            if dy is None or not self.weights.requires_grad:
                return
            gw = _f32_zeros((self.vocab_size, self.embed_dim), True)
            idd = N.DeviceArray.from_host(ids.reshape(-1))
            N.check(N.lib.nml_embedding_backward_device(dy.ptr, idd.ptr, gw.ptr, ids.size,
                                                        self.embed_dim, self.vocab_size,
                                                        N.np_dtype_code(dt)))
            self.weights._accumulate_grad(gw.numpy())

        return _output(out.reshape(shape), shape, None, self.parameters(), "embedding", backward)

    def forward_prefix(self, seq_len: int):
        """layers/embedding.py:72-118: rows ``[0, seq_len)`` of the table, (seq_len, dim)."""
        if seq_len < 0 or seq_len > self.vocab_size:
            raise ValueError(f"seq_len must be in [0, {self.vocab_size}), got {seq_len}.")
        dt = _compute_dtype()
        table = self._device_table(dt)
        shape = (seq_len, self.embed_dim)
        rows = N.DeviceArray(shape, dt)
        if rows.nbytes:
            N.check(N.lib.nml_memcpy_d2d(rows.ptr, table.ptr, rows.nbytes))

        def backward(o):  # layers/embedding.py:111-117: rows [0, seq_len) take the gradient
            if o.grad is None or not self.weights.requires_grad:
                return
            g = np.zeros((self.vocab_size, self.embed_dim), np.float32)
            g[:seq_len] = np.asarray(o.grad, dtype=np.float32).reshape(shape)
            self.weights._accumulate_grad(g)

        return _output(rows, shape, None, self.parameters(), "embedding_prefix", backward)

    def _device_table(self, dt):
        return _resident(self, "table", _params_key(self.parameters(), dt),
                         lambda: N.DeviceArray.from_host(
                             _host(self.weights, (self.vocab_size, self.embed_dim), dt)))

    def parameters(self):
        return [self.weights]


class RMSNorm(Module):
    def __init__(self, normalized_shape, epsilon=1e-5):
        self.normalized_shape = normalized_shape
        self.epsilon = epsilon
        self.gamma = _param(np.ones(normalized_shape), (normalized_shape,))

    def forward(self, inputs):
        """layers/rms_norm.py:25-95: ``gamma · x / sqrt(mean(x²) + eps)`` over the last dim."""
        if inputs.shape[-1] != self.normalized_shape:
            raise ValueError(f"Expected last dim {self.normalized_shape}, got {inputs.shape[-1]}")
        from nimbleml_amd import kernels as K

        dt = _compute_dtype()
        d = self.normalized_shape
        rows = prod(inputs.shape[:-1]) if len(inputs.shape) > 1 else 1
        x = _device_input(inputs, dt).reshape(rows, d)
        g = _resident(self, "gamma", _params_key(self.parameters(), dt),
                      lambda: N.DeviceArray.from_host(_host(self.gamma, (d,), dt)))
        out = K.fused_rmsnorm_forward(x, g, self.epsilon)[0]

        def backward(o):  # layers/rms_norm.py:76-94
            dy = _dy(o, dt)
            if dy is None:
                return
            dx = N.DeviceArray((rows, d), dt)
            dg = _f32_zeros((d,), True)
            N.check(N.lib.nml_rmsnorm_backward_typed_device(dy.ptr, x.ptr, g.ptr, dx.ptr, dg.ptr,
                                                            rows, d, float(self.epsilon),
                                                            N.np_dtype_code(dt)))
            self.gamma._accumulate_grad(dg.numpy())
            _to_input(inputs, dx)

        return _output(out.reshape(inputs.shape), inputs.shape, inputs, self.parameters(),
                       "rms_norm", backward)

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

    def forward(self, x, mask=None):
        """neural_network/attention.py:139-168: per-head softmax(q·kᵀ / sqrt(d_k) + mask)·v
        of x's projections, heads merged, then W_o. ``mask=None`` attends to every key;
        the RoPE cache is not applied here (the reference applies it in the fused block)."""
        if len(x.shape) != 3:
            raise ValueError(f"expected (batch, seq, d_model), got {x.shape}")
        b, s, d = x.shape
        if d != self.d_model:
            raise ValueError(f"Expected d_model {self.d_model}, got {d}")
        dt = _compute_dtype()
        causal, mdev = _mask_mode(mask, s, dt, none_is_causal=False)
        vec = 8 if dt == np.float16 else 4
        p = _seq_capacity(s)
        hit = self.__dict__.get("_device_copies", {}).get("mha")
        if hit is not None and hit[1].max_seq_len >= s:
            p = hit[1].max_seq_len
        model = _resident(self, "mha", _params_key(self.parameters(), dt, p),
                          lambda: _CallModel(d, self.num_heads, 1, p, vec, dt,
                                             mha_device_arrays(self, 0, dt)))
        xd = _device_input(x, dt)
        out = N.DeviceArray((b, s, d), dt)
        params = self.parameters()
        if not _needs_grad(x, params):
            N.check(N.lib.nml_model_mha_forward(model.handle, 0, xd.ptr, out.ptr, b, s, causal,
                                                N.ptr(mdev)))
            N.check(N.lib.nml_synchronize())
            return _output(out, (b, s, d), x, params, "multi_head_attention")
        N.check(N.lib.nml_model_mha_forward_train(model.handle, 0, xd.ptr, out.ptr, b, s, causal,
                                                  N.ptr(mdev)))
        N.check(N.lib.nml_synchronize())
        state = [_saved_generation(model)]

        def rerun():
            tmp = N.DeviceArray((b, s, d), dt)
            N.check(N.lib.nml_model_mha_forward_train(model.handle, 0, xd.ptr, tmp.ptr, b, s,
                                                      causal, N.ptr(mdev)))

        def backward(o):  # the projections' closures around attention.py:103-119
            dy = _dy(o, dt)
            if dy is None:
                return
            _saved_forward(model, state, rerun)
            N.check(N.lib.nml_model_zero_grad(model.handle))
            dx = N.DeviceArray((b, s, d), dt) if _wants(x) else None
            N.check(N.lib.nml_model_mha_backward(model.handle, dy.ptr, N.ptr(dx)))
            _mha_grads(model, self, 0)
            _to_input(x, dx)

        return _output(out, (b, s, d), x, params, "multi_head_attention", backward)

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

    def forward(self, x):
        """neural_network/feed_forward.py: ``GELU(x·W₁ + b₁)·W₂ + b₂`` per token, the GELU
        fused into the first GEMM's epilogue."""
        from nimbleml_amd import kernels as K

        w1, w2 = self.dense1, self.dense2
        if x.shape[-1] != w1.in_features:
            raise ValueError(f"Expected last dim {w1.in_features}, got {x.shape[-1]}")
        if w1.out_features != w2.in_features:
            raise ValueError(f"Dense1 out ({w1.out_features}) must match Dense2 in "
                             f"({w2.in_features})")
        if w2.out_features != x.shape[-1]:
            raise ValueError(f"Expected output last dim {x.shape[-1]}, got {w2.out_features}")
        dt = _compute_dtype()
        xd = _device_input(x, dt)
        w1_t, b1 = w1._device_weights(dt)
        w2_t, b2 = w2._device_weights(dt)
        zero = None
        if b1 is None or b2 is None:  # the GELU epilogue takes a bias: zeros for none
            n = max(w1.out_features, w2.out_features)
            zero = _resident(self, "zero_bias", (np.dtype(dt).str, n),
                             lambda: N.DeviceArray.from_host(np.zeros(n, dtype=dt)))
        b1d = b1 if b1 is not None else zero
        b2d = b2 if b2 is not None else zero
        params = self.parameters()
        if not _needs_grad(x, params):
            h = K.linear_t(xd, w1_t, b1d, epilogue=K.EPI_BIAS_GELU)
            out = K.linear_t(h, w2_t, b2d, epilogue=K.EPI_BIAS)
            return _output(out.reshape(x.shape), x.shape, x, params, "feed_forward")
        # the backward reads the pre-activation: the GELU runs as its own kernel
        pre = K.linear_t(xd, w1_t, b1d, epilogue=K.EPI_BIAS)
        h = K.fused_gelu_forward(pre)[0]
        out = K.linear_t(h, w2_t, b2d, epilogue=K.EPI_BIAS)
        rows, hid = pre.shape
        d = w1.in_features

        def backward(o):  # neural_network/feed_forward.py:105-129
            dy = _dy(o, dt)
            if dy is None:
                return
            code = N.np_dtype_code(dt)
            dpre = N.DeviceArray((rows, hid), dt)
            dw2 = _f32_zeros((d, hid), w2.weights.requires_grad)
            db2 = _f32_zeros((d,), _wants(w2.biases))
            N.check(N.lib.nml_linear_backward_device(dy.ptr, h.ptr, w2_t.ptr, dpre.ptr,
                                                     N.ptr(dw2), N.ptr(db2), rows, hid, d,
                                                     pre.ptr, code))
            dx = N.DeviceArray((rows, d), dt) if _wants(x) else None
            dw1 = _f32_zeros((hid, d), w1.weights.requires_grad)
            db1 = _f32_zeros((hid,), _wants(w1.biases))
            N.check(N.lib.nml_linear_backward_device(dpre.ptr, xd.ptr, w1_t.ptr, N.ptr(dx),
                                                     N.ptr(dw1), N.ptr(db1), rows, d, hid, None,
                                                     code))
            _add_dense_grads(w2, None if dw2 is None else dw2.numpy(),
                             None if db2 is None else db2.numpy())
            _add_dense_grads(w1, None if dw1 is None else dw1.numpy(),
                             None if db1 is None else db1.numpy())
            _to_input(x, dx)

        return _output(out.reshape(x.shape), x.shape, x, params, "feed_forward", backward)

    def parameters(self):
        return self.dense1.parameters() + self.dense2.parameters()


class FusedTransformerBlock(Module):
    """Pre-norm block (x + MHA(LN1(x)); x + FFN(LN2(x)))."""

    def __init__(self, d_model, num_heads, ff_mult=4, *, gradient_checkpointing: bool = False):
        self.d_model = d_model
        self.num_heads = num_heads
        self.gradient_checkpointing = bool(gradient_checkpointing)
        self.ln1 = RMSNorm(d_model)
        self.mha = MultiHeadAttention(d_model, num_heads)
        self.ln2 = RMSNorm(d_model)
        self.ffn = FeedForward(d_model, ff_mult=ff_mult)

    def forward(self, x, mask=None):
        """neural_network/transformer_fused.py:44-95 → fused_block_forward_arrays
        (_fused_arrays.py:251-284); ``mask=None`` is causal."""
        return _blocks_forward(self, [self], None, x, mask, "fused_transformer_block",
                               self.parameters())

    def parameters(self):
        params = []
        for layer in (self.ln1, self.mha, self.ln2, self.ffn):
            params.extend(layer.parameters())
        return params


class TransformerBlock(FusedTransformerBlock):
    """The unfused pre-norm block of ``GPT(fused_blocks=False)``
    (neural_network/transformer.py:9-55): the same parameters (ln1, mha, ln2, ffn) and the
    same function, x + MHA(RMSNorm₁(x)) then + FFN(RMSNorm₂(·)), causal when mask is None.
    The reference builds it from Tensor-level ops; here it runs the fused block's device
    path, forward and backward."""

    def __init__(self, d_model, num_heads, ff_mult=4):
        super().__init__(d_model, num_heads, ff_mult)

    def forward(self, x, mask=None):
        """transformer.py:19-48."""
        return _blocks_forward(self, [self], None, x, mask, "transformer_block",
                               self.parameters())


class FusedGPTTrunk(Module):
    """All blocks plus the final RMSNorm as one module (transformer_fused.py:103-144)."""

    def __init__(self, blocks, ln: RMSNorm):
        self.blocks = list(blocks)
        self.ln = ln

    def forward(self, x, mask=None):
        """transformer_fused.py:103-144: every block, then the final RMSNorm."""
        return _blocks_forward(self, self.blocks, self.ln, x, mask, "fused_gpt_trunk",
                               self.parameters())

    def parameters(self):
        params = []
        for block in self.blocks:
            params.extend(block.parameters())
        params.extend(self.ln.parameters())
        return params
