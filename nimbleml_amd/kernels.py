"""Array-level device ops under the reference kernel names (NimbleML/kernels/).

Each takes host arrays or ``DeviceArray``s in the compute dtype and returns
``DeviceArray`` results computed by the HIP kernels:
  fused_rmsnorm_forward       kernels/fused_rmsnorm.py:130-162
  fused_gelu_forward          kernels/fused_gelu.py:57-83
  fused_sdpa_forward          kernels/fused_sdpa.py:256-289 (any additive mask, or none)
  decode_attention            one cached decode step of that attention (the KV-cache seam of
                              models/generate.py:93-100; no reference kernel)
  embedding_lookup            kernels/embedding_scatter.py:25-36
  fused_tied_crossentropy_forward  kernels/fused_tied_crossentropy.py:8-24 (loss only)
  linear                      the `x @ W + b` of neural_network/_fused_arrays.py:25-30
  sample_tokens               models/generate.py:23-59 on a (batch, vocab) logits block
  adamw_step                  native adamw_step (native/src/adamw.cpp:6-20), in place
  clip_grad_norm              native clip_grad_norm (native/src/adamw.cpp:22-37), in place
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from nimbleml_amd import _native as N
from nimbleml_amd import np_backend

EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESID = 0, 1, 2, 3


def _dev(x, dtype=None):
    if isinstance(x, N.DeviceArray):
        if dtype is not None and x.dtype != np.dtype(dtype):
            raise TypeError(f"expected {np.dtype(dtype)}, got {x.dtype}")
        return x
    return N.DeviceArray.from_host(np.asarray(x, dtype=dtype if dtype is not None else None))


def _float_dtype(x):
    dt = np.dtype(x.dtype) if hasattr(x, "dtype") else np.dtype(np_backend.dtype)
    N.np_dtype_code(dt)
    return dt


def fused_rmsnorm_forward(x, gamma, epsilon=1e-5):
    """Returns (out, x, ms, rms) with ms/rms shaped (rows, 1) like the reference."""
    dt = _float_dtype(x)
    xd, gd = _dev(x, dt), _dev(gamma, dt)
    d = xd.shape[-1]
    rows = xd.size // d
    out = N.DeviceArray(xd.shape, dt)
    ms = N.DeviceArray((rows, 1), np.float32)
    rms = N.DeviceArray((rows, 1), np.float32)
    N.check(N.lib.nml_rmsnorm_forward_device(xd.ptr, gd.ptr, out.ptr, ms.ptr, rms.ptr, rows, d,
                                             float(epsilon), N.np_dtype_code(dt)))
    return out, xd, ms, rms


def fused_gelu_forward(x):
    """Returns (out, tanh_u) — tanh_u in float32 as in the reference."""
    dt = _float_dtype(x)
    xd = _dev(x, dt)
    out = N.DeviceArray(xd.shape, dt)
    tu = N.DeviceArray(xd.shape, np.float32)
    N.check(N.lib.nml_gelu_forward_device(xd.ptr, out.ptr, tu.ptr, xd.size, N.np_dtype_code(dt)))
    return out, tu


def fused_sdpa_forward(q, k, v, scale, mask_arr=None, *, batch=None, num_heads=None):
    """Attention over (bh, seq, dk) (kernels/fused_sdpa.py:256-289); ``scale`` is the
    sqrt(dk) divisor. ``mask_arr``: None attends to every key (the reference's
    ``_matmul_sdpa_forward`` without a mask); the causal mask (−inf above the diagonal)
    runs the causal kernels; any other additive (seq, seq) mask is added to the scaled
    scores. Returns ``(out, None)``: no probability matrix is formed."""
    dt = _float_dtype(q)
    qd, kd, vd = _dev(q, dt), _dev(k, dt), _dev(v, dt)
    bh, seq, dk = qd.shape
    causal, md = 0, None
    if mask_arr is not None:
        m = np.ascontiguousarray(np.asarray(mask_arr).astype(dt, copy=False))
        if m.shape != (seq, seq):
            raise ValueError(f"mask must be ({seq}, {seq}), got {m.shape}")
        if np.array_equal(m, np.triu(np.full((seq, seq), -np.inf, dtype=dt), k=1)):
            causal = 1
        else:
            md = N.DeviceArray.from_host(m)
    out = N.DeviceArray((bh, seq, dk), dt)
    N.check(N.lib.nml_sdpa_forward_device(qd.ptr, kd.ptr, vd.ptr, N.ptr(md), out.ptr, bh, seq, dk,
                                          float(scale), causal, N.np_dtype_code(dt)))
    return out, None


def flash_sdpa_forward(q, k, v, scale):
    """The reference's native flash path (kernels/fused_sdpa.py:91-115): float32 causal
    attention over (bh, seq, dk) with ``scale`` the sqrt(dk) divisor, returning
    ``(out, m, l)`` — m, l the per-row softmax max and sum from
    ``flash_sdpa_forward_device`` called with the multiplier ``1/scale``."""
    qd, kd, vd = _dev(q, np.float32), _dev(k, np.float32), _dev(v, np.float32)
    bh, seq, dk = qd.shape
    out = N.DeviceArray((bh, seq, dk), np.float32)
    m = N.DeviceArray((bh, seq), np.float32)
    lsum = N.DeviceArray((bh, seq), np.float32)
    N.check(N.lib.nml_flash_sdpa_forward_device(qd.ptr, kd.ptr, vd.ptr, out.ptr, m.ptr, lsum.ptr,
                                                bh, seq, dk, float(1.0 / scale)))
    return out, m, lsum


def decode_attention(q, kcache, vcache, lens, scale):
    """Attention of one new query per (row, head) over a KV cache: ``q`` (batch, heads, dk),
    ``kcache``/``vcache`` (batch, heads, max_seq, dk), ``lens`` (batch,) keys attended per
    row, ``scale`` the sqrt(dk) divisor (kernels/fused_sdpa.py:71-78 on the cached keys).
    Returns the merged-head output (batch, heads·dk). Raises ValueError for a length
    outside [1, max_seq]."""
    dt = _float_dtype(q)
    qd, kd, vd = _dev(q, dt), _dev(kcache, dt), _dev(vcache, dt)
    batch, heads, max_seq, dk = kd.shape
    if qd.shape != (batch, heads, dk) or vd.shape != kd.shape:
        raise ValueError(f"decode_attention: q {qd.shape}, kcache {kd.shape}, vcache {vd.shape}")
    ln = _dev(np.ascontiguousarray(lens, dtype=np.int32) if not isinstance(lens, N.DeviceArray)
              else lens, np.int32)
    if ln.shape != (batch,):
        raise ValueError(f"decode_attention: lens must be ({batch},), got {ln.shape}")
    err = N.DeviceArray.from_host(np.zeros(1, np.int32))
    out = N.DeviceArray((batch, heads * dk), dt)
    N.check(N.lib.nml_decode_attention_device(qd.ptr, kd.ptr, vd.ptr, ln.ptr, out.ptr, batch,
                                              heads, max_seq, dk, float(scale), err.ptr,
                                              N.np_dtype_code(dt)))
    if int(err.numpy()[0]):
        raise ValueError(f"decode_attention: a length is outside [1, {max_seq}]")
    return out


def flash_sdpa_backward(grad_out, q, k, v, m, lsum, scale):
    """``flash_sdpa_backward_device`` (kernels/fused_sdpa.py:118-140): float32 gradients
    (grad_q, grad_k, grad_v) of the causal flash forward, ``scale`` the sqrt(dk) divisor."""
    arrs = [_dev(a, np.float32) for a in (grad_out, q, k, v, m, lsum)]
    bh, seq, dk = arrs[1].shape
    gq, gk, gv = (N.DeviceArray((bh, seq, dk), np.float32) for _ in range(3))
    N.check(N.lib.nml_flash_sdpa_backward_device(*[a.ptr for a in arrs], gq.ptr, gk.ptr, gv.ptr,
                                                 bh, seq, dk, float(1.0 / scale)))
    return gq, gk, gv


def fused_rmsnorm_backward(grad, x, gamma, epsilon=1e-5):
    """``rmsnorm_backward_device`` (kernels/fused_rmsnorm.py:104-128 device branch, float32):
    returns (grad_x, grad_gamma)."""
    gd, xd, gmd = _dev(grad, np.float32), _dev(x, np.float32), _dev(gamma, np.float32)
    d = xd.shape[-1]
    rows = xd.size // d
    gx = N.DeviceArray(xd.shape, np.float32)
    gg = N.DeviceArray((d,), np.float32)
    N.check(N.lib.nml_rmsnorm_backward_device(gd.ptr, xd.ptr, gmd.ptr, None, None, gx.ptr, gg.ptr,
                                              rows, d, float(epsilon)))
    return gx, gg


def embedding_lookup(weights, ids, pos_weights=None):
    """``weights[ids]`` (plus ``pos_weights[s]`` when given) on the device."""
    dt = _float_dtype(weights)
    wd = _dev(weights, dt)
    ids_np = np.asarray(ids, dtype=np.int64)
    shape = ids_np.shape
    ids2 = ids_np.reshape(1, -1) if ids_np.ndim != 2 else ids_np
    vocab, dim = wd.shape
    if ids2.size and (int(ids2.min()) < 0 or int(ids2.max()) >= vocab):
        raise ValueError(f"Token ID out of range [0, {vocab})")
    b, s = ids2.shape
    if pos_weights is None:
        pd = N.DeviceArray((max(s, 1), dim), dt)
        N.check(N.lib.nml_memset(pd.ptr, 0, pd.nbytes))
    else:
        pd = _dev(pos_weights, dt)
    idd = N.DeviceArray.from_host(ids2)
    out = N.DeviceArray((b, s, dim), dt)
    N.check(N.lib.nml_embedding_gather_device(wd.ptr, pd.ptr, idd.ptr, out.ptr, b, s, dim, vocab,
                                              pd.shape[0], None, None, N.np_dtype_code(dt)))
    return out.reshape(*shape, dim)


def linear(x, weights, bias=None, *, epilogue=None, resid=None):
    """``epi(x @ weights + bias)`` with ``weights`` in the reference layout (in, out)."""
    dt = _float_dtype(x)
    xd = _dev(x, dt)
    w = np.ascontiguousarray(np.asarray(weights, dtype=dt).T)
    wd = N.DeviceArray.from_host(w)
    n_out, k = w.shape
    rows = xd.size // k
    if epilogue is None:
        epilogue = EPI_BIAS if bias is not None else EPI_NONE
    bd = _dev(bias, dt) if bias is not None else None
    rd = _dev(resid, dt) if resid is not None else None
    out = N.DeviceArray((rows, n_out), dt)
    N.check(N.lib.nml_linear_device(xd.ptr, k, wd.ptr, N.ptr(bd), N.ptr(rd), out.ptr, rows, k,
                                    n_out, int(epilogue), N.np_dtype_code(dt)))
    return out


def linear_t(x, w_t, bias=None, *, epilogue=None):
    """``epi(x @ w_tᵀ + bias)`` with ``w_t`` a DeviceArray already in the device layout
    (out, in) and ``bias`` a DeviceArray or None: no host copy of the weights."""
    dt = _float_dtype(x)
    xd = _dev(x, dt)
    n_out, k = w_t.shape
    rows = xd.size // k
    if epilogue is None:
        epilogue = EPI_BIAS if bias is not None else EPI_NONE
    out = N.DeviceArray((rows, n_out), dt)
    N.check(N.lib.nml_linear_device(xd.ptr, k, w_t.ptr, N.ptr(bias), None, out.ptr, rows, k,
                                    n_out, int(epilogue), N.np_dtype_code(dt)))
    return out


def fused_tied_crossentropy_forward(hidden, weights, label_indices, ignore_index=None):
    """Mean CE of ``hidden @ weights.T`` against labels (float)."""
    dt = _float_dtype(hidden)
    hd, wd = _dev(hidden, dt), _dev(weights, dt)
    rows, dim = hd.shape
    labels = np_backend.as_label_indices(label_indices, batch_size=rows)
    ld = N.DeviceArray.from_host(labels)
    loss = C.c_double()
    has = ignore_index is not None
    N.check(N.lib.nml_tied_ce_forward_device(hd.ptr, wd.ptr, ld.ptr, rows, dim, wd.shape[0],
                                             int(ignore_index) if has else 0, int(has),
                                             C.byref(loss), N.np_dtype_code(dt)))
    return float(loss.value)


def sample_tokens(logits, *, temperature, top_k=0, top_p=1.0, uniforms=None, history=None,
                  repetition_penalty=1.0):
    """One token per row of (batch, vocab) logits with ``_sample_logits`` semantics;
    ``uniforms[b]`` replaces row b's RandomState draw; ``history`` is a list of the
    token ids already in each row (repetition penalty)."""
    dt = _float_dtype(logits)
    ld = _dev(logits, dt)
    batch, vocab = ld.shape
    ud = None
    if temperature > 0:
        ud = N.DeviceArray.from_host(np.asarray(uniforms, dtype=np.float64).reshape(batch))
    hd = hl = None
    stride = 0
    if history is not None:
        stride = max(1, max(len(h) for h in history))
        hist = np.zeros((batch, stride), dtype=np.int64)
        for b, h in enumerate(history):
            hist[b, :len(h)] = h
        hd = N.DeviceArray.from_host(hist)
        hl = N.DeviceArray.from_host(np.asarray([len(h) for h in history], dtype=np.int32))
    out = N.DeviceArray((batch,), np.int64)
    N.check(N.lib.nml_sample_device(ld.ptr, batch, vocab, float(temperature), int(top_k or 0),
                                    float(top_p if top_p is not None else 1.0),
                                    float(repetition_penalty), N.ptr(ud), N.ptr(hd), stride,
                                    N.ptr(hl), out.ptr, N.np_dtype_code(dt)))
    return out.numpy()


def adamw_step(param, grad, m, v, lr, beta1, beta2, bias1, bias2, eps, weight_decay):
    """AdamW update of float32 ``DeviceArray``s in place, the reference native kernel's
    arithmetic (``native.adamw_step``, module.cpp:175-188): bias1/bias2 are the caller's
    ``1 − β^t`` bias corrections, as optimizers/adam.py:93-94 passes them."""
    arrs = [param, grad, m, v]
    for a in arrs:
        if not isinstance(a, N.DeviceArray) or a.dtype != np.float32:
            raise TypeError("adamw_step takes float32 DeviceArrays")
    n = param.size
    if any(a.size != n for a in arrs):
        raise ValueError("adamw_step: param, grad, m and v must have the same size")
    N.check(N.lib.nml_adamw_step_device(param.ptr, grad.ptr, m.ptr, v.ptr, n, float(lr),
                                        float(beta1), float(beta2), float(bias1), float(bias2),
                                        float(eps), float(weight_decay)))


def clip_grad_norm(grads, max_norm):
    """Global L2 norm of float32 gradient ``DeviceArray``s, scaled in place to max_norm
    when above it (``native.clip_grad_norm``, module.cpp:190-200). Returns the norm."""
    grads = list(grads)
    for g in grads:
        if not isinstance(g, N.DeviceArray) or g.dtype != np.float32:
            raise TypeError("clip_grad_norm takes float32 DeviceArrays")
    ptrs = (C.c_void_p * max(1, len(grads)))(*[g.ptr for g in grads])
    sizes = (C.c_size_t * max(1, len(grads)))(*[g.size for g in grads])
    norm = C.c_float()
    N.check(N.lib.nml_clip_grad_norm_device(ptrs, sizes, len(grads), float(max_norm),
                                            C.byref(norm)))
    return float(norm.value)
