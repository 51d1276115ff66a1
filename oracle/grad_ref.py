"""Backward of ``GPT.compute_loss`` in NumPy — the oracle for the device training path
(test infrastructure: only tests use this module).

``loss_and_grads`` runs the forward of :mod:`oracle.gpt_ref` keeping what the
reference's array-level ops keep for backward, then the reference's backward in the
order its autograd runs it (``loss.backward()`` after ``compute_loss``):

* tied cross-entropy: kernels/fused_tied_crossentropy.py:27-48 with
  kernels/fused_crossentropy.py:33-50 (``probs − onehot`` times ``grad_scale / n``),
  ``ignore_index`` rows dropped first and their hidden-state gradient left zero
  (losses/cross_entropy.py:130-191);
* final RMSNorm and every block in reverse: neural_network/_fused_arrays.py:307-377
  (``grad_mid = g + RMSNorm₂ᵀ(FFNᵀ(g))``, ``grad_x0 = grad_mid + RMSNorm₁ᵀ(MHAᵀ(grad_mid))``);
* FFN: _fused_arrays.py:225-248; GELU: kernels/fused_gelu.py:86-111 (native/src/gelu.cpp:23-33);
* MHA: _fused_arrays.py:129-184; SDPA: kernels/fused_sdpa.py:26-29, :81-88 (the scores
  gradient divided by ``scale = sqrt(dk)``); RoPE inverse rotation at :151-154;
* RMSNorm: kernels/fused_rmsnorm.py:208-217 (the fp32 CPU branch);
* embeddings: token rows scatter-added (kernels/embedding_scatter.py:39-60), positions
  summed over the batch into ``pos_emb[:S]`` (layers/embedding.py:110-116).

The arithmetic is carried in the dtype of ``w`` (float64 for the checks: the device's
fp32 result is compared with the float64 gradient under a stated tolerance). Gradients
come back under the reference's parameter names, in the reference's ``(in, out)``
layouts.
"""
from __future__ import annotations

import numpy as np

from oracle.gpt_ref import GELU_COEF, GELU_K, RMS_EPS, _merge_heads, _split_heads, apply_rope

DU_DX_COEF = 3.0 * GELU_COEF  # native/src/gelu.cpp:9


def _rms_fwd(x, g, eps=RMS_EPS):
    ms = np.mean(x * x, axis=-1, keepdims=True)
    rms = np.sqrt(ms + eps)
    return (x / rms) * g, ms, rms


def _rms_bwd(grad, x, g, ms, rms, eps=RMS_EPS):
    """kernels/fused_rmsnorm.py:208-217."""
    d = x.shape[-1]
    x_hat = x / rms
    grad_gamma = np.sum(grad * x_hat, axis=0)
    gxh = grad * g
    row_dot = np.sum(gxh * x, axis=-1, keepdims=True)
    grad_ms = row_dot * (-0.5) * (ms + eps) ** (-1.5)
    coef = (2.0 / d) * grad_ms
    return gxh / rms + x * coef, grad_gamma


def _gelu_fwd(x):
    tu = np.tanh(GELU_K * (x + GELU_COEF * x * x * x))
    return 0.5 * x * (1.0 + tu), tu


def _gelu_bwd(grad, x, tu):
    """native/src/gelu.cpp:23-33."""
    du_dx = GELU_K * (1.0 + DU_DX_COEF * x * x)
    sech2 = 1.0 - tu * tu
    return grad * (0.5 * (1.0 + tu) + 0.5 * x * sech2 * du_dx)


def _rope_inv(x, cos, sin):
    """R(−θ)·x: the transpose of apply_rope's rotation (_fused_arrays.py:151-154)."""
    return apply_rope(x, cos, -sin)


def _layer_names(i):
    p = f"blocks.layers.{i}."
    return p, p + "mha.", p + "ffn."


def _mha_fwd(x2d, w, pm, b, s, num_heads, mask, rope):
    """mha_forward_arrays (_fused_arrays.py:52-126) on (b·s, d) rows: ``(out, saved)``.
    ``mask``: an additive (s, s) array, or None for none."""
    n, d = x2d.shape
    dk = d // num_heads
    scale = float(dk) ** 0.5
    w_qkv = np.concatenate([w[pm + "W_q.weights"], w[pm + "W_k.weights"],
                            w[pm + "W_v.weights"]], axis=1)
    b_qkv = np.concatenate([w[pm + "W_q.biases"], w[pm + "W_k.biases"],
                            w[pm + "W_v.biases"]])
    qkv = x2d @ w_qkv + b_qkv
    q = _split_heads(qkv[:, :d], b, s, num_heads, dk)
    k = _split_heads(qkv[:, d:2 * d], b, s, num_heads, dk)
    v = _split_heads(qkv[:, 2 * d:], b, s, num_heads, dk)
    if rope is not None:
        q = apply_rope(q, rope[0], rope[1])
        k = apply_rope(k, rope[0], rope[1])
    sc = np.matmul(q, np.swapaxes(k, -2, -1)) / scale
    if mask is not None:
        sc = sc + mask
    sc = sc - np.max(sc, axis=-1, keepdims=True)
    e = np.exp(sc)
    probs = e / np.sum(e, axis=-1, keepdims=True)
    att = np.matmul(probs, v)
    merged = _merge_heads(att, b, s, num_heads, dk).reshape(n, d)
    out = merged @ w[pm + "W_o.weights"] + w[pm + "W_o.biases"]
    return out, (x2d, w_qkv, q, k, v, probs, merged)


def _mha_bwd(g, saved, w, pm, b, s, num_heads, grads, rope):
    """mha_backward_arrays (_fused_arrays.py:129-184): adds the projection gradients to
    ``grads`` and returns d/d(input rows). SDPA: kernels/fused_sdpa.py:26-29, :81-88 (the
    scores gradient divided by ``scale = sqrt(dk)``); RoPE inverse rotation at :151-154."""
    x2d, w_qkv, q, k, v, probs, merged = saved
    n, d = x2d.shape
    dk = d // num_heads
    scale = float(dk) ** 0.5
    grads[pm + "W_o.weights"] += merged.T @ g
    grads[pm + "W_o.biases"] += g.sum(axis=0)
    dmerged = g @ w[pm + "W_o.weights"].T
    datt = _split_heads(dmerged, b, s, num_heads, dk)
    dprobs = np.matmul(datt, np.swapaxes(v, -2, -1))
    dsc = probs * (dprobs - np.sum(dprobs * probs, axis=-1, keepdims=True))
    dsc = dsc / scale
    dq = np.matmul(dsc, k)
    dk_ = np.matmul(np.swapaxes(dsc, -2, -1), q)
    dv = np.matmul(np.swapaxes(probs, -2, -1), datt)
    if rope is not None:
        dq = _rope_inv(dq, rope[0], rope[1])
        dk_ = _rope_inv(dk_, rope[0], rope[1])
    dqkv = np.concatenate([_merge_heads(t, b, s, num_heads, dk).reshape(n, d)
                           for t in (dq, dk_, dv)], axis=1)
    dw_qkv = x2d.T @ dqkv
    db_qkv = dqkv.sum(axis=0)
    for j, nm in enumerate(("W_q", "W_k", "W_v")):
        grads[pm + nm + ".weights"] += dw_qkv[:, j * d:(j + 1) * d]
        grads[pm + nm + ".biases"] += db_qkv[j * d:(j + 1) * d]
    return dqkv @ w_qkv.T


def _ffn_fwd(x2d, w, pf):
    """ffn_forward_arrays (_fused_arrays.py:187-222)."""
    pre = x2d @ w[pf + "dense1.weights"] + w[pf + "dense1.biases"]
    hid, tu = _gelu_fwd(pre)
    return hid @ w[pf + "dense2.weights"] + w[pf + "dense2.biases"], (x2d, pre, hid, tu)


def _ffn_bwd(g, saved, w, pf, grads):
    """ffn_backward_arrays (_fused_arrays.py:225-248); GELU: kernels/fused_gelu.py:86-111
    (native/src/gelu.cpp:23-33)."""
    x2d, pre, hid, tu = saved
    grads[pf + "dense2.weights"] += hid.T @ g
    grads[pf + "dense2.biases"] += g.sum(axis=0)
    dpre = _gelu_bwd(g @ w[pf + "dense2.weights"].T, pre, tu)
    grads[pf + "dense1.weights"] += x2d.T @ dpre
    grads[pf + "dense1.biases"] += dpre.sum(axis=0)
    return dpre @ w[pf + "dense1.weights"].T


def _block_fwd(x, w, i, b, s, num_heads, mask, rope):
    """fused_block_forward_arrays (_fused_arrays.py:251-284) on (b·s, d) rows."""
    p, pm, pf = _layer_names(i)
    n1, ms1, rms1 = _rms_fwd(x, w[p + "ln1.gamma"])
    a_out, msave = _mha_fwd(n1, w, pm, b, s, num_heads, mask, rope)
    x_mid = x + a_out
    n2, ms2, rms2 = _rms_fwd(x_mid, w[p + "ln2.gamma"])
    f_out, fsave = _ffn_fwd(n2, w, pf)
    return x_mid + f_out, (x, ms1, rms1, msave, x_mid, ms2, rms2, fsave)


def _block_bwd(g, saved, w, i, b, s, num_heads, grads, rope):
    """fused_block_backward_arrays (_fused_arrays.py:335-377):
    ``grad_mid = g + RMSNorm₂ᵀ(FFNᵀ(g))``, ``grad_x0 = grad_mid + RMSNorm₁ᵀ(MHAᵀ(grad_mid))``."""
    p, pm, pf = _layer_names(i)
    x0, ms1, rms1, msave, x_mid, ms2, rms2, fsave = saved
    dn2 = _ffn_bwd(g, fsave, w, pf, grads)
    gx, dg2 = _rms_bwd(dn2, x_mid, w[p + "ln2.gamma"], ms2, rms2)
    grads[p + "ln2.gamma"] += dg2
    g = g + gx
    dn1 = _mha_bwd(g, msave, w, pm, b, s, num_heads, grads, rope)
    gx, dg1 = _rms_bwd(dn1, x0, w[p + "ln1.gamma"], ms1, rms1)
    grads[p + "ln1.gamma"] += dg1
    return g + gx


def loss_and_grads(w, ids, labels, num_heads, num_layers, ignore_index=None, rope=None,
                   grad_scale=1.0):
    """``(loss, {name: grad})`` of ``compute_loss(ids, labels)`` and one ``backward()``.

    ``w``: parameters under the reference names (``oracle.weights``), all one float dtype.
    ``rope``: the (cos, sin) cache of a ``use_rope=True`` model (then no ``pos_emb``).
    """
    dt = w["token_emb.weights"].dtype
    ids = np.asarray(ids, dtype=np.int64)
    b, s = ids.shape
    emb = w["token_emb.weights"]
    d = emb.shape[1]
    n = b * s
    if rope is not None:
        rope = (rope[0].astype(dt), rope[1].astype(dt))

    # ---------------------------------------------------------------- forward
    x = emb[ids.reshape(-1)].reshape(n, d).astype(dt)
    if rope is None:
        x = x + np.tile(w["pos_emb.weights"][:s], (b, 1))
    mask = np.triu(np.full((s, s), -np.inf, dtype=dt), k=1)
    saves = []
    for i in range(num_layers):
        x, sv = _block_fwd(x, w, i, b, s, num_heads, mask, rope)
        saves.append(sv)
    hf, msf, rmsf = _rms_fwd(x, w["ln.gamma"])

    labels = np.asarray(labels, dtype=np.int64).reshape(-1)
    if labels.size != n:
        raise ValueError(f"label count ({labels.size}) must match batch size ({n}).")
    valid = np.ones(n, bool) if ignore_index is None else labels != ignore_index
    grads = {name: np.zeros_like(a) for name, a in w.items()}
    nv = int(valid.sum())
    if nv == 0:
        return 0.0, grads
    hv = hf[valid]
    lv = labels[valid]
    logits = hv @ emb.T
    mx = np.max(logits, axis=1, keepdims=True)
    ex = np.exp(logits - mx)
    se = np.sum(ex, axis=1, keepdims=True)
    loss = float(np.mean(mx.ravel() + np.log(se.ravel()) - logits[np.arange(nv), lv]))

    # --------------------------------------------------------------- backward
    dlog = ex / se
    dlog[np.arange(nv), lv] -= 1.0
    dlog *= grad_scale / nv
    dh = np.zeros((n, d), dt)
    dh[valid] = dlog @ emb
    grads["token_emb.weights"] += dlog.T @ hv

    g, dgf = _rms_bwd(dh, x, w["ln.gamma"], msf, rmsf)
    grads["ln.gamma"] += dgf
    for i in reversed(range(num_layers)):
        g = _block_bwd(g, saves[i], w, i, b, s, num_heads, grads, rope)
    np.add.at(grads["token_emb.weights"], ids.reshape(-1), g)
    if rope is None:
        grads["pos_emb.weights"][:s] += g.reshape(b, s, d).sum(axis=0)
    return loss, grads


# ------------------------------------------------------ module-level vector-Jacobian products
# Each returns the module's output, d(<dout, out>)/d(input) and {name: gradient} for the
# parameters it reads (reference names and (in, out) layouts): the closures the reference's
# modules attach (utils/tensor.py:286-332 runs them).

def logits_vjp(w, ids, dlogits, num_heads, num_layers, rope=None):
    """GPT.forward (models/gpt.py:92-121) and the backward its graph runs for a given
    d(loss)/d(logits) (batch, seq, vocab): ``(logits, {name: grad})`` — the tied head
    (gpt.py:150-153), the final RMSNorm, every block in reverse, the embeddings."""
    dt = w["token_emb.weights"].dtype
    ids = np.asarray(ids, dtype=np.int64)
    b, s = ids.shape
    emb = w["token_emb.weights"]
    d = emb.shape[1]
    n = b * s
    if rope is not None:
        rope = (rope[0].astype(dt), rope[1].astype(dt))
    x = emb[ids.reshape(-1)].reshape(n, d).astype(dt)
    if rope is None:
        x = x + np.tile(w["pos_emb.weights"][:s], (b, 1))
    mask = np.triu(np.full((s, s), -np.inf, dtype=dt), k=1)
    saves = []
    for i in range(num_layers):
        x, sv = _block_fwd(x, w, i, b, s, num_heads, mask, rope)
        saves.append(sv)
    hf, msf, rmsf = _rms_fwd(x, w["ln.gamma"])
    logits = hf @ emb.T
    grads = {name: np.zeros_like(a) for name, a in w.items()}
    dl = np.asarray(dlogits, dtype=dt).reshape(n, -1)
    grads["token_emb.weights"] += dl.T @ hf
    g, dgf = _rms_bwd(dl @ emb, x, w["ln.gamma"], msf, rmsf)
    grads["ln.gamma"] += dgf
    for i in reversed(range(num_layers)):
        g = _block_bwd(g, saves[i], w, i, b, s, num_heads, grads, rope)
    np.add.at(grads["token_emb.weights"], ids.reshape(-1), g)
    if rope is None:
        grads["pos_emb.weights"][:s] += g.reshape(b, s, d).sum(axis=0)
    return logits.reshape(b, s, -1), grads


def blocks_vjp(w, layers, x, dout, num_heads, mask=None, rope=None, final_gamma=None):
    """FusedTransformerBlock (``layers = [i]``, transformer_fused.py:65-78) or
    FusedGPTTrunk (every layer then the final RMSNorm of ``final_gamma``,
    transformer_fused.py:128-136 → _fused_arrays.py:311-332) over x (b, s, d). ``mask``:
    additive (s, s) or None for none (the modules' own None is the causal mask). The
    final norm's gradient comes back under ``"final.gamma"``."""
    b, s, d = x.shape
    cur = x.reshape(b * s, d)
    saves = []
    for i in layers:
        cur, sv = _block_fwd(cur, w, i, b, s, num_heads, mask, rope)
        saves.append(sv)
    grads = {name: np.zeros_like(a) for name, a in w.items()}
    g = dout.reshape(b * s, d)
    out = cur
    if final_gamma is not None:
        out, msf, rmsf = _rms_fwd(cur, final_gamma)
        g, dgf = _rms_bwd(g, cur, final_gamma, msf, rmsf)
        grads["final.gamma"] = dgf
    for i, sv in reversed(list(zip(layers, saves))):
        g = _block_bwd(g, sv, w, i, b, s, num_heads, grads, rope)
    return out.reshape(b, s, d), g.reshape(b, s, d), grads


def mha_vjp(w, prefix, x, dout, num_heads, mask=None):
    """MultiHeadAttention.forward (attention.py:139-168; its SDPA closure :103-119) with the
    parameters under ``prefix`` (e.g. ``"blocks.layers.0.mha."``)."""
    b, s, d = x.shape
    out, saved = _mha_fwd(x.reshape(b * s, d), w, prefix, b, s, num_heads, mask, None)
    grads = {name: np.zeros_like(a) for name, a in w.items()}
    dx = _mha_bwd(dout.reshape(b * s, d), saved, w, prefix, b, s, num_heads, grads, None)
    return out.reshape(b, s, d), dx.reshape(b, s, d), grads


def ffn_vjp(w, prefix, x, dout):
    """FeedForward.forward and its closure (neural_network/feed_forward.py:105-129)."""
    d = x.shape[-1]
    out, saved = _ffn_fwd(x.reshape(-1, d), w, prefix)
    grads = {name: np.zeros_like(a) for name, a in w.items()}
    dx = _ffn_bwd(dout.reshape(-1, d), saved, w, prefix, grads)
    return out.reshape(x.shape), dx.reshape(x.shape), grads


def dense_vjp(weights, biases, x, dout):
    """Dense.forward's closure (layers/dense.py:81-94): ``(out, dx, dW, db)``."""
    x2 = x.reshape(-1, weights.shape[0])
    g2 = dout.reshape(-1, weights.shape[1])
    out = x2 @ weights + (biases if biases is not None else 0)
    return (out.reshape(*x.shape[:-1], weights.shape[1]), (g2 @ weights.T).reshape(x.shape),
            x2.T @ g2, g2.sum(axis=0))


def embedding_vjp(vocab, ids, dout):
    """Embedding.forward's closure (layers/embedding.py:63-69 → embedding_scatter.py:39-60):
    the (vocab, dim) gradient with each id's rows of dout added in."""
    dim = dout.shape[-1]
    g = np.zeros((vocab, dim), dout.dtype)
    np.add.at(g, np.asarray(ids, np.int64).reshape(-1), dout.reshape(-1, dim))
    return g


# ------------------------------------------------ single ops of the native extension
def flash_forward(q, k, v, scale):
    """The reference's native flash attention forward (native/src/sdpa_cuda.cu:40-77) in the
    dtype of ``q``: causal over (bh, seq, dk), scores ``(q_i·k_j)·scale`` (``scale``
    multiplies), returning ``out`` and each query row's max score ``m`` and
    ``l = Σ_j exp(s_ij − m)``."""
    s = np.matmul(q, np.swapaxes(k, -2, -1)) * scale
    seq = q.shape[-2]
    s = np.where(np.tril(np.ones((seq, seq), dtype=bool)), s, -np.inf)
    m = s.max(axis=-1)
    e = np.exp(s - m[..., None])
    lsum = e.sum(axis=-1)
    return np.matmul(e, v) / lsum[..., None], m, lsum


def flash_backward(grad_out, q, k, v, scale):
    """Its backward (sdpa_cuda.cu:79-133): P = softmax of the causal scores,
    dV = Pᵀ·dO, dP = dO·Vᵀ, D_i = Σ_j P_ij dP_ij, dS = P∘(dP − D), dQ = dS·K·scale,
    dK = dSᵀ·Q·scale."""
    out, m, lsum = flash_forward(q, k, v, scale)
    s = np.matmul(q, np.swapaxes(k, -2, -1)) * scale
    seq = q.shape[-2]
    s = np.where(np.tril(np.ones((seq, seq), dtype=bool)), s, -np.inf)
    p = np.exp(s - m[..., None]) / lsum[..., None]
    dv = np.matmul(np.swapaxes(p, -2, -1), grad_out)
    dp = np.matmul(grad_out, np.swapaxes(v, -2, -1))
    dvec = (p * dp).sum(axis=-1, keepdims=True)
    ds = p * (dp - dvec)
    return np.matmul(ds, k) * scale, np.matmul(np.swapaxes(ds, -2, -1), q) * scale, dv


def rmsnorm_backward(grad, x, gamma, eps=RMS_EPS):
    """RMSNorm backward of the native extension (sdpa_cuda.cu:167-201; the fp32 CPU branch
    kernels/fused_rmsnorm.py:208-217 is the same mathematics): ``(grad_x, grad_gamma)``."""
    x2 = x.reshape(-1, x.shape[-1])
    g2 = grad.reshape(-1, x.shape[-1])
    ms = np.mean(x2 * x2, axis=-1, keepdims=True)
    rms = np.sqrt(ms + eps)
    gx, gg = _rms_bwd(g2, x2, gamma, ms, rms, eps)
    return gx.reshape(x.shape), gg
