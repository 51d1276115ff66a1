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
    h_ = num_heads
    dk = d // h_
    scale = float(dk) ** 0.5
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
        p, pm, pf = _layer_names(i)
        n1, ms1, rms1 = _rms_fwd(x, w[p + "ln1.gamma"])
        w_qkv = np.concatenate([w[pm + "W_q.weights"], w[pm + "W_k.weights"],
                                w[pm + "W_v.weights"]], axis=1)
        b_qkv = np.concatenate([w[pm + "W_q.biases"], w[pm + "W_k.biases"],
                                w[pm + "W_v.biases"]])
        qkv = n1 @ w_qkv + b_qkv
        q = _split_heads(qkv[:, :d], b, s, h_, dk)
        k = _split_heads(qkv[:, d:2 * d], b, s, h_, dk)
        v = _split_heads(qkv[:, 2 * d:], b, s, h_, dk)
        if rope is not None:
            q = apply_rope(q, rope[0], rope[1])
            k = apply_rope(k, rope[0], rope[1])
        sc = np.matmul(q, np.swapaxes(k, -2, -1)) / scale + mask
        sc = sc - np.max(sc, axis=-1, keepdims=True)
        e = np.exp(sc)
        probs = e / np.sum(e, axis=-1, keepdims=True)
        att = np.matmul(probs, v)
        merged = _merge_heads(att, b, s, h_, dk).reshape(n, d)
        x_mid = x + merged @ w[pm + "W_o.weights"] + w[pm + "W_o.biases"]
        n2, ms2, rms2 = _rms_fwd(x_mid, w[p + "ln2.gamma"])
        pre = n2 @ w[pf + "dense1.weights"] + w[pf + "dense1.biases"]
        hid, tu = _gelu_fwd(pre)
        x_out = x_mid + hid @ w[pf + "dense2.weights"] + w[pf + "dense2.biases"]
        saves.append((x, n1, ms1, rms1, w_qkv, q, k, v, probs, merged, x_mid, n2, ms2, rms2,
                      pre, hid, tu))
        x = x_out
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
        p, pm, pf = _layer_names(i)
        (x0, n1, ms1, rms1, w_qkv, q, k, v, probs, merged, x_mid, n2, ms2, rms2, pre, hid,
         tu) = saves[i]
        # FFN (_fused_arrays.py:225-248)
        grads[pf + "dense2.weights"] += hid.T @ g
        grads[pf + "dense2.biases"] += g.sum(axis=0)
        dpre = _gelu_bwd(g @ w[pf + "dense2.weights"].T, pre, tu)
        grads[pf + "dense1.weights"] += n2.T @ dpre
        grads[pf + "dense1.biases"] += dpre.sum(axis=0)
        dn2 = dpre @ w[pf + "dense1.weights"].T
        gx, dg2 = _rms_bwd(dn2, x_mid, w[p + "ln2.gamma"], ms2, rms2)
        grads[p + "ln2.gamma"] += dg2
        g = g + gx
        # MHA (_fused_arrays.py:129-184)
        grads[pm + "W_o.weights"] += merged.T @ g
        grads[pm + "W_o.biases"] += g.sum(axis=0)
        dmerged = g @ w[pm + "W_o.weights"].T
        datt = _split_heads(dmerged, b, s, h_, dk)
        dprobs = np.matmul(datt, np.swapaxes(v, -2, -1))
        dsc = probs * (dprobs - np.sum(dprobs * probs, axis=-1, keepdims=True))
        dsc = dsc / scale
        dq = np.matmul(dsc, k)
        dk_ = np.matmul(np.swapaxes(dsc, -2, -1), q)
        dv = np.matmul(np.swapaxes(probs, -2, -1), datt)
        if rope is not None:
            dq = _rope_inv(dq, rope[0], rope[1])
            dk_ = _rope_inv(dk_, rope[0], rope[1])
        dqkv = np.concatenate([_merge_heads(t, b, s, h_, dk).reshape(n, d) for t in (dq, dk_, dv)],
                              axis=1)
        dw_qkv = n1.T @ dqkv
        db_qkv = dqkv.sum(axis=0)
        for j, nm in enumerate(("W_q", "W_k", "W_v")):
            grads[pm + nm + ".weights"] += dw_qkv[:, j * d:(j + 1) * d]
            grads[pm + nm + ".biases"] += db_qkv[j * d:(j + 1) * d]
        dn1 = dqkv @ w_qkv.T
        gx, dg1 = _rms_bwd(dn1, x0, w[p + "ln1.gamma"], ms1, rms1)
        grads[p + "ln1.gamma"] += dg1
        g = g + gx
    np.add.at(grads["token_emb.weights"], ids.reshape(-1), g)
    if rope is None:
        grads["pos_emb.weights"][:s] += g.reshape(b, s, d).sum(axis=0)
    return loss, grads


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
