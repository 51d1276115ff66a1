"""NumPy restatement of the reference's optimizer step (test infrastructure).

adamw_step: native/src/adamw.cpp:6-20 (adamw_step_cpu), float32 throughout, every op in
the C++ order (NumPy float32 ufuncs round each op once, as the C++ float ops do without
contraction). clip_grad_norm: adamw.cpp:22-37 (clip_grad_norm_cpu): Σ double(g)·g over
every element of every tensor in order, norm = float(√total), and when norm > max_norm
(and > 0) each gradient times max_norm / (norm + 1e-6) in float32.

Only tests and bench.py's CPU-baseline leg use this module.
"""
from __future__ import annotations

import numpy as np


def adamw_step(param, grad, m, v, lr, beta1, beta2, bias1, bias2, eps, weight_decay):
    """In place on float32 arrays, like native.adamw_step."""
    f = np.float32
    lr, b1, b2, bc1, bc2, ep, wd = (f(x) for x in (lr, beta1, beta2, bias1, bias2, eps, weight_decay))
    g = grad
    m[...] = b1 * m + (f(1.0) - b1) * g
    v[...] = b2 * v + ((f(1.0) - b2) * g) * g
    mhat = m / bc1
    vhat = v / bc2
    scratch = (lr * mhat) / (np.sqrt(vhat) + ep)
    if wd != f(0.0):
        decay = f(1.0) - lr * wd
        param *= decay
    param -= scratch


def clip_grad_norm(grads, max_norm):
    """In place on float32 arrays; returns the float32 norm."""
    sq = [np.asarray(g, np.float64).ravel() ** 2 for g in grads]
    total = np.cumsum(np.concatenate(sq))[-1] if sq and sum(s.size for s in sq) else 0.0
    norm = np.float32(np.sqrt(total))
    mx = np.float32(max_norm)
    if norm > mx and norm > np.float32(0.0):
        scale = mx / (norm + np.float32(1e-6))
        for g in grads:
            g *= scale
    return norm
