"""NumPy restatement of NimbleML's CPU GPT path — the oracle (test infrastructure).

Every function follows the reference CPU branch it cites, with the same NumPy
operations in the same order and dtypes, so that fp16 runs round after every
op exactly like the reference (NumPy fp16 matmul/sum: fp32 accumulate, one
rounding per op). ``weights`` is a ``{name: ndarray}`` dict as produced by
``oracle.weights.make_weights`` (reference checkpoint names).

Only tests, ``__graft_entry__.smoke`` and ``bench.py``'s CPU-baseline leg use
this module.
"""
from __future__ import annotations

import numpy as np

from oracle import halfmm

GELU_K = 0.7978845608028654  # sqrt(2/pi), native/src/gelu.cpp:7
GELU_COEF = 0.044715  # native/src/gelu.cpp:8
RMS_EPS = 1e-5  # layers/rms_norm.py:16


# --------------------------------------------------------------------------- ops
def _mm(a, b):
    """``a @ b`` with NumPy's semantics; float16 products go through the exact C
    restatement of NumPy's float16 loop (oracle/halfmm.c), which is much faster."""
    if a.dtype == np.float16 and b.dtype == np.float16:
        return halfmm.matmul16(a, b)
    return np.matmul(a, b)


def embed(tok_w, pos_w, ids):
    """``token_emb(ids) + pos_emb.forward_prefix(S)``.

    models/gpt.py:85-86; gather = kernels/embedding_scatter.py:25-36 (``w[ids]``);
    prefix view = layers/embedding.py:72-118 (``W[:S]``), broadcast over batch.
    """
    ids = np.asarray(ids, dtype=np.int64)
    s = ids.shape[1]
    x = tok_w[ids.reshape(-1)].reshape(ids.shape[0], s, tok_w.shape[1])
    if pos_w is None:  # rotary positions: no learned table (models/gpt.py:85)
        return x
    if s > pos_w.shape[0]:
        raise ValueError(f"Sequence length {s} exceeds maximum sequence length {pos_w.shape[0]}")
    return x + pos_w[:s]


def rope_cache(seq_len, head_dim, base=10000.0):
    """utils/rope.py:12-19: float32 ``(cos, sin)``, ``(seq_len, head_dim)``, both halves of
    a row holding ``position · base^(-i/half)``."""
    half = head_dim // 2
    inv_freq = 1.0 / (base ** (np.arange(0, half, dtype=np.float32) / float(half)))
    t = np.arange(seq_len, dtype=np.float32)
    freqs = np.outer(t, inv_freq)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def apply_rope(x, cos, sin, offset=0):
    """utils/rope.py:22-44 (GPT-NeoX half split) on ``x`` (..., seq, head_dim): pair
    (i, i + half) rotated by position·θ_i, the tables cast to x's dtype first. ``offset``
    is the first row's position (0 in the reference, which re-forwards from position 0;
    the incremental oracle feeds later positions)."""
    seq = x.shape[-2]
    half = x.shape[-1] // 2
    c = cos[offset:offset + seq, :half].astype(x.dtype, copy=False)
    s = sin[offset:offset + seq, :half].astype(x.dtype, copy=False)
    x1 = x[..., :half]
    x2 = x[..., half:]
    out = np.empty_like(x)
    out[..., :half] = x1 * c - x2 * s
    out[..., half:] = x1 * s + x2 * c
    return out


def rmsnorm(x, gamma, eps=RMS_EPS):
    """kernels/fused_rmsnorm.py:153-162 (CPU branches: fp16 at :153-158, else :159-162)."""
    if x.dtype == np.float16:
        ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
        rms = np.sqrt(ms + np.float32(eps))
        inv = (1.0 / rms).astype(np.float16)
        return (x * inv) * gamma
    ms = np.mean(x * x, axis=-1, keepdims=True)
    rms = np.sqrt(ms + eps)
    return (x / rms) * gamma


def gelu(x):
    """tanh-GELU. fp32: native gelu_forward_cpu (native/src/gelu.cpp:12-21, reached
    via kernels/fused_gelu.py:61-64); other dtypes: NumPy at fused_gelu.py:67-69."""
    if x.dtype == np.float32:
        x3 = x * x * x
        tu = np.tanh(np.float32(GELU_K) * (x + np.float32(GELU_COEF) * x3))
        return np.float32(0.5) * x * (np.float32(1.0) + tu)
    tu = np.tanh(GELU_K * (x + GELU_COEF * x * x * x))
    out = 0.5 * x * (1.0 + tu)
    return out.astype(x.dtype, copy=False)


def causal_mask(s, dtype):
    """utils/mask.py:8-13: ``triu(full(-inf), k=1)`` in the compute dtype."""
    return np.triu(np.full((s, s), -np.inf, dtype=dtype), k=1)


def softmax(a, axis=-1):
    """kernels/fused_sdpa.py:19-23."""
    m = np.max(a, axis=axis, keepdims=True)
    e = np.exp(a - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def sdpa(q, k, v, scale, mask):
    """kernels/fused_sdpa.py:71-78 (the CPU ``auto`` path, :284-288)."""
    scores = _mm(q, np.swapaxes(k, -2, -1))
    np.divide(scores, scale, out=scores)
    if mask is not None:
        np.add(scores, mask, out=scores)
    probs = softmax(scores, axis=-1)
    return _mm(probs, v)


def _split_heads(a, b, s, h, dk):
    """neural_network/_fused_arrays.py:42-45."""
    return np.transpose(a.reshape(b, s, h, dk), (0, 2, 1, 3)).reshape(b * h, s, dk)


def _merge_heads(a, b, s, h, dk):
    """neural_network/_fused_arrays.py:48-50."""
    return np.transpose(a.reshape(b, h, s, dk), (0, 2, 1, 3)).reshape(b, s, h * dk)


def mha(x, w, prefix, num_heads, mask, rope=None):
    """neural_network/_fused_arrays.py:52-126; rope = (cos, sin) rotates q and k after the
    head split (:95-98)."""
    b, s, d = x.shape
    dk = d // num_heads
    scale = float(dk) ** 0.5  # neural_network/attention.py:135
    x2d = x.reshape(b * s, d)
    w_qkv = np.concatenate([w[prefix + "W_q.weights"], w[prefix + "W_k.weights"],
                            w[prefix + "W_v.weights"]], axis=1)
    qkv = _mm(x2d, w_qkv)
    qkv = qkv + np.concatenate([w[prefix + "W_q.biases"], w[prefix + "W_k.biases"],
                                w[prefix + "W_v.biases"]])
    q = _split_heads(qkv[:, :d].reshape(b, s, d), b, s, num_heads, dk)
    k = _split_heads(qkv[:, d:2 * d].reshape(b, s, d), b, s, num_heads, dk)
    v = _split_heads(qkv[:, 2 * d:].reshape(b, s, d), b, s, num_heads, dk)
    if rope is not None:
        q = apply_rope(q, rope[0], rope[1])
        k = apply_rope(k, rope[0], rope[1])
    att = sdpa(q, k, v, scale, mask)
    merged = _merge_heads(att, b, s, num_heads, dk).reshape(b * s, d)
    out = _mm(merged, w[prefix + "W_o.weights"])
    out = out + w[prefix + "W_o.biases"]
    return out.reshape(b, s, d)


def ffn(x, w, prefix):
    """neural_network/_fused_arrays.py:187-222."""
    shape = x.shape
    x2d = x.reshape(-1, shape[-1])
    pre = _mm(x2d, w[prefix + "dense1.weights"])
    pre = pre + w[prefix + "dense1.biases"]
    hidden = gelu(pre)
    out = _mm(hidden, w[prefix + "dense2.weights"])
    out = out + w[prefix + "dense2.biases"]
    return out.reshape(shape)


def block(x, w, i, num_heads, mask, rope=None):
    """neural_network/_fused_arrays.py:251-284: x + MHA(LN1(x)); x + FFN(LN2(x))."""
    p = f"blocks.layers.{i}."
    b, s, d = x.shape
    n1 = rmsnorm(x.reshape(b * s, d), w[p + "ln1.gamma"]).reshape(x.shape)
    x_mid = x + mha(n1, w, p + "mha.", num_heads, mask, rope)
    n2 = rmsnorm(x_mid.reshape(b * s, d), w[p + "ln2.gamma"]).reshape(x.shape)
    return x_mid + ffn(n2, w, p + "ffn.")


def hidden_states(w, ids, num_heads, num_layers, rope=None):
    """models/gpt.py:76-90 (``fused_blocks=True``, no fused trunk); rope = the (cos, sin)
    cache of a ``use_rope=True`` model, which has no pos_emb."""
    if rope is not None and np.asarray(ids).shape[1] > rope[0].shape[0]:
        raise ValueError("Sequence length exceeds maximum sequence length")
    x = embed(w["token_emb.weights"], None if rope is not None else w["pos_emb.weights"], ids)
    mask = causal_mask(x.shape[1], x.dtype)
    for i in range(num_layers):
        x = block(x, w, i, num_heads, mask, rope)
    b, s, d = x.shape
    return rmsnorm(x.reshape(b * s, d), w["ln.gamma"]).reshape(x.shape)


def tied_logits(h, emb):
    """models/gpt.py:139-153: ``h2d @ swapaxes(E)`` → (B, S, V)."""
    b, s, d = h.shape
    return _mm(h.reshape(b * s, d), np.swapaxes(emb, -2, -1)).reshape(b, s, emb.shape[0])


def forward(w, ids, num_heads, num_layers, rope=None):
    """``GPT.forward`` (models/gpt.py:92-121): all-position logits (B, S, V)."""
    return tied_logits(hidden_states(w, ids, num_heads, num_layers, rope), w["token_emb.weights"])


def crossentropy(logits, labels):
    """kernels/fused_crossentropy.py:14-30: mean(max + log Σexp(l-max) − l[y])."""
    n = logits.shape[0]
    labels = np.asarray(labels, dtype=np.int64).reshape(-1)
    if labels.size != n:
        raise ValueError(f"label count ({labels.size}) must match batch size ({n}).")
    acc = np.float32 if logits.dtype == np.float16 else logits.dtype
    max_vals = np.max(logits, axis=1, keepdims=True)
    shifted = logits - max_vals
    sum_exp = np.sum(np.exp(shifted), axis=1, keepdims=True, dtype=acc)
    lse = max_vals.ravel().astype(acc, copy=False) + np.log(sum_exp.ravel())
    correct = logits[np.arange(n, dtype=np.int64), labels]
    per_sample = lse - correct
    return float(np.sum(per_sample) / n)


def compute_loss(w, ids, labels, num_heads, num_layers, ignore_index=None, rope=None):
    """``GPT.compute_loss`` (models/gpt.py:123-137) → ``forward_tied``
    (losses/cross_entropy.py:109-148) → kernels/fused_tied_crossentropy.py:8-24.
    ``ignore_index`` rows are dropped first (losses/_ce_prepare.py:46-69)."""
    h = hidden_states(w, ids, num_heads, num_layers, rope)
    b, s, d = h.shape
    h2d = h.reshape(b * s, d)
    labels = np.asarray(labels, dtype=np.int64).reshape(-1)
    if labels.size != b * s:
        raise ValueError(f"label count ({labels.size}) must match batch size ({b * s}).")
    if ignore_index is not None:
        valid = labels != ignore_index
        if not bool(np.any(valid)):
            return 0.0
        h2d, labels = h2d[valid], labels[valid]
    emb = w["token_emb.weights"]
    logits = _mm(h2d, np.swapaxes(emb, -2, -1))
    return crossentropy(logits, labels)


# ----------------------------------------------------------------------- sampling
def choice_from_uniform(p, u):
    """``RandomState.choice(len(p), p=p)`` given its one uniform draw ``u``:
    float64 cumsum, normalised by its last entry, ``searchsorted(u, 'right')``."""
    cdf = np.asarray(p, dtype=np.float64).cumsum()
    cdf /= cdf[-1]
    return int(cdf.searchsorted(u, side="right"))


def apply_repetition_penalty(logits, token_ids, penalty):
    """models/generate.py:9-20."""
    if penalty == 1.0 or not token_ids:
        return logits
    out = logits.copy()
    for tid in {int(t) for t in token_ids}:
        if 0 <= tid < out.size:
            if out[tid] < 0:
                out[tid] *= penalty
            else:
                out[tid] /= penalty
    return out


def sample_logits(logits_1d, *, temperature, top_k, top_p, u=None, token_ids=None,
                  repetition_penalty=1.0):
    """models/generate.py:23-59 with the RNG draw supplied as ``u``."""
    logits = np.asarray(logits_1d, dtype=np.float32).reshape(-1)
    if token_ids:
        logits = apply_repetition_penalty(logits, token_ids, repetition_penalty)
    if temperature <= 0:
        return int(np.argmax(logits))
    logits = logits / float(temperature)
    if top_k and top_k > 0:
        k = min(top_k, logits.size)
        thresh = np.partition(logits, -k)[-k]
        logits = np.where(logits < thresh, -1e9, logits)
    probs = np.exp(logits - np.max(logits))
    probs = probs / np.sum(probs)
    if top_p and 0.0 < top_p < 1.0:
        order = np.argsort(probs)[::-1]
        sorted_p = probs[order]
        cdf = np.cumsum(sorted_p)
        mask = cdf > top_p
        mask[0] = False
        sorted_p = np.where(mask, 0.0, sorted_p)
        sorted_p = sorted_p / np.sum(sorted_p)
        return int(order[choice_from_uniform(sorted_p, u)])
    return choice_from_uniform(probs, u)


def generate(w, ids, num_heads, num_layers, *, max_new_tokens=64, temperature=0.8, top_k=0,
             top_p=0.9, eos_id=None, repetition_penalty=1.0, uniforms=None, rope=None):
    """models/generate.py:62-119 for a model without ``forward_with_cache`` (the
    reference ``GPT``): every step re-forwards the whole sequence and samples each
    row from its last-position logits. ``uniforms[t][b]`` replaces the t-th step's
    draw for row b (the reference draws them from NumPy's global legacy RNG in
    that order)."""
    ids = np.asarray(ids, dtype=np.int64)
    if ids.ndim == 1:
        ids = ids.reshape(1, -1)
    batch = ids.shape[0]
    generated = [list(ids[b].tolist()) for b in range(batch)]
    for t in range(max_new_tokens):
        cur = np.asarray(generated, dtype=np.int64)
        logits = forward(w, cur, num_heads, num_layers, rope)
        for b in range(batch):
            u = None if uniforms is None else uniforms[t][b]
            tok = sample_logits(logits[b, -1], temperature=temperature, top_k=top_k, top_p=top_p,
                                u=u, token_ids=generated[b],
                                repetition_penalty=repetition_penalty)
            generated[b].append(tok)
        if eos_id is not None and all(generated[b][-1] == eos_id for b in range(batch)):
            break
    return np.asarray(generated, dtype=np.int64)


# ------------------------------------------------------- incremental (KV) variant
class KVOracle:
    """Incremental decode with a per-layer K/V cache, fp32 or fp16.

    Not a reference code path (the reference GPT has no ``forward_with_cache``):
    it is the same arithmetic per position, pinned against :func:`forward` by the
    invariant that causal attention makes row t of a full re-forward depend only
    on tokens 0..t. Used where a full re-forward per token is too slow.
    """

    def __init__(self, w, num_heads, num_layers, rope=None):
        self.w = w
        self.rope = rope
        self.h = num_heads
        self.n_layers = num_layers
        self.k = [None] * num_layers  # (B*H, t, dk)
        self.v = [None] * num_layers
        self.t = 0
        self._qkv = {}  # layer → (stacked W, stacked b); the same values every step

    def _stacked(self, i):
        if i not in self._qkv:
            w, p = self.w, f"blocks.layers.{i}."
            self._qkv[i] = (
                np.concatenate([w[p + "mha.W_q.weights"], w[p + "mha.W_k.weights"],
                                w[p + "mha.W_v.weights"]], axis=1),
                np.concatenate([w[p + "mha.W_q.biases"], w[p + "mha.W_k.biases"],
                                w[p + "mha.W_v.biases"]]))
        return self._qkv[i]

    def step(self, ids):
        """Feed ``ids`` (B, s) at positions t..t+s-1; return logits (B, s, V)."""
        w = self.w
        ids = np.asarray(ids, dtype=np.int64)
        b, s = ids.shape
        x = w["token_emb.weights"][ids.reshape(-1)].reshape(b, s, -1)
        if self.rope is None:
            x = x + w["pos_emb.weights"][self.t:self.t + s]
        d = x.shape[-1]
        dk = d // self.h
        scale = float(dk) ** 0.5
        total = self.t + s
        mask = np.triu(np.full((total, total), -np.inf, dtype=x.dtype), k=1)[self.t:total]
        for i in range(self.n_layers):
            p = f"blocks.layers.{i}."
            n1 = rmsnorm(x.reshape(b * s, d), w[p + "ln1.gamma"])
            w_qkv, b_qkv = self._stacked(i)
            qkv = _mm(n1, w_qkv) + b_qkv
            q = _split_heads(qkv[:, :d], b, s, self.h, dk)
            k = _split_heads(qkv[:, d:2 * d], b, s, self.h, dk)
            v = _split_heads(qkv[:, 2 * d:], b, s, self.h, dk)
            if self.rope is not None:
                q = apply_rope(q, self.rope[0], self.rope[1], self.t)
                k = apply_rope(k, self.rope[0], self.rope[1], self.t)
            self.k[i] = k if self.k[i] is None else np.concatenate([self.k[i], k], axis=1)
            self.v[i] = v if self.v[i] is None else np.concatenate([self.v[i], v], axis=1)
            att = sdpa(q, self.k[i], self.v[i], scale, mask)
            merged = _merge_heads(att, b, s, self.h, dk).reshape(b * s, d)
            x = x + (_mm(merged, w[p + "mha.W_o.weights"]) + w[p + "mha.W_o.biases"]).reshape(b, s, d)
            n2 = rmsnorm(x.reshape(b * s, d), w[p + "ln2.gamma"]).reshape(b, s, d)
            x = x + ffn(n2, w, p + "ffn.")
        self.t = total
        h = rmsnorm(x.reshape(b * s, d), w["ln.gamma"]).reshape(b, s, d)
        return tied_logits(h, w["token_emb.weights"])


class RaggedKVOracle:
    """Rows of different lengths decoded in lockstep, one :class:`KVOracle` per row.

    Each row is prefilled on its own, as the reference runs one sequence at a time. A
    decode step then feeds one token per row and runs the row-independent ops (GEMMs,
    RMSNorm, GELU, the tied head) on all rows at once; attention runs per row over its
    own cache. NumPy computes every row of those ops as it would at batch 1, so each
    row's logits equal its own batch-1 :class:`KVOracle` (pinned by a test)."""

    def __init__(self, w, num_heads, num_layers):
        self.w = w
        self.h = num_heads
        self.n_layers = num_layers
        self.rows = []

    def prefill(self, rows):
        """``rows``: list of 1-D id arrays. Returns the last-position logits (B, V)."""
        out = []
        self.rows = []
        for r in rows:
            kv = KVOracle(self.w, self.h, self.n_layers)
            out.append(kv.step(np.asarray(r, dtype=np.int64).reshape(1, -1))[0, -1])
            self.rows.append(kv)
        return np.stack(out)

    def step(self, tokens):
        """Feed one token per row (B,); return the logits (B, V)."""
        w = self.w
        tokens = np.asarray(tokens, dtype=np.int64).reshape(-1)
        B = tokens.size
        pos = np.asarray([kv.t for kv in self.rows])
        x = w["token_emb.weights"][tokens] + w["pos_emb.weights"][pos]
        d = x.shape[-1]
        dk = d // self.h
        scale = float(dk) ** 0.5
        for i in range(self.n_layers):
            p = f"blocks.layers.{i}."
            n1 = rmsnorm(x, w[p + "ln1.gamma"])
            w_qkv, b_qkv = self.rows[0]._stacked(i)
            qkv = _mm(n1, w_qkv) + b_qkv
            merged = np.empty_like(x)
            for b, kv in enumerate(self.rows):
                q = _split_heads(qkv[b:b + 1, :d], 1, 1, self.h, dk)
                k = _split_heads(qkv[b:b + 1, d:2 * d], 1, 1, self.h, dk)
                v = _split_heads(qkv[b:b + 1, 2 * d:], 1, 1, self.h, dk)
                kv.k[i] = np.concatenate([kv.k[i], k], axis=1)
                kv.v[i] = np.concatenate([kv.v[i], v], axis=1)
                total = kv.t + 1
                mask = np.triu(np.full((total, total), -np.inf, dtype=x.dtype), k=1)[kv.t:total]
                att = sdpa(q, kv.k[i], kv.v[i], scale, mask)
                merged[b] = _merge_heads(att, 1, 1, self.h, dk).reshape(d)
            x = x + (_mm(merged, w[p + "mha.W_o.weights"]) + w[p + "mha.W_o.biases"])
            n2 = rmsnorm(x, w[p + "ln2.gamma"])
            x = x + ffn(n2, w, p + "ffn.")
        for kv in self.rows:
            kv.t += 1
        h = rmsnorm(x, w["ln.gamma"])
        return tied_logits(h.reshape(B, 1, d), w["token_emb.weights"])[:, 0]


# ------------------------------------------------------------ decision robustness
def sample_flip_tol(logits, u, token, *, temperature, top_k):
    """Largest ε such that changing every logit by at most ε provably cannot change
    ``token``, the pick of ``sample_logits(logits, temperature, top_k, top_p=1, u)`` (no
    repetition penalty). With η = ε/T the bound on each scaled logit's move: a kept token
    and a dropped one can trade places only if their scaled logits are within 2η, so the
    top-k set can change only among tokens whose scaled logit lies in
    [v_k − 2η, v_{k+1} + 2η] (v_k the k-th largest, v_{k+1} the next; no change at all
    when v_k − v_{k+1} > 2η),
    and their probability mass — kept or joining, each at most e^{2η} times its present
    share — may then shift the CDF; every CDF value c also moves by at most
    c(1 − c)(e^{2η} − 1) from the common rescaling. The pick must stay strictly inside its
    CDF interval under both, and may not itself be one of the tokens that can leave.
    Greedy (temperature ≤ 0): half the top-2 gap."""
    x = np.asarray(logits, dtype=np.float32).reshape(-1).astype(np.float64)
    if temperature <= 0:
        top2 = np.sort(x)[-2:]
        return float(top2[1] - top2[0]) / 2.0
    xt = np.asarray(logits, dtype=np.float32).reshape(-1) / np.float32(temperature)
    k = min(top_k, xt.size) if top_k and top_k > 0 else xt.size
    th = float(np.partition(xt, -k)[-k])
    keep = xt >= th
    p = np.exp((xt - xt[keep].max()).astype(np.float64)) * keep
    z = p.sum()
    p /= z
    cdf = np.cumsum(p)
    j = int(token)
    lo = cdf[j - 1] if j > 0 else 0.0
    hi = cdf[j]
    if not (lo <= u < hi):
        return 0.0
    xt64 = xt.astype(np.float64)
    share = np.exp(xt64 - float(xt[keep].max())) / z  # present share of every token
    srt = np.sort(xt64)[::-1]
    vk = srt[k - 1]
    vk1 = srt[k] if k < xt.size else -np.inf

    def robust(eps):
        e = 2.0 * eps / float(temperature)  # 2η
        # the window, widened by the float32 roundings of the perturbed logits and of the
        # division by T in the reference's sampler (a few ulps of the scaled logits)
        w = e + 1e-6 * max(1.0, abs(vk))
        mass = 0.0
        if k < xt.size and vk - vk1 <= w:
            amb = (xt64 >= vk - w) & (xt64 <= vk1 + w)
            if amb[j]:
                return False
            mass = share[amb].sum() * np.exp(e)

        def shift(c):  # |Δc| for a CDF value c (+ float32 rounding of the probabilities)
            return c * (1.0 - c) * (np.exp(e) - 1.0) + mass + 1e-6

        return (u - lo) > shift(lo) and (hi - u) > shift(hi)

    if not robust(0.0):
        return 0.0
    a, b = 0.0, 1.0
    if robust(b):
        return b
    for _ in range(40):
        mid = 0.5 * (a + b)
        if robust(mid):
            a = mid
        else:
            b = mid
    return a
