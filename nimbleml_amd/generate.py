"""Autoregressive generation on the GPU (models/generate.py:62-119).

Same signature and results as the reference: greedy when ``temperature <= 0``,
otherwise temperature, top-k, top-p and repetition penalty exactly as
``_sample_logits`` (generate.py:23-59). The loop runs on the device — prefill,
then one decode step per token over the KV cache, with the choice made on the
device — and the host sees the tokens once, at the end.

Randomness: the reference draws one uniform per row per step from NumPy's
global legacy generator (``np.random.choice``, generate.py:57,59), rows in
order within a step. Here the same ``max_new_tokens × batch`` draws are taken
up front from that generator (``np.random.random_sample``) and consumed in that
order on the device, so a seeded run gives the reference's tokens. With ``eos_id``
the reference stops drawing at the eos step; the global generator is then rewound
to the state those fewer draws leave, so later draws of the caller agree too.

Ragged batches: ``input_ids`` may be a list of rows of different lengths; each
row then generates as if run alone (the result is a list of arrays).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from nimbleml_amd import _native as N
from nimbleml_amd.tensor import Tensor


def _rows(input_ids):
    if isinstance(input_ids, Tensor):
        arr = np.asarray(input_ids.data, dtype=np.int64).reshape(input_ids.shape)
        return [r for r in np.atleast_2d(arr)], False
    if isinstance(input_ids, np.ndarray):
        arr = np.asarray(input_ids, dtype=np.int64)
        return [r for r in np.atleast_2d(arr)], False
    rows = list(input_ids)
    if rows and np.ndim(rows[0]) == 0:
        return [np.asarray(rows, dtype=np.int64)], False
    rows = [np.asarray(r, dtype=np.int64).reshape(-1) for r in rows]
    ragged = len({len(r) for r in rows}) > 1
    return rows, ragged


def generate(model, input_ids, *, max_new_tokens: int = 64, temperature: float = 0.8,
             top_k: int = 0, top_p: float = 0.9, eos_id=None, repetition_penalty: float = 1.0,
             use_kv_cache: bool = True, use_graph: bool = True):
    from nimbleml_amd.gpt import GPT

    if not isinstance(model, GPT):
        raise TypeError("nimbleml_amd.generate drives nimbleml_amd.GPT models")
    rows, ragged = _rows(input_ids)
    batch = len(rows)
    n = int(max_new_tokens)
    if batch == 0 or n <= 0:
        return rows if ragged else np.asarray(rows, dtype=np.int64).reshape(batch, -1)
    for r in rows:
        if r.size == 0:
            raise ValueError("prompts must not be empty")
        if int(r.min()) < 0 or int(r.max()) >= model.vocab_size:
            raise ValueError(f"Token ID out of range [0, {model.vocab_size})")
    plen = np.asarray([len(r) for r in rows], dtype=np.int32)
    longest = int(plen.max())
    if longest + n - 1 > model.max_seq_len:
        raise ValueError(f"Sequence length {longest + n - 1} exceeds maximum sequence length "
                         f"{model.max_seq_len}")

    sampling = temperature > 0
    rng_state = np.random.get_state() if sampling else None
    u = np.random.random_sample((n, batch)) if sampling else None

    if use_kv_cache:
        tokens = _generate_device(model, rows, plen, n, temperature, top_k, top_p,
                                  repetition_penalty, u, use_graph)
    else:
        tokens = _generate_reforward(model, rows, plen, n, temperature, top_k, top_p,
                                     repetition_penalty, u)

    # eos: the reference stops after the first step at which every row emitted eos.
    steps = n
    if eos_id is not None:
        for t in range(n):
            if all(int(tokens[b, plen[b] + t]) == eos_id for b in range(batch)):
                steps = t + 1
                break
    if sampling and steps < n:
        # the reference drew one uniform per row per step only up to the eos step
        # (generate.py:116-117): leave the global generator where its draws end
        np.random.set_state(rng_state)
        np.random.random_sample((steps, batch))
    out = [tokens[b, :plen[b] + steps].copy() for b in range(batch)]
    return out if ragged else np.asarray(out, dtype=np.int64)


def _generate_device(model, rows, plen, n, temperature, top_k, top_p, penalty, u, use_graph):
    h = model._device_model()
    batch = len(rows)
    stride = int(plen.max())
    prompts = np.zeros((batch, stride), dtype=np.int64)
    for b, r in enumerate(rows):
        prompts[b, :len(r)] = r
    out_stride = stride + n
    dprompt = N.DeviceArray.from_host(prompts)
    dtok = N.DeviceArray((batch, out_stride), np.int64)
    du = N.DeviceArray.from_host(np.ascontiguousarray(u, dtype=np.float64)) if u is not None else None
    plen_c = np.ascontiguousarray(plen, dtype=np.int32)
    N.check(N.lib.nml_model_generate(
        h, dprompt.ptr, stride, plen_c.ctypes.data_as(N.PI32), batch, n, float(temperature),
        int(top_k or 0), float(top_p if top_p is not None else 1.0), float(penalty),
        du.ptr if du is not None else None, dtok.ptr, out_stride, int(bool(use_graph))))
    return dtok.numpy()


def _generate_reforward(model, rows, plen, n, temperature, top_k, top_p, penalty, u):
    """use_kv_cache=False: re-forward the whole sequence for every token, as the
    reference does for models without ``forward_with_cache``; the choice is made
    on the device from the last-position logits."""
    batch = len(rows)
    if len(set(plen.tolist())) != 1:
        raise ValueError("use_kv_cache=False needs prompts of equal length")
    seq = np.asarray(rows, dtype=np.int64)
    dt = N.np_dtype_code(model._dtype)
    du = N.DeviceArray.from_host(np.ascontiguousarray(u, dtype=np.float64)) if u is not None else None
    out_ids = N.DeviceArray((batch,), np.int64)
    for t in range(n):
        logits = model.forward_last(seq).data
        hist = N.DeviceArray.from_host(seq)
        hl = N.DeviceArray.from_host(np.full(batch, seq.shape[1], dtype=np.int32))
        uptr = (du.ptr + t * batch * 8) if du is not None else None
        N.check(N.lib.nml_sample_device(logits.ptr, batch, model.vocab_size, float(temperature),
                                        int(top_k or 0), float(top_p if top_p is not None else 1.0),
                                        float(penalty), uptr, hist.ptr, seq.shape[1], hl.ptr,
                                        out_ids.ptr, dt))
        seq = np.concatenate([seq, out_ids.numpy().reshape(batch, 1)], axis=1)
    return seq
