"""Benchmark: generated tokens/s of NimbleML's GPT token loop on one MI355X.

Headline workload ("C3"): GPT vocab 32000, d_model 1024,
16 heads, 24 layers, MLP 4x GELU, RMSNorm, max_seq_len 2048, fp16 weights ~N(0, 0.02)
(seeded, synthetic), batch 1, prompt of 512 uniform ids, greedy decode of 512 new
tokens. One step = one whole generate() call (prefill + 511 decode steps, each one
launch of the persistent decode kernel with the greedy choice fused), inputs resident
on the device when the timed region starts. `value` = generated tokens / wall time.

`roofline` is for that dominant kernel (one launch per decode token): algorithmic
bytes per launch = every weight once, 2·(L·(12d²+11d) + V·d + d) B, plus the K/V cache
read, 2·2·L·d·ctx B, and written, 2·2·L·d B, averaged over the run's contexts
513…1023; divided by the kernel's average duration, measured with HIP events on the
library stream around the decode loop. `traffic` (HBM bytes per launch) comes from
the committed rocprofv3 PMC summary profiles/c3_decode_b1_pmc.md when present.

Two more lines of the same metric ride along (BASELINE.json "batch 1 & 32"):
  c4: batch 32, prompts U[128,1024], 256 sampled tokens each (T=0.8, top-k 50), HBM
      roofline of the decode step (weights once + every row's K/V);
  c5: d2048/L24/V50304 fp16, 4×4096 causal prefill + tied cross-entropy over all
      16384 positions (compute_loss), MFMA roofline (49.56 TFLOP algorithmic).
`cpu_baseline` times the oracle (the reference algorithm restated: full re-forward per
token, host sampling; fp32 because NumPy fp16 has no BLAS path) on a bounded sample:
C3 tokens spread over the run's contexts; c4 and c5 carry their own (c4: a few rows at
batch 1, as the reference runs ragged prompts; c5: one block and the head on one
sequence, extrapolated). `cpu_baseline_fp16` is the same algorithm in the reference's
fp16 arithmetic, truncated to one layer at the run's first and last contexts plus the
head and extrapolated (labelled so).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "generated tokens/sec + % HBM/MFMA roofline, d1024 L24 fp16 GPT, batch 1 & 32"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
PMC_SUMMARY = os.path.join(REPO, "profiles", "c3_decode_b1_pmc.md")


def weight_bytes(cfg, es=2):
    d, L, V = cfg.d_model, cfg.num_layers, cfg.vocab_size
    return es * (L * (12 * d * d + 11 * d) + V * d + d)


def kv_bytes(cfg, ctx, es=2):
    """K/V read over `ctx` keys plus the new key/value written, all layers."""
    return 2 * es * cfg.num_layers * cfg.d_model * (ctx + 1)


def pmc_traffic():
    """HBM bytes per decode launch from the committed PMC summary, if any."""
    try:
        text = open(PMC_SUMMARY).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", text)
    return float(m.group(1)) if m else None


def cpu_threads():
    try:
        from threadpoolctl import threadpool_info

        return max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        return os.cpu_count() or 1


def cpu_baseline(cfg, w16, prompt, n_new, samples):
    """Reference algorithm on the host (oracle): fp32, full re-forward per token.

    The reference's cost per generated token grows with the context, so the sample
    spreads `samples` tokens evenly over the run's contexts prompt … prompt + n_new - 1
    (each one generate step: a full forward over the context and the greedy choice) and
    reports their mean rate, the rate of the whole run to within the sampling."""
    from oracle import gpt_ref as R

    w = {k: v.astype(np.float32) for k, v in w16.items()}
    s0 = prompt.shape[1]
    ctxs = np.linspace(s0, s0 + n_new - 1, samples).round().astype(int)
    rng = np.random.default_rng(4)
    ids = np.concatenate([prompt, rng.integers(0, cfg.vocab_size, (1, n_new), dtype=np.int64)], axis=1)
    t0 = time.perf_counter()
    for c in ctxs:
        R.generate(w, ids[:, :c], cfg.num_heads, cfg.num_layers, max_new_tokens=1, temperature=0.0)
    dt = time.perf_counter() - t0
    return {"value": round(len(ctxs) / dt, 4), "unit": "tokens/s", "cores": int(cpu_threads()),
            "kind": "port",
            "sample": f"C3 shapes at fp32, batch 1: {len(ctxs)} greedy tokens at contexts "
                      f"{ctxs[0]}..{ctxs[-1]} evenly spread over the run's {s0}..{s0 + n_new - 1}, "
                      f"each a full re-forward as the reference does ({dt:.1f} s)"}


def cpu_baseline_fp16(cfg, w16, prompt, n_new):
    """The reference algorithm in its own fp16 arithmetic (oracle, every op rounded to fp16
    as NumPy does), truncated: one re-forward token costs L blocks over the context plus
    the last row's tied head. Timed here: layer 0 over the run's first and last contexts
    (prompt and prompt + n_new − 1 tokens) and the head; the per-token cost of the run is
    extrapolated as L × the mean block time + the head. The fp16 products go through the
    oracle's C restatement of NumPy's fp16 matmul loop (bit-exact; NumPy's own loop, the
    reference's, is about two orders of magnitude slower still)."""
    from oracle import gpt_ref as R

    s0 = prompt.shape[1]
    rng = np.random.default_rng(4)
    ids = np.concatenate([prompt, rng.integers(0, cfg.vocab_size, (1, n_new), dtype=np.int64)],
                         axis=1)
    blocks = []
    for c in (s0, s0 + n_new - 1):
        x = R.embed(w16["token_emb.weights"], w16["pos_emb.weights"], ids[:, :c])
        t0 = time.perf_counter()
        y = R.block(x, w16, 0, cfg.num_heads, R.causal_mask(c, x.dtype))
        blocks.append(time.perf_counter() - t0)
    t0 = time.perf_counter()
    h = R.rmsnorm(y[0, -1:], w16["ln.gamma"])
    R._mm(h, np.swapaxes(w16["token_emb.weights"], -2, -1))
    head = time.perf_counter() - t0
    per_token = cfg.num_layers * float(np.mean(blocks)) + head
    return {"value": round(1.0 / per_token, 5), "unit": "tokens/s", "cores": int(cpu_threads()),
            "kind": "port", "extrapolated": True,
            "sample": f"C3 at fp16 (the reference's fp16 rounding): layer 0 re-forwarded over "
                      f"{s0} and {s0 + n_new - 1} tokens ({blocks[0]:.1f} s, {blocks[1]:.1f} s) and "
                      f"the last row's tied head ({head:.2f} s), extrapolated to {cfg.num_layers} "
                      f"layers per generated token ({per_token:.1f} s per token)"}


def bench_c3(nm, cfg, model, prompt, n, steps, warmup, use_graph):
    kw = dict(max_new_tokens=n, temperature=0.0, use_graph=use_graph)
    for _ in range(warmup):
        nm.generate(model, prompt, **kw)
    nm._native.synchronize()
    decode_ms = []
    t0 = time.perf_counter()
    for _ in range(steps):
        out = nm.generate(model, prompt, **kw)
        decode_ms.append(model.last_decode_ms())
    nm._native.synchronize()
    elapsed = time.perf_counter() - t0
    assert out.shape == (1, prompt.shape[1] + n)
    ctxs = np.arange(prompt.shape[1] + 1, prompt.shape[1] + n)
    bytes_avg = float(np.mean([weight_bytes(cfg) + kv_bytes(cfg, c) for c in ctxs]))
    step_ms = float(np.mean(decode_ms))
    return elapsed, step_ms, bytes_avg, model.last_decode_persistent()


def cpu_baseline_c4(cfg, w16, rows, new, samples=4):
    """Reference algorithm on the host for a bounded sample of C4: the reference cannot
    batch ragged prompts, so each row generates at batch 1 (full re-forward per token,
    temperature 0.8, top-k 50); `samples` rows take one sampled token each at a context
    spread over their own run, and the rate is that of one row after another."""
    from oracle import gpt_ref as R

    w = {k: v.astype(np.float32) for k, v in w16.items()}
    rng = np.random.default_rng(6)
    t0 = time.perf_counter()
    for i in range(samples):
        row = np.asarray(rows[i], dtype=np.int64)
        extra = int(round(i * (new - 1) / max(1, samples - 1)))
        ids = np.concatenate([row, rng.integers(0, cfg.vocab_size, extra)])[None, :]
        u = np.random.RandomState(i).random_sample()  # the reference's legacy-RNG draw
        R.generate(w, ids, cfg.num_heads, cfg.num_layers, max_new_tokens=1, temperature=0.8,
                   top_k=50, top_p=1.0, uniforms=[[u]])
    dt = time.perf_counter() - t0
    return {"value": round(samples / dt, 4), "unit": "tokens/s", "cores": int(cpu_threads()),
            "kind": "port",
            "sample": f"C4 rows 0..{samples - 1} at fp32, batch 1 each (the reference cannot batch "
                      f"ragged prompts), one sampled token per row at contexts spread over its "
                      f"{new} steps, full re-forward per token ({dt:.1f} s)"}


def bench_c4(nm, cfg, model, use_graph, reps=2, w16=None, uniform=False):
    """C4 line: one warm-up generate() and `reps` timed ones (reps 0: the warm-up only,
    for counter passes). uniform: every prompt at the ragged prompts' mean length (the
    same decode kernels and per-step bytes, through the uniform prefill path)."""
    rng = np.random.default_rng(5)
    lens = rng.integers(128, 1025, 32)
    if uniform:
        lens = np.full(32, int(round(lens.mean())))
    rows = [rng.integers(0, cfg.vocab_size, int(n)) for n in lens]
    new = 256
    kw = dict(max_new_tokens=new, temperature=0.8, top_k=50, top_p=1.0, use_graph=use_graph)
    np.random.seed(0)
    nm.generate(model, rows, **kw)  # warm-up
    nm._native.synchronize()
    if reps == 0:
        return {"workload": "C4 warm-up generate() only (counter pass)",
                "decode_ms_per_step": round(model.last_decode_ms(), 4)}
    t0 = time.perf_counter()
    decode_ms = []
    for _ in range(reps):
        np.random.seed(0)
        nm.generate(model, rows, **kw)
        decode_ms.append(model.last_decode_ms())
    nm._native.synchronize()
    elapsed = (time.perf_counter() - t0) / reps
    # decode step s (1 … new-1) attends len_b + s keys in every row
    bytes_steps = [weight_bytes(cfg) + sum(kv_bytes(cfg, int(n) + s - 1) for n in lens)
                   for s in range(1, new)]
    step_ms = float(np.mean(decode_ms))
    achieved = float(np.mean(bytes_steps)) / (step_ms * 1e-3) / 1e9
    base = cpu_baseline_c4(cfg, w16, rows, new) if w16 is not None else None
    return {**({"cpu_baseline": base} if base else {}),
            "workload": "C4: same model, batch 32, prompts U[128,1024], 256 sampled tokens each "
                        "(T=0.8, top-k 50, top_p 1.0)",
            "value": round(32 * new / elapsed, 1), "unit": "tokens/s",
            "ms_per_generate": round(elapsed * 1e3, 2), "decode_ms_per_step": round(step_ms, 4),
            "roofline": {"bound": "hbm", "kernel": "decode step (all kernels of one token)",
                         "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4)}}


def bench_adamw(nm, n=337_100_000, steps=20):
    """AdamW over one float32 buffer the size of the C3 model (337.1 M parameters): the
    step reads param, grad, m, v and writes param, m, v — 28 B per element."""
    N = nm._native
    from nimbleml_amd import kernels as K

    bufs = [N.DeviceArray((n,), np.float32) for _ in range(4)]
    for b, val in zip(bufs, (1, 0, 0, 0)):
        N.check(N.lib.nml_memset(b.ptr, val, b.nbytes))
    p, g, m, v = bufs
    args = (1e-3, 0.9, 0.999, 0.1, 0.001, 1e-8, 0.01)
    K.adamw_step(p, g, m, v, *args)
    N.synchronize()
    t = N.Timer()
    t.start()
    for _ in range(steps):
        K.adamw_step(p, g, m, v, *args)
    ms = t.stop() / steps
    gbs = 28.0 * n / (ms * 1e-3) / 1e9
    return {"workload": "AdamW step, float32 state, 337.1 M parameters (the C3 model's count)",
            "ms_per_step": round(ms, 4), "elements": n,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes_per_element": 28}}


MFMA_F32_PEAK_TFLOPS = 157.3


def bench_train(nm, batch=4, seq=1024, steps=3, dtype=np.float32, skew=False):
    """One training step of the C3 architecture in float32: zero_grad, compute_loss keeping
    the activations (nml_model_loss_train), loss.backward() into the device gradients
    (nml_model_backward) and AdamW over every parameter (nml_model_adamw_step), batch × seq
    tokens. Algorithmic flops: 3× the forward's
    (GEMMs 2·rows·12·d²·L + head 2·rows·d·V, attention 4·d·S(S+1)/2 per sequence and
    layer), i.e. without the backward's recomputation of the logits and scores."""
    import ctypes as C

    from oracle.weights import C3, make_weights, random_ids

    N = nm._native
    cfg = C3
    w = make_weights(cfg, seed=11, dtype=dtype)
    model = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, dtype=dtype)
    del w
    h = model._device_model()
    ids_h = random_ids((batch, seq), cfg.vocab_size, seed=3)
    if skew:  # half of the positions hold one id (a pad token): the embedding scatter's worst case
        ids_h.reshape(-1)[::2] = 7
    ids = N.DeviceArray.from_host(ids_h)
    lab = N.DeviceArray.from_host(random_ids((batch * seq,), cfg.vocab_size, seed=4))
    loss = C.c_double()
    t_step = [0]

    def step():
        t_step[0] += 1
        t = t_step[0]
        N.check(N.lib.nml_model_zero_grad(h))
        N.check(N.lib.nml_model_loss_train(h, ids.ptr, lab.ptr, batch, seq, 0, 0, C.byref(loss)))
        N.check(N.lib.nml_model_backward(h, 1.0))
        N.check(N.lib.nml_model_adamw_step(h, 1e-4, 0.9, 0.999, 1 - 0.9 ** t, 1 - 0.999 ** t,
                                           1e-8, 0.01))

    step()  # warm-up (allocates the saved activations)
    t = N.Timer()
    t.start()
    for _ in range(steps):
        step()
    ms = t.stop() / steps
    d, L, V, R = cfg.d_model, cfg.num_layers, cfg.vocab_size, batch * seq
    fwd = 2 * R * L * 12 * d * d + L * batch * 4 * d * seq * (seq + 1) / 2 + 2 * R * d * V
    tf = 3 * fwd / (ms * 1e-3) / 1e12
    name = "float32" if dtype == np.float32 else "float16 (float32 gradients and masters)"
    # the peak of the GEMMs' arithmetic: fp32 MFMA, or fp16 MFMA for a float16 model (whose
    # attention backward still runs on the fp32 MFMA, from fp16 operands)
    peak = MFMA_F32_PEAK_TFLOPS if dtype == np.float32 else MFMA_F16_PEAK_TFLOPS
    return {"workload": f"train step: GPT V32000 d1024 H16 L24 {name}, batch {batch} x {seq}, "
                        "zero_grad + compute_loss + backward + AdamW on the device"
                        + (" (half of the ids one token)" if skew else ""),
            "value": round(R / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 3),
            "loss": round(loss.value, 5),
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": peak,
                         "unit": "TFLOP/s", "frac": round(tf / peak, 4), "flops": 3 * fwd}}


def cpu_baseline_c5(cfg, w16, ids, lab):
    """Reference algorithm on the host (oracle, fp32: NumPy fp16 has no BLAS path) for a
    bounded sample of C5: layer 0 of the first sequence (the reference's full (S, S)
    scores), then the tied logits and cross-entropy of that sequence's 4096 positions;
    the whole compute_loss is extrapolated as B·(L·block + head)."""
    from oracle import gpt_ref as R

    B, S = ids.shape
    w = {k: w16[k].astype(np.float32) for k in w16 if k.startswith("blocks.layers.0.")}
    w["token_emb.weights"] = w16["token_emb.weights"].astype(np.float32)
    w["pos_emb.weights"] = w16["pos_emb.weights"].astype(np.float32)
    w["ln.gamma"] = w16["ln.gamma"].astype(np.float32)
    x = R.embed(w["token_emb.weights"], w["pos_emb.weights"], ids[:1])
    mask = R.causal_mask(S, x.dtype)
    t0 = time.perf_counter()
    x = R.block(x, w, 0, cfg.num_heads, mask)
    t1 = time.perf_counter()
    h = R.rmsnorm(x.reshape(S, -1), w["ln.gamma"])
    R.crossentropy(R._mm(h, np.swapaxes(w["token_emb.weights"], -2, -1)), lab[:1])
    t2 = time.perf_counter()
    total = B * (cfg.num_layers * (t1 - t0) + (t2 - t1))
    return {"value": round(B * S / total, 2), "unit": "positions/s", "cores": int(cpu_threads()),
            "kind": "port", "extrapolated": True,
            "sample": f"C5 shapes at fp32: one block over one 4096-token sequence ({t1 - t0:.1f} s) "
                      f"and its tied head + cross-entropy ({t2 - t1:.1f} s), extrapolated to "
                      f"{B} sequences x {cfg.num_layers} layers ({total:.0f} s per compute_loss)"}


def bench_c5(nm, reps=5, cpu=False):
    from oracle.weights import C5, make_weights, random_ids

    cfg = C5
    w = make_weights(cfg, seed=7, dtype=np.float16)
    model = nm.GPT.from_arrays(w, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, dtype=np.float16)
    ids = random_ids((4, 4096), cfg.vocab_size, seed=1)
    lab = random_ids((4, 4096), cfg.vocab_size, seed=2)
    base = cpu_baseline_c5(cfg, w, ids, lab) if cpu else None
    del w
    model.to_device()
    from nimbleml_amd.grad_mode import no_grad

    with no_grad():  # the loss alone: no activations kept for a backward
        model.compute_loss(ids, lab)  # warm-up
        t0 = time.perf_counter()
        for _ in range(reps):
            loss = model.compute_loss(ids, lab).item()
        dt = (time.perf_counter() - t0) / reps
    d, L, V, B, S = cfg.d_model, cfg.num_layers, cfg.vocab_size, 4, 4096
    flops = 2 * B * S * L * 12 * d * d + L * B * 4 * d * S * (S + 1) / 2 + 2 * B * S * d * V
    tf = flops / dt / 1e12
    return {"workload": "C5: GPT V50304 d2048 H16 L24 fp16, 4x4096 causal prefill + tied "
                        "cross-entropy over 16384 positions (compute_loss)",
            "value": round(B * S / dt, 1), "unit": "positions/s", "seconds": round(dt, 4),
            "loss": round(float(loss), 5),
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                         "flops": flops},
            **({"cpu_baseline": base} if base else {})}


def bench_c4_attention(nm, reps=20):
    """The C4 step's decode attention alone — the kernel the step launches once per layer
    and half — as one launch over all 32 rows and 16 heads, through the C-ABI export
    nml_decode_attention_device: K/V caches of the C4 shape (max 1280 positions, head dim
    64, fp16), every row 128 steps into its 256 (contexts len_b + 128 over the C4
    prompts). HIP events over `reps` launches; bytes are each row's K and V rows read once
    (the query and output rows are 4 KB a row)."""
    N = nm._native
    rng = np.random.default_rng(5)
    lens = (rng.integers(128, 1025, 32) + 128).astype(np.int32)
    B, H, P, dk = 32, 16, 1280, 64
    q = rng.standard_normal((B, H, dk)).astype(np.float16)
    kc = rng.standard_normal((B, H, P, dk), dtype=np.float32).astype(np.float16)
    vc = rng.standard_normal((B, H, P, dk), dtype=np.float32).astype(np.float16)
    dq, dkc, dvc, dl = (N.DeviceArray.from_host(a) for a in (q, kc, vc, lens))
    del kc, vc
    err = N.DeviceArray.from_host(np.zeros(1, np.int32))
    out = N.DeviceArray((B, H * dk), np.float16)
    call = lambda: N.check(N.lib.nml_decode_attention_device(
        dq.ptr, dkc.ptr, dvc.ptr, dl.ptr, out.ptr, B, H, P, dk, ctypes.c_float(8.0), err.ptr,
        N.np_dtype_code(np.float16)))
    call()
    N.synchronize()
    t = N.Timer()
    t.start()
    for _ in range(reps):
        call()
    ms = t.stop() / reps
    N.synchronize()
    if int(err.numpy()[0]) != 0:
        raise RuntimeError("decode attention flagged a length")
    nbytes = int(lens.sum()) * H * dk * 2 * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": "C4 decode attention, one launch: 32 rows x 16 heads, dk 64, fp16, "
                        f"contexts {int(lens.min())}..{int(lens.max())}",
            "us_per_launch": round(ms * 1e3, 2), "bytes_per_launch": nbytes,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}


def bench_c4_projections(nm, reps=50):
    """The C4 step's four projections alone, as the step launches them for one 16-row half
    (d1024 fp16: QKV 1024→3072 + bias, W_o 1024→1024 + bias + residual, W1 1024→4096 +
    bias + GELU, W2 4096→1024 + bias + residual) through the C-ABI export nml_linear_device
    on the skinny MFMA kernel (without the fused RMSNorm of the step's QKV and W1). HIP events
    over `reps` back-to-back launches of each; bytes are the weights read once (the 16 input
    and output rows are 32–128 KB)."""
    N = nm._native
    rng = np.random.default_rng(7)
    rows = 16
    out = {}
    for name, k, n, epi in (("qkv", 1024, 3072, 1), ("w_o", 1024, 1024, 3), ("w1", 1024, 4096, 2),
                            ("w2", 4096, 1024, 3)):
        x = N.DeviceArray.from_host(rng.standard_normal((rows, k)).astype(np.float16))
        w = N.DeviceArray.from_host((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16))
        b = N.DeviceArray.from_host(rng.standard_normal(n).astype(np.float16))
        r = N.DeviceArray.from_host(rng.standard_normal((rows, n)).astype(np.float16))
        y = N.DeviceArray((rows, n), np.float16)
        call = lambda: N.check(N.lib.nml_linear_device(x.ptr, k, w.ptr, b.ptr, r.ptr if epi == 3 else None,
                                                       y.ptr, rows, k, n, epi, N.np_dtype_code(np.float16)))
        call()
        N.synchronize()
        t = N.Timer()
        t.start()
        for _ in range(reps):
            call()
        ms = t.stop() / reps
        N.synchronize()
        nbytes = n * k * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us_per_launch": round(ms * 1e3, 2), "weight_bytes": nbytes,
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    return {"workload": "C4 projections of one 16-row half, d1024 fp16, nml_linear_device, "
                        f"{reps} back-to-back launches each", **out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--new-tokens", type=int, default=512)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--only-c3", action="store_true", help="skip the batch-32 and prefill lines")
    ap.add_argument("--only", choices=["c3", "c4", "c4attn", "c4proj", "c5", "adamw", "train",
                                       "train16"],
                    default=None,
                    help="run one workload only (for profiling); c4/c5 print their own line")
    ap.add_argument("--train-skew", action="store_true",
                    help="train lines with half of the input ids one token (embedding scatter)")
    ap.add_argument("--c4-uniform", action="store_true",
                    help="C4 with every prompt at the ragged lengths' mean (counter passes)")
    ap.add_argument("--c4-reps", type=int, default=2,
                    help="timed generate() calls of the C4 line (0: the warm-up only)")
    ap.add_argument("--cpu-samples", type=int, default=8,
                    help="tokens of the CPU baseline, spread over the run's contexts")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 256 MiB device to device three times (the known-size "
                         "reference for scaling the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this path does "
              f"not shard across GPUs (the sharding design is described in DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)

    import nimbleml_amd as nm
    from oracle.weights import C3, make_weights, random_ids

    cfg = C3
    nm._native.ensure_init()
    if args.copy_calibration:
        N = nm._native
        nbytes = 256 << 20
        src, dst = N.DeviceArray((nbytes,), "uint8"), N.DeviceArray((nbytes,), "uint8")
        N.check(N.lib.nml_memset(src.ptr, 1, nbytes))
        for _ in range(3):
            N.check(N.lib.nml_memcpy_d2d(dst.ptr, src.ptr, nbytes))
        N.synchronize()
        print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 3}), flush=True)
        return
    if args.only == "c5":
        print(json.dumps({"c5": bench_c5(nm, cpu=not args.no_cpu_baseline)}), flush=True)
        return
    if args.only == "c4attn":
        print(json.dumps({"c4attn": bench_c4_attention(nm)}), flush=True)
        return
    if args.only == "c4proj":
        print(json.dumps({"c4proj": bench_c4_projections(nm)}), flush=True)
        return
    if args.only == "adamw":
        print(json.dumps({"adamw": bench_adamw(nm)}), flush=True)
        return
    if args.only == "train":
        print(json.dumps({"train": bench_train(nm)}), flush=True)
        return
    if args.only == "train16":
        print(json.dumps({"train16": bench_train(nm, dtype=np.float16, skew=args.train_skew)}),
              flush=True)
        return
    w16 = make_weights(cfg, seed=1234, dtype=np.float16)
    model = nm.GPT.from_arrays(w16, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, dtype=np.float16)
    model.to_device()
    prompt = random_ids((1, args.prompt), cfg.vocab_size, seed=99)
    n = args.new_tokens
    use_graph = not args.no_graph
    if args.only == "c4":
        print(json.dumps({"c4": bench_c4(nm, cfg, model, use_graph, reps=args.c4_reps,
                                         w16=None if args.no_cpu_baseline else w16,
                                         uniform=args.c4_uniform)}), flush=True)
        return

    elapsed, step_ms, bytes_avg, persistent = bench_c3(nm, cfg, model, prompt, n, args.steps,
                                                       args.warmup, use_graph)
    achieved = bytes_avg / (step_ms * 1e-3) / 1e9
    traffic = pmc_traffic() if persistent else None
    result = {
        "metric": METRIC,
        "value": round(args.steps * n / elapsed, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * elapsed / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        "config": {"workload": f"C3: GPT V32000 d1024 H16 L24 fp16, batch 1, prompt {args.prompt}, "
                               f"greedy {n} new tokens; one step = one generate() call",
                   "global_batch": 1, "seq_len": args.prompt + n, "parallelism": "none"},
        "decode_ms_per_token": round(step_ms, 4),
        "roofline": {"bound": "hbm",
                     "kernel": "decode_persist_kernel (one launch per token)" if persistent
                     else "decode step (all kernels of one token)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": round(traffic) if traffic else None,
                     "bytes_per_launch": round(bytes_avg)},
    }
    if not (args.only_c3 or args.only == "c3"):
        result["c4"] = bench_c4(nm, cfg, model, use_graph, w16=None if args.no_cpu_baseline else w16)
        del model
        result["c5"] = bench_c5(nm, cpu=not args.no_cpu_baseline)
        result["train"] = bench_train(nm)
        result["train16"] = bench_train(nm, dtype=np.float16)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, w16, prompt, args.new_tokens, args.cpu_samples)
        result["cpu_baseline_fp16"] = cpu_baseline_fp16(cfg, w16, prompt, args.new_tokens)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
