"""Benchmark: generated tokens/s of the GPT token loop on one MI355X.

Workload ("C3"): GPT vocab 32000, d_model 1024, 16 heads,
24 layers, MLP 4x GELU, RMSNorm, max_seq_len 2048, fp16 weights ~N(0, 0.02) (seeded,
synthetic), batch 1, prompt of 512 uniform ids, greedy decode of 512 new tokens.
One step = one whole generate() call (prefill + 511 decode steps + on-device
selection), inputs resident on the device when the timed region starts.

Prints one JSON line. ``roofline`` is for the decode step (the dominant work):
algorithmic bytes = every weight once (2·(L·(12d²+11d) + V·d + d) B) plus the K/V
cache read, 2·2·L·d·ctx B, and written, 2·2·L·d B, per step, averaged over the
run's contexts 513…1023; divided by the decode time measured with HIP events on
the library stream around the decode loop. ``cpu_baseline`` times the oracle (the
reference algorithm restated: full re-forward per token, host sampling) on the
host cores on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = BASELINE_METRIC = "generated tokens/sec + % HBM/MFMA roofline, d1024 L24 fp16 GPT, batch 1 & 32"
HBM_PEAK_GBS = 8000.0


def c3_bytes_per_step(cfg, ctx):
    d, L, V = cfg.d_model, cfg.num_layers, cfg.vocab_size
    weights = 2 * (L * (12 * d * d + 11 * d) + V * d + d)
    kv_read = 2 * 2 * L * d * ctx
    kv_write = 2 * 2 * L * d
    return weights + kv_read + kv_write


def cpu_baseline(cfg, w16, prompt, tokens=3):
    """Reference algorithm on the host: fp32 (NumPy fp16 has no BLAS path)."""
    from oracle import gpt_ref as R

    try:
        from threadpoolctl import threadpool_info

        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    w = {k: v.astype(np.float32) for k, v in w16.items()}
    t0 = time.perf_counter()
    R.generate(w, prompt, cfg.num_heads, cfg.num_layers, max_new_tokens=tokens, temperature=0.0)
    dt = time.perf_counter() - t0
    return {"value": round(tokens / dt, 4), "unit": "tokens/s", "cores": int(threads),
            "kind": "port",
            "sample": f"C3 shapes, fp32, batch 1, prompt {prompt.shape[1]}, {tokens} greedy tokens "
                      f"by full re-forward per token as the reference does ({dt:.1f} s)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--new-tokens", type=int, default=512)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path does "
              f"not shard across GPUs)", file=sys.stderr)
        sys.exit(2)

    import nimbleml_amd as nm
    from nimbleml_amd import _native as N
    from oracle.weights import C3, make_weights, random_ids

    cfg = C3
    N.ensure_init()
    w16 = make_weights(cfg, seed=1234, dtype=np.float16)
    model = nm.GPT.from_arrays(w16, cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers,
                               cfg.max_seq_len, dtype=np.float16)
    model.to_device()
    prompt = random_ids((1, args.prompt), cfg.vocab_size, seed=99)
    n = args.new_tokens
    kw = dict(max_new_tokens=n, temperature=0.0, use_graph=not args.no_graph)

    for _ in range(args.warmup):
        nm.generate(model, prompt, **kw)
    N.synchronize()
    decode_ms = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = nm.generate(model, prompt, **kw)
        decode_ms.append(model.last_decode_ms())
    N.synchronize()
    elapsed = time.perf_counter() - t0
    assert out.shape == (1, args.prompt + n)

    ms_per_step = 1000.0 * elapsed / args.steps
    value = args.steps * n / elapsed
    ctxs = np.arange(args.prompt + 1, args.prompt + n)  # attention lengths of the decode steps
    bytes_avg = float(np.mean([c3_bytes_per_step(cfg, c) for c in ctxs]))
    step_ms = float(np.mean(decode_ms))
    achieved = bytes_avg / (step_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        "config": {"workload": f"C3 decode: GPT V32000 d1024 H16 L24 fp16, batch 1, prompt "
                               f"{args.prompt}, greedy {n} new tokens",
                   "global_batch": 1, "seq_len": args.prompt + n, "parallelism": "none"},
        "decode_ms_per_token": round(step_ms, 4),
        "roofline": {"bound": "hbm", "kernel": "decode step (embed … sample)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_step": round(bytes_avg)},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, w16, prompt)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
