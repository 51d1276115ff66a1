"""Reader for the phase trace of the persistent decode kernel.

With NIMBLEML_PERSIST_TRACE=<file> set, the library writes, after a generate() call
that used the persistent decode step, the timestamps (s_memrealtime, 100 MHz) that
thread 0 of every workgroup took at the phase boundaries of the last decode step:
a header of three int32 (workgroups G, stride S per workgroup, layers L), then G·S
uint64. Per layer there are 16 marks (kernels.hpp, persist_trace_stride), then head
x in, logits out and the choice.

    python -m nimbleml_amd.persist_trace trace.bin

prints two tables, medians over the layers 1 … L-2:
  * the critical path: for each mark in the order a layer passes them, the latest
    workgroup's time of the next mark minus the latest workgroup's time of this one;
  * per-workgroup segments: the time one workgroup spends between two of its own
    marks (median and maximum over the workgroups).
"""
from __future__ import annotations

import sys

import numpy as np

MARKS = 16
NAMES = {0: "P1 loads issued", 1: "x in", 2: "QKV out", 14: "K/V loads issued", 3: "q in",
         4: "chunks out", 5: "merged", 15: "W_o loads issued", 6: "att in", 10: "x_mid out",
         11: "W1 loads issued", 7: "x_mid in", 12: "h out", 13: "W2 loads issued", 8: "h in",
         9: "x out"}
CHAIN = [0, 1, 2, 14, 3, 4, 5, 15, 6, 10, 11, 7, 12, 13, 8, 9]
SEGMENTS = [(0, 1, "QKV loads issued -> x in (x exchange, behind the loads)"),
            (1, 2, "x in -> QKV out (RMSNorm1, QKV rows)"),
            (2, 14, "QKV out -> K/V loads issued"),
            (14, 3, "K/V issued -> q in (team exchange)"),
            (3, 4, "q in -> chunks out (attention chunk)"),
            (15, 6, "W_o issued -> att in (attention exchange)"),
            (6, 10, "att in -> x_mid out (W_o rows)"),
            (10, 11, "x_mid out -> W1 loads issued"),
            (11, 7, "W1 issued -> x_mid in (exchange, behind the loads)"),
            (7, 12, "x_mid in -> h out (RMSNorm2, W1 rows, GELU)"),
            (12, 13, "h out -> W2 loads issued"),
            (13, 8, "W2 issued -> h in (exchange, behind the loads)"),
            (8, 9, "h in -> x out (W2 rows)")]
TICK_NS = 10.0  # s_memrealtime runs at 100 MHz


def load(path):
    raw = open(path, "rb").read()
    g, s, layers = (int(v) for v in np.frombuffer(raw[:12], dtype=np.int32))
    t = np.frombuffer(raw[12:], dtype=np.uint64).reshape(g, s).astype(np.int64)
    return t, layers


def summary(t, layers):
    t0 = t[:, 0][t[:, 0] > 0].min()
    us = np.where(t > 0, (t - t0) * TICK_NS / 1e3, np.nan)

    def col(l, k):
        return us[:, 4 + MARKS * l + k]

    def latest(l, k):
        v = col(l, k)
        return np.nanmax(v) if np.isfinite(v).any() else float("nan")

    mid = range(1, layers - 1)
    lines = []
    period = [latest(l + 1, 1) - latest(l, 1) for l in mid]
    lines.append(f"layer period (latest 'x in' to the next): median {np.median(period):.2f} us")
    lines.append("critical path (latest mark to latest next mark):")
    for i, k in enumerate(CHAIN):
        d = []
        for l in mid:
            nl, nk = (l, CHAIN[i + 1]) if i + 1 < len(CHAIN) else (l + 1, CHAIN[0])
            d.append(latest(nl, nk) - latest(l, k))
        nxt = NAMES[CHAIN[i + 1]] if i + 1 < len(CHAIN) else NAMES[CHAIN[0]] + " (next layer)"
        lines.append(f"  {NAMES[k]:17s} -> {nxt:28s} {np.nanmedian(d):6.2f} us")
    lines.append("per-workgroup segments (median / max over workgroups):")
    for a, b, name in SEGMENTS:
        med, mx = [], []
        for l in mid:
            d = col(l, b) - col(l, a)
            d = d[np.isfinite(d)]
            if d.size:
                med.append(np.median(d))
                mx.append(d.max())
        lines.append(f"  {name:55s} {np.median(med):6.2f} / {np.median(mx):6.2f} us")
    h = 4 + MARKS * layers
    lines.append(f"head: x in {np.nanmax(us[:, h]):.2f} us, logits out {np.nanmax(us[:, h + 1]):.2f} us, "
                 f"choice {np.nanmax(us[:, h + 2]):.2f} us (from the first mark)")
    lines.extend(placement(t))
    return "\n".join(lines)


def placement(t, xcds=8, heads=16):
    """Mark 2 holds each workgroup's XCD (HW_REG_XCC_ID): the offset c with workgroup g on
    XCD (g + c) % 8 (and how many follow it), and whether every head team (workgroups
    x + 8·k, k in the head's range) shares one XCD."""
    g = t.shape[0]
    xcc = t[:, 2]
    c = int((xcc[0] - 0) % xcds)
    same = int(np.sum(xcc == (np.arange(g) + c) % xcds))
    team = g // heads
    split = 0
    for h in range(heads):
        x, k0 = h % xcds, (h // xcds) * team
        members = [x + xcds * (k0 + k) for k in range(team)]
        split += len(set(int(v) for v in xcc[members])) > 1
    return [f"placement: {same}/{g} workgroups on XCD (g + {c}) % {xcds}; "
            f"{split}/{heads} head teams spread over more than one XCD"]


def main(argv):
    t, layers = load(argv[1])
    print(summary(t, layers))


if __name__ == "__main__":
    main(sys.argv)
