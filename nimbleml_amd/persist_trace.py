"""Reader for the phase trace of the persistent decode kernel.

With NIMBLEML_PERSIST_TRACE=<file> set, the library writes, after a generate() call
that used the persistent decode step, the timestamps (s_memrealtime, 100 MHz) that
thread 0 of every workgroup took at the phase boundaries of the last decode step:
a header of three int32 (workgroups G, stride S per workgroup, layers L), then G·S
uint64. Per layer there are 10 marks (see decode_persist.hip: P1 issued, x in, QKV
out, q in, chunks out, merged, att in, xm in, h in, x out), then head x in, logits
out and the choice.

    python -m nimbleml_amd.persist_trace trace.bin

prints, per stage, the critical-path time to the next stage: the latest workgroup's
mark of the next stage minus the latest workgroup's mark of this one, median over
the layers.
"""
from __future__ import annotations

import sys

import numpy as np

NAMES = ["P1 issued", "x in", "QKV out", "q in", "chunks out", "merged", "att in", "xm in",
         "h in", "x out"]
TICK_NS = 10.0  # s_memrealtime runs at 100 MHz


def load(path):
    raw = open(path, "rb").read()
    g, s, layers = (int(v) for v in np.frombuffer(raw[:12], dtype=np.int32))
    t = np.frombuffer(raw[12:], dtype=np.uint64).reshape(g, s).astype(np.int64)
    return t, layers


def summary(t, layers):
    m = len(NAMES)
    t0 = t[:, 0][t[:, 0] > 0].min()

    def latest(k):
        v = t[:, k]
        v = v[v > 0]
        return (v.max() - t0) * TICK_NS / 1e3 if v.size else float("nan")

    lines = []
    period = [latest(4 + m * (l + 1) + 1) - latest(4 + m * l + 1) for l in range(1, layers - 1)]
    lines.append(f"layer period (latest 'x in' to the next): median {np.median(period):.2f} us")
    for k, name in enumerate(NAMES):
        d = []
        for l in range(1, layers - 1):
            nxt = 4 + m * l + k + 1 if k + 1 < m else 4 + m * (l + 1)
            d.append(latest(nxt) - latest(4 + m * l + k))
        lines.append(f"  {name:11s} -> next stage: {np.nanmedian(d):6.2f} us")
    h = 4 + m * layers
    lines.append(f"head: x in {latest(h):.2f} us, logits out {latest(h + 1):.2f} us, "
                 f"choice {latest(h + 2):.2f} us (from the first mark)")
    return "\n".join(lines)


def main(argv):
    t, layers = load(argv[1])
    print(summary(t, layers))


if __name__ == "__main__":
    main(sys.argv)
