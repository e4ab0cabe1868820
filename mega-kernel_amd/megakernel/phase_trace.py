"""Per-phase timing and barrier-stall report from a decode-kernel phase trace.

The kernel's optional trace (``mk_set_trace``; ``mk_bench --trace FILE``) stores, per workgroup,
``s_memrealtime`` stamps (100 MHz): slot ``10*layer + 2*phase`` when phase A..E of a layer starts
(its barrier released) and ``+1`` when the workgroup arrives at the barrier ending it; slots
640.. = kernel start, end of the last layer, LM-head start, LM-head end.

For each phase kind the report gives, summed over layers: the mean and max per-workgroup busy time
(start -> arrival), the mean barrier stall (arrival -> next phase start) and the bytes the phase
moves from HBM (algorithmic, from the model shape), so GB/s per phase = bytes / span.

    python -m megakernel.phase_trace trace.bin [--shape qwen3-0.6b] [--ctx N]
"""
import argparse
import sys

import numpy as np

TICK_US = 0.01
TRACE_LAYERS = 64
TRACE_N = TRACE_LAYERS * 10 + 8
PHASES = ("A qkv", "B attention", "C o_proj", "D gate/up", "E down")


def phase_bytes(hidden, inter, ctx):
    """Algorithmic HBM bytes per layer of each phase (bf16 weights, K/V cache)."""
    q, kv = 16 * 128, 8 * 128
    return {
        "A qkv": (q + 2 * kv) * hidden * 2 + hidden * 2,
        "B attention": 8 * 128 * 2 * 2 * ctx + 2 * 128 * 2,
        "C o_proj": hidden * q * 2,
        "D gate/up": 2 * inter * hidden * 2 + hidden * 2,
        "E down": hidden * inter * 2,
    }


def load(path, grid=256):
    t = np.fromfile(path, dtype=np.uint64)
    if t.size != grid * TRACE_N:
        raise ValueError(f"{path}: expected {grid * TRACE_N} stamps, got {t.size}")
    return t.reshape(grid, TRACE_N).astype(np.int64)


def report(t, layers, hidden, inter, ctx):
    base = t[:, 640].min()
    t = t - base
    out = []
    tot = {p: [0.0, 0.0, 0.0, 0.0] for p in PHASES}  # mean busy, max busy, mean stall, span
    for layer in range(layers):
        for p in range(5):
            s = t[:, 10 * layer + 2 * p]
            a = t[:, 10 * layer + 2 * p + 1]
            if p < 4:
                nxt = t[:, 10 * layer + 2 * p + 2]
            elif layer + 1 < layers:
                nxt = t[:, 10 * (layer + 1)]
            else:
                nxt = t[:, 641]
            busy = (a - s) * TICK_US
            stall = (nxt - a) * TICK_US
            k = PHASES[p]
            tot[k][0] += busy.mean()
            tot[k][1] += busy.max()
            tot[k][2] += stall.mean()
            tot[k][3] += (nxt.max() - s.min()) * TICK_US
    pb = phase_bytes(hidden, inter, ctx)
    kernel_us = (t[:, 643].max() - 0) * TICK_US
    out.append(f"kernel {kernel_us:.1f} us (first start -> last LM-head end); layers {layers}")
    out.append(f"{'phase':12s} {'busy mean':>10s} {'busy max':>9s} {'stall mean':>11s} {'span':>8s} {'MB':>8s} {'GB/s':>8s}")
    for k in PHASES:
        b = pb[k] * layers
        out.append(f"{k:12s} {tot[k][0]:10.1f} {tot[k][1]:9.1f} {tot[k][2]:11.1f} {tot[k][3]:8.1f} "
                   f"{b / 1e6:8.2f} {b / (tot[k][3] * 1e-6) / 1e9 if tot[k][3] > 0 else 0:8.0f}")
    emb = (t[:, 640 + 0].max()) * TICK_US
    tail = (t[:, 642] - t[:, 641]).mean() * TICK_US
    lm = (t[:, 643].max() - t[:, 642].min()) * TICK_US
    lmb = 151936 * hidden * 2
    out.append(f"final norm (mean) {tail:.1f} us; LM head span {lm:.1f} us, {lmb / 1e6:.1f} MB, "
               f"{lmb / (lm * 1e-6) / 1e9:.0f} GB/s")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--shape", default="qwen3-0.6b", choices=["qwen3-0.6b", "qwen3-1.7b"])
    ap.add_argument("--ctx", type=int, default=288, help="context length of the traced step")
    ap.add_argument("--layers", type=int, default=28)
    a = ap.parse_args(argv)
    h, i = (1024, 3072) if a.shape == "qwen3-0.6b" else (2048, 6144)
    print(report(load(a.trace), a.layers, h, i, a.ctx))


if __name__ == "__main__":
    sys.exit(main())
