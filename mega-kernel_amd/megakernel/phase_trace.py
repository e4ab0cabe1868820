"""Per-phase timing and barrier-stall report from a decode-kernel phase trace.

The kernel's optional trace (``mk_set_trace``; ``mk_bench --trace FILE``) stores, per workgroup,
``s_memrealtime`` stamps (100 MHz): slot ``20*layer + 2*phase`` when the math of phase A..E of a
layer starts and ``+1`` when the phase's outputs are published; ``20*layer + 10 + k`` when the
communication wave finishes its k-th wait (QKV, attention partials, o_proj cross-XCD, o_proj
local, MLP, down cross-XCD, down local); slots 1280.. = kernel start, end of the last layer,
LM-head start, LM-head end.

For each phase kind the report gives, summed over layers: the mean and max per-workgroup busy time
(start -> published), the mean exchange stall (published -> next phase start) and the bytes the
phase moves from HBM (algorithmic, from the model shape), so GB/s per phase = bytes / span; then
the time each exchange wait took.

    python -m megakernel.phase_trace trace.bin [--shape qwen3-0.6b] [--ctx N]
"""
import argparse
import sys

import numpy as np

TICK_US = 0.01
TRACE_LAYERS = 64
TRACE_PER_LAYER = 20
TRACE_N = TRACE_LAYERS * TRACE_PER_LAYER + 8
TAIL = TRACE_LAYERS * TRACE_PER_LAYER
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
    base = t[:, TAIL].min()
    t = t - base
    out = []
    tot = {p: [0.0, 0.0, 0.0, 0.0] for p in PHASES}  # mean busy, max busy, mean stall, span
    for layer in range(layers):
        for p in range(5):
            s = t[:, TRACE_PER_LAYER * layer + 2 * p]
            a = t[:, TRACE_PER_LAYER * layer + 2 * p + 1]
            if p < 4:
                nxt = t[:, TRACE_PER_LAYER * layer + 2 * p + 2]
            elif layer + 1 < layers:
                nxt = t[:, TRACE_PER_LAYER * (layer + 1)]
            else:
                nxt = t[:, TAIL + 1]
            busy = (a - s) * TICK_US
            stall = (nxt - a) * TICK_US
            k = PHASES[p]
            tot[k][0] += busy.mean()
            tot[k][1] += busy.max()
            tot[k][2] += stall.mean()
            tot[k][3] += (nxt.max() - s.min()) * TICK_US
    pb = phase_bytes(hidden, inter, ctx)
    kernel_us = (t[:, TAIL + 3].max() - 0) * TICK_US
    out.append(f"kernel {kernel_us:.1f} us (first start -> last LM-head end); layers {layers}")
    out.append(f"{'phase':12s} {'busy mean':>10s} {'busy max':>9s} {'stall mean':>11s} {'span':>8s} {'MB':>8s} {'GB/s':>8s}")
    for k in PHASES:
        b = pb[k] * layers
        out.append(f"{k:12s} {tot[k][0]:10.1f} {tot[k][1]:9.1f} {tot[k][2]:11.1f} {tot[k][3]:8.1f} "
                   f"{b / 1e6:8.2f} {b / (tot[k][3] * 1e-6) / 1e9 if tot[k][3] > 0 else 0:8.0f}")
    emb = (t[:, TAIL].max()) * TICK_US
    tail = (t[:, TAIL + 2] - t[:, TAIL + 1]).mean() * TICK_US
    lm = (t[:, TAIL + 3].max() - t[:, TAIL + 2].min()) * TICK_US
    lmb = 151936 * hidden * 2
    waits = ("qkv", "att", "o cross", "o local", "mlp", "down cross", "down local")
    prev_slot = (1, 3, 5, 12, 7, 9, 15)  # the event each wait follows, same layer
    row = []
    for k, name in enumerate(waits):
        d = 0.0
        for layer in range(layers):
            prev = t[:, TRACE_PER_LAYER * layer + prev_slot[k]]
            d += ((t[:, TRACE_PER_LAYER * layer + 10 + k] - prev) * TICK_US).mean()
        row.append(f"{name} {d:.1f}")
    out.append("comm waits (mean us, summed over layers; from the previous event): " + ", ".join(row))
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
