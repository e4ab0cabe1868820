"""Per-phase timeline and exchange-stall report from a decode-kernel phase trace.

The kernel's optional trace (``mk_set_trace``; ``mk_bench --trace FILE``) stores, per workgroup,
``s_memrealtime`` stamps (100 MHz) taken by the communication wave at fixed points of every layer
(``SLOTS``: phase start = the barrier after which the comm wave waits for the math waves, "pub"
= this workgroup's result published, "poll" = the exchange it waits on completed) and four tail
stamps: kernel start, LM-head start, LM-head end, exit.

The report averages over the middle layers: for each slot, the time since the layer's first
stamp (mean over workgroups, and the latest workgroup), so the gaps between consecutive slots show
where a layer's time goes: math (start -> pub), exchange latency plus skew (pub -> poll) and comm
work (poll -> next start). It also gives the algorithmic bytes of each phase and the LM-head rate.

    python -m megakernel.phase_trace trace.bin [--shape qwen3-0.6b] [--layers 28]
"""
import argparse
import sys

import numpy as np

TICK_US = 0.01
TRACE_LAYERS = 64
TRACE_PER_LAYER = 32
TRACE_N = TRACE_LAYERS * TRACE_PER_LAYER + 8
TAIL = TRACE_LAYERS * TRACE_PER_LAYER
SLOTS = ("A start", "A pub (qkv)", "A poll (qkv)", "B start", "B pub (partial)", "B poll (merge)",
         "C start", "C pub", "C cross poll", "C local poll", "D start", "D pub (mlp)", "D poll (mlp)",
         "E start", "E pub", "E cross poll", "E local poll", "math A end", "math B start", "math B end",
         "B merge max", "B merge sum", "math A dot done",
         "math D issued", "math D dot done", "math B issued", "math B scores done")


def phase_bytes(hidden, inter, ctx):
    """Algorithmic HBM bytes per layer of each phase (bf16 weights, K/V cache)."""
    q, kv = 16 * 128, 8 * 128
    return {
        "A qkv": (q + 2 * kv) * hidden * 2,
        "B attention": kv * 2 * 2 * ctx,
        "C o_proj": hidden * q * 2,
        "D gate/up": 2 * inter * hidden * 2,
        "E down": hidden * inter * 2,
    }


def load(path, grid=256):
    t = np.fromfile(path, dtype=np.uint64)
    if t.size != grid * TRACE_N:
        raise ValueError(f"{path}: expected {grid * TRACE_N} stamps, got {t.size}")
    return t.reshape(grid, TRACE_N).astype(np.int64)


def report(t, layers, hidden, inter, ctx):
    traw = t
    t = t - t[:, TAIL].min()
    lo, hi = (1, layers - 1) if layers > 4 else (0, layers)
    out = []
    kernel_us = t[:, TAIL + 3].max() * TICK_US
    layer_us = [(t[:, TRACE_PER_LAYER * (layer + 1)].mean() - t[:, TRACE_PER_LAYER * layer].mean()) * TICK_US
                for layer in range(lo, min(hi, layers - 1))]
    out.append(f"kernel {kernel_us:.1f} us; mean layer {np.mean(layer_us):.2f} us (layers {lo}..{hi - 1})")
    out.append(f"{'slot':18s} {'mean t':>8s} {'max t':>8s} {'d mean':>8s}   (us since the layer's first A start, mean over layers)")
    prev = 0.0
    for k, name in enumerate(SLOTS):
        rows = []
        for layer in range(lo, hi):
            base = t[:, TRACE_PER_LAYER * layer].min()
            raw = traw[:, TRACE_PER_LAYER * layer + k]
            col = t[:, TRACE_PER_LAYER * layer + k][raw != 0]  # slots some workgroups never stamp
            if col.size == 0:
                continue
            rows.append(((col - base).mean() * TICK_US, (col - base).max() * TICK_US))
        if not rows:
            continue
        m = float(np.mean([r[0] for r in rows]))
        x = float(np.mean([r[1] for r in rows]))
        out.append(f"{name:18s} {m:8.2f} {x:8.2f} {m - prev:8.2f}")
        prev = m
    pb = phase_bytes(hidden, inter, ctx)
    out.append("bytes per layer: " + ", ".join(f"{k} {v / 1e6:.2f} MB" for k, v in pb.items()))
    lm = (t[:, TAIL + 2].max() - t[:, TAIL + 1].min()) * TICK_US
    lmb = 151936 * hidden * 2
    out.append(f"LM head span {lm:.1f} us, {lmb / 1e6:.1f} MB, {lmb / (lm * 1e-6) / 1e9:.0f} GB/s")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--shape", default="qwen3-0.6b", choices=["qwen3-0.6b", "qwen3-1.7b"])
    ap.add_argument("--ctx", type=int, default=96, help="context length of the traced step")
    ap.add_argument("--layers", type=int, default=28)
    a = ap.parse_args(argv)
    h, i = (1024, 3072) if a.shape == "qwen3-0.6b" else (2048, 6144)
    print(report(load(a.trace), a.layers, h, i, a.ctx))


if __name__ == "__main__":
    sys.exit(main())
