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


def hop_report(t, layers, nxcd=8):
    """Latency of each exchange split into the hop itself and the wait for stragglers.

    For every reader and layer: ``lat`` = its poll completion minus the publish stamp of the LAST
    workgroup it reads from (the exchange's own latency: store visibility plus poll round trips),
    ``own`` = its poll completion minus its own publish stamp (``own - lat`` is the time spent waiting
    for slower writers). Workgroup b is local index b // nxcd on XCD b % nxcd. Writers per exchange:
    QKV and MLP slice -- the reader's XCD; cross hop -- local index j on every XCD; republish -- the
    reader's XCD at their cross-poll completion (the republish store follows it)."""
    idx = {n: i for i, n in enumerate(SLOTS)}
    grid = t.shape[0]
    x = np.arange(grid) % nxcd
    j = np.arange(grid) // nxcd
    lo, hi = (2, layers - 2) if layers > 6 else (0, layers)

    def col(layer, name):
        return t[:, TRACE_PER_LAYER * layer + idx[name]].astype(np.float64) * TICK_US

    acc = {}

    def add(key, lat, own):
        acc.setdefault(key, []).append((float(np.mean(lat)), float(np.mean(own))))

    for layer in range(lo, hi):
        apub, apoll = col(layer, "A pub (qkv)"), col(layer, "A poll (qkv)")
        m = t[:, TRACE_PER_LAYER * layer + idx["A poll (qkv)"]] != 0
        wx = np.array([apub[x == v].max() for v in x])
        add("A  qkv -> attention (local)", (apoll - wx)[m], (apoll - apub)[m])
        bpub, bpoll = col(layer, "B pub (partial)"), col(layer, "B poll (merge)")
        att = t[:, TRACE_PER_LAYER * layer + idx["math B scores done"]] != 0
        wb = np.array([bpub[(x == v) & att].max() if ((x == v) & att).any() else bpub[x == v].max() for v in x])
        # only the split workgroups publish; `own` is theirs
        add("B  split partials (local)", bpoll - wb, (bpoll - bpub)[att] if att.any() else bpoll - bpub)
        for ph in "CE":
            pub, cp, lp = col(layer, f"{ph} pub"), col(layer, f"{ph} cross poll"), col(layer, f"{ph} local poll")
            wj = np.array([pub[j == v].max() for v in j])
            add(f"{ph}  cross-XCD gather", cp - wj, cp - pub)
            wl = np.array([cp[x == v].max() for v in x])
            add(f"{ph}  republish (local)", lp - wl, lp - cp)
        dpub, dpoll = col(layer, "D pub (mlp)"), col(layer, "D poll (mlp)")
        wd = np.array([dpub[x == v].max() for v in x])
        add("D  MLP slice (local)", dpoll - wd, dpoll - dpub)
    out = [f"{'exchange':30s} {'lat us':>7s} {'own us':>7s}   (layers {lo}..{hi - 1}; lat = after the last writer, own = after this workgroup's publish)"]
    for k in ("A  qkv -> attention (local)", "B  split partials (local)", "C  cross-XCD gather", "C  republish (local)",
              "D  MLP slice (local)", "E  cross-XCD gather", "E  republish (local)"):
        v = acc.get(k)
        if v:
            out.append(f"{k:30s} {np.mean([a for a, _ in v]):7.2f} {np.mean([b for _, b in v]):7.2f}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--shape", default="qwen3-0.6b", choices=["qwen3-0.6b", "qwen3-1.7b"])
    ap.add_argument("--ctx", type=int, default=96, help="context length of the traced step")
    ap.add_argument("--layers", type=int, default=28)
    a = ap.parse_args(argv)
    h, i = (1024, 3072) if a.shape == "qwen3-0.6b" else (2048, 6144)
    t = load(a.trace)
    print(report(t, a.layers, h, i, a.ctx))
    print(hop_report(t, a.layers))


if __name__ == "__main__":
    sys.exit(main())
