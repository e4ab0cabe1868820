"""Phase timeline of the persistent batched decode kernel (``mk_set_batch_trace``).

Runs ``decode_batch`` on random-init bf16 weights of a Qwen3 shape (``model.build_model``, seed 0)
for B sequences at one context length, with the kernel's phase trace on, and reports for the middle
layers the mean time of each traced point since the layer's start (over workgroups; and the latest
workgroup), so the gaps between consecutive points show where a layer's time goes.

    cd mega-kernel_amd
    python -m megakernel.batch_trace --shape qwen3-0.6b --batch 8 --context 256

The points (thread 0 of each workgroup, comm wave 0, unless marked math: thread 0 of the first math
wave): A start; residual + input norm done (the previous layer's down sums polled); QKV tile done
(the math waves publish the rows); [attention workgroups: q/k/v polled and normalised; math:
attention start, scores done; attention done; math: split partial published]; split partials
polled; all comm waves' polls done (barrier C1); math: gate/up rows issued, merge done; splits
merged; o_proj tile done; math: o_proj rows published; the 8 XCDs' partials of row block j polled;
its sum republished; residual +
post-attention norm done (sums polled); gate/up tile done; SiLU outputs polled; down tile done;
down row block summed and republished.
"""
import argparse
import ctypes

import numpy as np

TICK_US = 0.01
MAXL, SLOTS, GRID = 32, 24, 256
NAMES = ("A start", "A residual+norm", "A qkv tile", "", "B qkv polled", "B attention",
         "C splits polled", "C merged", "C o tile", "D gather+pub", "E residual+norm", "E gate/up tile",
         "F silu polled", "F down tile", "G gather+pub", "B partial pub (math)", "D o rows pub (math)",
         "D gather polled", "B start (math)",
         "B scores done (math)", "C1 passed", "", "C gate/up issued (math)", "C merge done (math)")
ORDER = (0, 1, 2, 4, 18, 19, 5, 15, 6, 20, 22, 23, 7, 8, 16, 17, 9, 10, 11, 12, 13, 14)
ATT_SLOTS = (4, 5, 15, 18, 19)


def split_plan(positions):
    """The kernel's key-range length and number of ranges for sequences at these positions: the
    smallest candidate length (16 ceil(T / 512) + a multiple of a step) that gives at most 32 ranges,
    rounded up to a multiple of 32 keys."""
    B, T = len(positions), sum(p + 1 for p in positions)
    ks0 = 16 * -(-T // 512)
    kfit = 16 * -(-T // (16 * (32 - B)))
    step = 16 * max(1, -(-(kfit - ks0) // (16 * 63)))
    for i in range(64):
        cand = max(kfit, ks0 + step * 63) if i == 63 else ks0 + step * i
        if sum((p + cand) // cand for p in positions) <= 32:
            break
    ks = 32 * -(-cand // 32)
    return ks, sum((p + ks) // ks for p in positions)


def report(t, layers, att_mask):
    """t: int64 [GRID][MAXL + 1][SLOTS] stamps."""
    t = t - t[:, MAXL, 0].min()
    lo, hi = (1, layers - 1) if layers > 4 else (0, layers)
    lines = []
    kernel_us = t[:, MAXL, 2].max() * TICK_US
    lm_us = (t[:, MAXL, 2].max() - t[:, MAXL, 1].min()) * TICK_US
    per_layer = [(t[:, l + 1, 0].mean() - t[:, l, 0].mean()) * TICK_US for l in range(lo, min(hi, layers - 1))]
    lm_wg = (t[:, MAXL, 2] - t[:, MAXL, 1]) * TICK_US
    lines.append(f"kernel {kernel_us:.1f} us; mean layer {np.mean(per_layer):.2f} us (layers {lo}..{hi - 1}); "
                 f"LM head {lm_us:.1f} us (per workgroup mean {lm_wg.mean():.1f}, max {lm_wg.max():.1f}; starts "
                 f"spread over {(t[:, MAXL, 1].max() - t[:, MAXL, 1].min()) * TICK_US:.1f}); first layer starts "
                 f"{t[:, 0, 0].mean() * TICK_US:.1f} us after kernel start")
    lines.append(f"{'point':22s} {'mean us':>8s} {'max us':>8s}   (since the layer's A start, mean over layers)")
    for s in ORDER:
        name = NAMES[s]
        rows = att_mask if s in ATT_SLOTS else np.ones(GRID, bool)
        if not rows.any():
            continue
        d = np.stack([(t[rows, l, s] - t[rows, l, 0]) for l in range(lo, hi)]) * TICK_US
        lines.append(f"{name:22s} {d.mean():8.2f} {d.max(axis=1).mean():8.2f}")
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", default="qwen3-0.6b")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--context", type=int, default=256)
    ap.add_argument("--max-seq", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=3)
    a = ap.parse_args(argv)
    import torch
    import megakernel
    from megakernel import build as mkbuild
    from model import build_model

    kernel = megakernel.load()
    lib = ctypes.CDLL(mkbuild.LIB)
    lib.mk_batch_trace_bytes.restype = ctypes.c_size_t
    lib.mk_set_batch_trace.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    dev = torch.device("cuda:0")
    model = build_model(a.shape, a.max_seq)
    lw = [w.to(dev) for w in megakernel.layer_weight_list(model)]
    embed = model.model.embed_tokens.weight.detach().to(dev)
    fn = model.model.norm.weight.detach().to(dev)
    cos, sin = megakernel.rope_tables(model, a.max_seq, dev)
    L, B = len(model.model.layers), a.batch
    gen = torch.Generator(device=dev).manual_seed(2)
    kc = (torch.randn(B, L, 8, a.max_seq, 128, generator=gen, device=dev) * 0.5).to(torch.bfloat16)
    vc = torch.randn(B, L, 8, a.max_seq, 128, generator=gen, device=dev).to(torch.bfloat16)
    toks = torch.randint(0, embed.shape[0], (B,), device=dev, dtype=torch.int32)
    pos = torch.full((B,), a.context, dtype=torch.int32, device=dev)
    kernel.set_batch_engine(2)
    for _ in range(a.warmup):
        kernel.decode_batch(toks, pos, embed, embed, fn, lw, cos, sin, kc, vc, a.max_seq)
    buf = torch.zeros(lib.mk_batch_trace_bytes() // 8, dtype=torch.int64, device=dev)
    if lib.mk_set_batch_trace(ctypes.c_void_p(buf.data_ptr()), buf.numel() * 8) != 0:
        raise SystemExit("mk_set_batch_trace failed")
    torch.cuda.synchronize()
    kernel.decode_batch(toks, pos, embed, embed, fn, lw, cos, sin, kc, vc, a.max_seq)
    torch.cuda.synchronize()
    lib.mk_set_batch_trace(None, 0)
    t = buf.cpu().numpy().reshape(GRID, MAXL + 1, SLOTS)
    # workgroups with an attention split: the split plan of the kernel
    ks, nsplit = split_plan([a.context] * B)
    att = np.array([(w // 8) < nsplit for w in range(GRID)])
    print(f"[batch trace {a.shape} B={B} context={a.context}] {nsplit} key ranges of {ks}")
    print(report(t, L, att))
    if kernel.status() != 0:
        raise SystemExit(f"device status {kernel.status()}")


if __name__ == "__main__":
    main()
