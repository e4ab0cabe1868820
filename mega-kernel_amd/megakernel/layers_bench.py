"""Timing of the layer-by-layer engine: the batched prefill (``prefill``) and the batched decode
(``decode_batch``, either engine), on random-init bf16 weights of a Qwen3 shape (``model.build_model``, seed 0),
with HIP events around each call on the current stream.

    cd mega-kernel_amd
    python -m megakernel.layers_bench --shape qwen3-0.6b --prefill 32,64,3584 --batch 1,8 --context 256

Prints one line per prompt length / batch size: the median over ``--runs`` calls after ``--warmup``
calls, and tokens per second (prompt tokens, or sequences x 1 token for a decode step). Under
``rocprofv3 --kernel-trace --stats`` the same command gives the per-kernel split.

``--transformers`` also times the path ``prefill`` replaces, on the same GPU and prompts: the
reference's Transformers prefill ``model(input_ids, use_cache=True)`` and the copy of its cache into
the decode layout (/root/reference/model.py:72-87; ``megakernel.copy_prefill_cache``).
"""
import argparse
import statistics
import sys


def _time(fn, warmup, runs):
    import torch
    for _ in range(warmup):
        fn()
    out = []
    for _ in range(runs):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        out.append(e0.elapsed_time(e1))
    return statistics.median(out), out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", default="qwen3-0.6b")
    ap.add_argument("--prefill", default="", help="comma-separated prompt lengths")
    ap.add_argument("--batch", default="", help="comma-separated batch sizes (1..64)")
    ap.add_argument("--context", type=int, default=256, help="position of every sequence of a decode batch")
    ap.add_argument("--max-seq", type=int, default=4096)
    ap.add_argument("--offset", type=int, default=0,
                    help="prefill at this position: the prompt continues a cache of that many positions (a later "
                         "chunk of a longer prompt)")
    ap.add_argument("--runs", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--engine", type=int, default=0, choices=(0, 1, 2),
                    help="decode_batch engine: 0 automatic, 1 layer by layer, 2 persistent kernel (where it applies)")
    ap.add_argument("--graph", action="store_true",
                    help="decode_batch: capture one call in a HIP graph (torch.cuda.graph) and time its replays")
    ap.add_argument("--transformers", action="store_true",
                    help="also time the reference path: Transformers' GPU prefill plus the cache copy")
    a = ap.parse_args(argv)
    import torch
    import megakernel
    from model import build_model

    kernel = megakernel.load()
    kernel.set_batch_engine(a.engine)
    dev = torch.device("cuda:0")
    model = build_model(a.shape, a.max_seq)
    lw = [t.to(dev) for t in megakernel.layer_weight_list(model)]
    embed = model.model.embed_tokens.weight.detach().to(dev)
    fn = model.model.norm.weight.detach().to(dev)
    cos, sin = megakernel.rope_tables(model, a.max_seq, dev)
    L = len(model.model.layers)
    vocab = embed.shape[0]
    gen = torch.Generator().manual_seed(1)
    for P in [int(x) for x in a.prefill.split(",") if x]:
        if a.offset + P > a.max_seq:
            sys.exit(f"offset {a.offset} + prompt {P} exceeds --max-seq {a.max_seq}")
        kc, vc = megakernel.empty_cache(L, a.max_seq, dev)
        ids = torch.randint(0, vocab, (P,), generator=gen).to(dev, torch.int32)
        med, runs = _time(lambda: kernel.prefill(ids, embed, embed, fn, lw, cos, sin, kc, vc, a.offset, a.max_seq),
                          a.warmup, a.runs)
        at = f" at {a.offset}" if a.offset else ""
        print(f"[prefill {a.shape} P={P}{at}] {med:.3f} ms median of {len(runs)} ({P / med * 1e3:,.0f} tokens/s); "
              f"runs {[round(t, 3) for t in runs]}", flush=True)
        if a.transformers and not a.offset:
            gpu_model = model.to(dev)
            ids2 = ids.long().unsqueeze(0)

            def reference_path():
                with torch.inference_mode():
                    out = gpu_model(ids2, use_cache=True)
                megakernel.copy_prefill_cache(out.past_key_values, kc, vc)

            med_r, runs_r = _time(reference_path, a.warmup, a.runs)
            print(f"[transformers prefill + cache copy {a.shape} P={P}] {med_r:.3f} ms median of {len(runs_r)} "
                  f"({P / med_r * 1e3:,.0f} tokens/s); native prefill {med_r / med:.2f}x faster", flush=True)
        del kc, vc
    for B in [int(x) for x in a.batch.split(",") if x]:
        if a.context >= a.max_seq:
            sys.exit(f"--context {a.context} must be below --max-seq {a.max_seq}")
        dgen = torch.Generator(device=dev).manual_seed(2)
        kc = (torch.randn(B, L, 8, a.max_seq, 128, generator=dgen, device=dev) * 0.5).to(torch.bfloat16)
        vc = torch.randn(B, L, 8, a.max_seq, 128, generator=dgen, device=dev).to(torch.bfloat16)
        toks = torch.randint(0, vocab, (B,), generator=gen).to(dev, torch.int32)
        pos = torch.full((B,), a.context, dtype=torch.int32, device=dev)
        step = lambda: kernel.decode_batch(toks, pos, embed, embed, fn, lw, cos, sin, kc, vc, a.max_seq)
        if a.graph:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                step()
            torch.cuda.current_stream().wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step()
            step = g.replay
        med, runs = _time(step, a.warmup, a.runs)
        print(f"[decode_batch {a.shape} B={B} context={a.context} engine {a.engine}{' graph' if a.graph else ''}] "
              f"{med * 1e3:.1f} us per step median of "
              f"{len(runs)} ({B / med * 1e3:,.0f} tokens/s)", flush=True)
        del kc, vc
    if kernel.status() != 0:
        sys.exit(f"device status {kernel.status()}")


if __name__ == "__main__":
    main()
