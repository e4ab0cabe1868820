#!/usr/bin/env python
"""Batch-1 decode throughput of the MI355X mega-kernel on BASELINE.json's config 2.

Workload (config 2): Qwen3-0.6B-shaped model, random-init bf16 weights from seed 0 (std 0.02,
norms 1), 32-token random prompt (seed 1), cache 512, 256 teacher-forced greedy decode steps.
A "step" is one call of the decode operator (one cooperative kernel launch): one token through
the whole model at context position+1 in [33, 288].

Legs:
  * CPU baseline (rank 0, N=1): Transformers' bf16 CPU decode of the same model and prompt -- the
    reference path's own comparison decode -- timed per step with perf_counter on all host cores
    this process may use. It also yields the reference (teacher) tokens the GPU leg feeds.
  * GPU: the prefill K/V copied into the kernel cache, W untimed warm-up steps (then the cache is
    restored), K timed steps between synchronizations. HIP events on the operator's stream time
    every launch; the roofline divides each step's algorithmic bytes by its kernel time.

Algorithmic bytes per step B(ctx) = all weights read once (every layer, the full tied LM head,
one embedding row, the norms) + K/V read for ctx positions + the new K/V row + one cos/sin row.
Prints ONE JSON line.
"""
import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (REPO, os.path.join(REPO, "mega-kernel_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK = 8.0e12  # MI355X HBM3E, B/s
METRIC = "batch-1 decode tokens/sec (Qwen3-0.6B shape) + % of HBM roofline GB/s"
REF_TOKS_PER_S = 325.57  # reference's published mega-kernel decode rate (RTX 3090)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps (K)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed warm-up decode steps (W)")
    ap.add_argument("--shape", default="qwen3-0.6b", choices=["qwen3-0.6b", "qwen3-1.7b"])
    ap.add_argument("--prompt", type=int, default=32)
    ap.add_argument("--max-seq", type=int, default=512)
    ap.add_argument("--cpu-steps", type=int, default=None,
                    help="steps of the CPU baseline sample (default: same as --steps, capped at 256)")
    ap.add_argument("--cpu-min-seconds", type=float, default=10.0,
                    help="repeat the CPU baseline decode until it has run at least this long (at most 8 runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the Transformers CPU leg (random teacher tokens, cpu_baseline null)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the timed steps, copy a device buffer of this many MiB (device to device) so a "
                         "rocprofv3 --pmc run of this command also measures FETCH_SIZE/WRITE_SIZE of a plain copy")
    ap.add_argument("--traffic", default=os.path.join(REPO, "profiles", "decode_traffic_qwen3-0.6b_p32_c512.json"),
                    help="measured HBM traffic per launch (JSON written from the rocprofv3 --pmc runs); used only "
                         "when its kernel version and workload match this run")
    return ap.parse_args()


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: --gpus {a.gpus} is not supported: this build targets one MI355X; the decode step "
              "runs on one GPU (see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2
    import torch
    import megakernel
    from oracle import hf
    from oracle.spec import SHAPES

    shape = SHAPES[a.shape]
    if a.prompt + a.steps > a.max_seq:
        print("bench.py: prompt + steps exceeds the cache length", file=sys.stderr)
        return 2
    kernel = megakernel.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # ---- model (CPU, seeded) and its weights on the GPU ------------------------------------
    t0 = time.perf_counter()
    model = hf.build_model(a.shape, max_positions=max(4096, a.max_seq))
    build_s = time.perf_counter() - t0
    ids = hf.prompt_ids(a.prompt, shape.vocab)

    # ---- CPU baseline leg: Transformers decode on the host cores -----------------------------
    cpu = None
    n_cpu = min(a.cpu_steps or a.steps, 256)
    if not a.no_cpu_baseline:
        cores = hf.cpu_threads()
        torch.set_num_threads(cores)
        ref = hf.greedy_reference(model, ids, max(n_cpu, 1))
        secs = ref["seconds"][3:] if len(ref["seconds"]) > 6 else ref["seconds"]
        cpu_total = sum(ref["seconds"])
        runs = 1
        # a bounded sample of about 10-30 s of CPU work: repeat the same decode while it is shorter
        while cpu_total < a.cpu_min_seconds and runs < 8:
            again = hf.greedy_reference(model, ids, max(n_cpu, 1))
            secs += again["seconds"][3:] if len(again["seconds"]) > 6 else again["seconds"]
            cpu_total += sum(again["seconds"])
            runs += 1
        med = statistics.median(secs)
        teacher = list(ref["tokens"])
        cpu = {"value": round(1.0 / med, 3), "unit": "tokens/s", "cores": cores, "kind": "reference",
               "sample": (f"Transformers {__import__('transformers').__version__} Qwen3ForCausalLM bf16 on the host "
                          f"CPU: the reference path's own comparison decode (/root/reference/model.py:139-173) run "
                          f"on CPU, same weights and prompt, {len(ref['seconds'])} greedy decode steps after a "
                          f"{a.prompt}-token prefill ({runs} run(s)), median per-step time excluding 3 warm-up steps "
                          f"of each run; {cpu_total:.1f} s of CPU work on {cores} threads")}
    else:
        teacher = []
    g = torch.Generator().manual_seed(2)
    while len(teacher) < a.steps + a.warmup:
        teacher.append(int(torch.randint(0, shape.vocab, (1,), generator=g)))

    # ---- GPU leg -----------------------------------------------------------------------------
    embed = model.model.embed_tokens.weight.detach().to(dev)
    final_norm = model.model.norm.weight.detach().to(dev)
    layers = [t.to(dev) for t in megakernel.layer_weight_list(model)]
    cos, sin = hf.rope_tables(model, a.max_seq)
    cos, sin = cos.to(dev), sin.to(dev)
    _, cache = hf.prefill(model, ids)
    kc0, vc0 = megakernel.empty_cache(shape.layers, a.max_seq, dev)
    P = megakernel.copy_prefill_cache(cache, kc0, vc0)
    kc, vc = kc0.clone(), vc0.clone()
    del model, cache

    def step(tok, pos):
        return kernel.decode(tok, embed, embed, final_norm, layers, cos, sin, kc, vc, pos, a.max_seq)

    for w in range(a.warmup):
        step(teacher[w], P + w)
    torch.cuda.synchronize()
    kc.copy_(kc0)
    vc.copy_(vc0)
    torch.cuda.synchronize()
    # One HIP event pair brackets the timed region on the launch stream. (An event pair around every
    # launch would add an end-of-kernel cache release per event to the GPU timeline, ~20 us a step.)
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for t in range(a.steps):
        step(teacher[t], P + t)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    region_ms = ev0.elapsed_time(ev1)
    status = kernel.status()
    if status != 0:
        print(f"bench.py: device status {status}: a grid wait timed out, results invalid", file=sys.stderr)
        return 1

    if a.calibrate_copy_mib > 0:
        n = a.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    ctxs = [P + t + 1 for t in range(a.steps)]
    bytes_steps = [shape.bytes_per_token(c) for c in ctxs]
    achieved = sum(bytes_steps) / (region_ms * 1e-3)
    tok_s = a.steps / wall
    workload = (f"BASELINE config 2: {a.shape} random-init bf16, batch 1, prompt {a.prompt}, cache {a.max_seq}, "
                f"{a.steps} teacher-forced decode steps (ctx {ctxs[0]}..{ctxs[-1]})")
    traffic = None
    if a.traffic and os.path.exists(a.traffic):
        tr = json.load(open(a.traffic))
        if (tr.get("kernel_version") == kernel.version() and tr.get("shape") == a.shape
                and tr.get("prompt") == a.prompt and tr.get("max_seq_len") == a.max_seq):
            traffic = tr.get("hbm_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(wall * 1e3 / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tok_s / REF_TOKS_PER_S, 3),
        "dtype": "bf16",
        "data": "synthetic (random-init seeded weights, random prompt ids; no checkpoint or dataset)",
        "config": {
            "workload": workload,
            "batch": 1, "prompt": a.prompt, "max_seq_len": a.max_seq, "decode_steps": a.steps,
            "teacher_tokens": "transformers-cpu" if not a.no_cpu_baseline else "random",
            "arithmetic": "bf16 weights and K/V, bf16x2 dot products of weights with hi/lo-split fp32 "
                          "activations, fp32 accumulation",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved / 1e9, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK, 4),
            "traffic": traffic,
            # NKV = 1 while the attention splits are at most 32 positions long, 2 beyond
            "kernel": ("mk::decode_kernel<1024, 3072, NKV>" if a.shape == "qwen3-0.6b"
                       else "mk::decode_kernel<2048, 6144, NKV>"),
            "bytes_per_launch_avg": int(sum(bytes_steps) / a.steps),
            "kernel_us_avg": round(1e3 * region_ms / a.steps, 2),
        },
        "cpu_baseline": cpu,
        "model_build_s": round(build_s, 1),
    }
    print(json.dumps(out))
    return 0


def release_device():
    """Free the cached device memory and drain the GPU before interpreter exit, so that an
    attached profiler (rocprofv3) finalizes its output before the runtime tears down."""
    torch = sys.modules.get("torch")
    if torch is not None and torch.cuda.is_initialized():
        import gc
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


if __name__ == "__main__":
    rc = main()
    release_device()
    if rc:
        sys.exit(rc)
