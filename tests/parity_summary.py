"""Markdown summary of the parity records the GPU tests leave (``tests/gpu_common.write_record``):
one row per BASELINE config of the decode against Transformers and the same-run fp32 restatement,
and one per BASELINE prompt of the native prefill.

    python tests/parity_summary.py [RECORD_DIR]      (default: gpurun_out/parity)
"""
import glob
import json
import os
import sys


def _f(x, n=2):
    return f"{x:.{n}e}"


def summary(d):
    recs = {os.path.basename(p)[:-5]: json.load(open(p)) for p in sorted(glob.glob(os.path.join(d, "*.json")))}
    out = []
    dec = [(k, v) for k, v in recs.items() if k.startswith("decode_config")]
    if dec:
        v0 = dec[0][1]
        out.append(f"Kernel `{v0.get('kernel_version', '?').split(' (')[0]}` on `{v0.get('device', '?')}`.\n")
        out.append("| config | workload | steps | tokens = Transformers: kernel / oracle | max-abs vs Transformers: "
                   "kernel / oracle | min cosine: kernel / oracle | kernel = oracle tokens | tight: tokens, max-abs | "
                   "north star met (tokens, max-abs, cos): kernel / oracle |")
        out.append("|---|---|---|---|---|---|---|---|---|")
        for k, v in dec:
            n = v["steps"]
            t = v["tokens_equal_transformers"]
            ma, mc, tg = v["max_abs_vs_transformers"], v["min_cos_vs_transformers"], v["tight"]
            ns = v["north_star_met"]
            flags = lambda m: "".join("y" if m[q] else "n" for q in ("tokens", "max_abs", "cos"))
            out.append(f"| {k[len('decode_config'):]} | {v['workload']} | {n} | {t['kernel']} / {t['oracle']} "
                       f"({100 * t['kernel'] / n:.1f}%) | {_f(ma['kernel'])} / {_f(ma['oracle'])} | "
                       f"{mc['kernel']:.8f} / {mc['oracle']:.8f} | {v['tokens_kernel_equal_oracle']}/{n} | "
                       f"{tg['tokens_same']}/{tg['steps']}, {_f(tg['max_abs'])} | {flags(ns['kernel'])} / "
                       f"{flags(ns['oracle'])} |")
    pre = [(k, v) for k, v in recs.items() if k.startswith("prefill_")]
    if pre:
        out.append("")
        out.append("| prefill | time | tight max-abs | tokens: kernel / oracle / Transformers | last logits vs "
                   "Transformers max-abs: kernel / oracle | cosine: kernel / oracle |")
        out.append("|---|---|---|---|---|---|")
        for k, v in pre:
            lt, tk = v["last_logits_vs_transformers"], v["tokens"]
            out.append(f"| {v['workload']} | {v['prefill_ms']:.2f} ms | {_f(v['tight']['max_abs'])} | "
                       f"{tk['kernel']} / {tk['oracle']} / {tk['transformers']} | {_f(lt['kernel']['max_abs'])} / "
                       f"{_f(lt['oracle']['max_abs'])} | {lt['kernel']['cos']:.8f} / {lt['oracle']['cos']:.8f} |")
    return "\n".join(out)


if __name__ == "__main__":
    print(summary(sys.argv[1] if len(sys.argv) > 1 else os.path.join("gpurun_out", "parity")))
