"""HBM traffic per decode launch from two rocprofv3 counter runs of ``bench.py``.

``bench.py --calibrate-copy-mib M`` ends with one device-to-device copy of M MiB; the counters that
copy reads calibrate the counter units (FETCH_SIZE reads half the copied bytes in KiB on this
part, WRITE_SIZE the full amount), and the same scale turns the decode kernel's per-dispatch counts
into bytes. Writes the JSON that ``bench.py --traffic`` reads (it is used only when its kernel
version, shape, prompt and cache length match the run).

    python -m megakernel.pmc_traffic FETCH_CSV WRITE_CSV --copy-mib 1024 --version "..." \\
        --shape qwen3-0.6b --prompt 32 --max-seq 512 --algorithmic-bytes B -o traffic.json
"""
import argparse
import csv
import json
import statistics
import sys

KERNEL = "mk::decode_kernel"
COPY = "__amd_rocclr_copyBuffer"


def counter_rows(path, counter):
    with open(path, newline="") as f:
        return [r for r in csv.DictReader(f) if r["Counter_Name"] == counter]


def summarize(path, counter, copy_bytes):
    rows = counter_rows(path, counter)
    dec = [float(r["Counter_Value"]) for r in rows if r["Kernel_Name"].startswith(f"void {KERNEL}<")]
    names = {r["Kernel_Name"] for r in rows if r["Kernel_Name"].startswith(f"void {KERNEL}<")}
    copies = [float(r["Counter_Value"]) for r in rows if r["Kernel_Name"] == COPY]
    if not dec or not copies:
        raise SystemExit(f"{path}: no {KERNEL} or {COPY} dispatches with {counter}")
    cal = max(copies)  # the calibration copy is the largest copyBuffer dispatch
    return {"kernels": sorted(names), "dispatches": len(dec), "kib_per_dispatch": statistics.mean(dec),
            "copy_kib": cal, "scale": copy_bytes / (cal * 1024.0)}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("fetch_csv")
    ap.add_argument("write_csv")
    ap.add_argument("--copy-mib", type=int, required=True)
    ap.add_argument("--version", required=True, help="kernel version string (megakernel.load().version())")
    ap.add_argument("--shape", required=True)
    ap.add_argument("--prompt", type=int, required=True)
    ap.add_argument("--max-seq", type=int, required=True)
    ap.add_argument("--algorithmic-bytes", type=int, required=True, help="mean algorithmic bytes per launch")
    ap.add_argument("--command", action="append", default=[], help="the profiler commands, for the record")
    ap.add_argument("-o", "--out", required=True)
    a = ap.parse_args(argv)
    copy_bytes = a.copy_mib * (1 << 20)
    fe = summarize(a.fetch_csv, "FETCH_SIZE", copy_bytes)
    wr = summarize(a.write_csv, "WRITE_SIZE", copy_bytes)
    fs, ws = round(fe["scale"], 5), round(wr["scale"], 5)
    hbm = fe["kib_per_dispatch"] * 1024 * fs + wr["kib_per_dispatch"] * 1024 * ws
    out = {
        # the decode kernel's instantiations (register rows per context), averaged over all dispatches
        "kernel": ", ".join(k.replace("void ", "").split("(")[0] for k in fe["kernels"]),
        "kernel_version": a.version,
        "shape": a.shape, "prompt": a.prompt, "max_seq_len": a.max_seq,
        "dispatches": fe["dispatches"],
        "fetch_size_kib_per_dispatch": round(fe["kib_per_dispatch"], 2),
        "write_size_kib_per_dispatch": round(wr["kib_per_dispatch"], 2),
        "copy_calibration": {"bytes": copy_bytes, "fetch_size_kib": fe["copy_kib"], "write_size_kib": wr["copy_kib"],
                             "fetch_scale": fs, "write_scale": ws},
        "hbm_bytes_per_launch": int(round(hbm)),
        "algorithmic_bytes_per_launch_avg": a.algorithmic_bytes,
        "commands": a.command,
    }
    with open(a.out, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
