"""Collect the rocprofv3 evidence behind bench.py's roofline numbers (run on the GPU box; needs no GPU itself).

For one workload it runs, each as a child process under its own time limit:
  1. rocprofv3 --kernel-trace --stats          -> per-kernel average durations
  2. rocprofv3 --pmc FETCH_SIZE                -> HBM KiB fetched per dispatch
  3. rocprofv3 --pmc WRITE_SIZE                -> HBM KiB written per dispatch
and the same two counter passes over a plain device-to-device copy of known size (bench.py --calibrate-copy), whose
counter/actual ratio scales the conv kernel's counters into bytes. It writes, under profiles/:
  <kernel>_<config>.md       the commands and the figures (what the numbers in DESIGN.md cite)
  traffic_<config>.json      HBM bytes per launch of the dominant kernel (read by bench.py)

usage: python bench_profile.py --config c3 [--out gpurun_out/prof]
"""
import argparse
import csv
import glob
import json
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
COPY_BYTES = 1 << 30


def run(cmd, timeout, log):
    print("+", " ".join(cmd), flush=True)
    with open(log, "w") as f:
        r = subprocess.run(["timeout", "-s", "KILL", str(timeout)] + cmd, stdout=f, stderr=subprocess.STDOUT,
                           cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"))
    if r.returncode != 0:
        sys.exit(f"failed ({r.returncode}): {' '.join(cmd)} -- see {log}")


def csv_rows(d, suffix):
    fs = glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)
    if not fs:
        sys.exit(f"no *{suffix} under {d}")
    with open(fs[0]) as f:
        return list(csv.DictReader(f))


def counter_avg(d, counter, pattern):
    vals = [float(r["Counter_Value"]) for r in csv_rows(d, "counter_collection.csv")
            if r["Counter_Name"] == counter and pattern in r["Kernel_Name"]]
    if not vals:
        sys.exit(f"no {counter} rows for kernels matching {pattern!r} in {d}")
    return sum(vals) / len(vals), len(vals)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c3")
    ap.add_argument("--out", default=os.path.join(ROOT, "gpurun_out", "prof"))
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--profiles-dir", default=os.path.join(ROOT, "profiles"),
                    help="where the summary and traffic_<config>.json go (on a GPU box: somewhere that is copied back)")
    args = ap.parse_args()
    out = os.path.join(args.out, args.config)
    os.makedirs(out, exist_ok=True)
    py = sys.executable
    bench = [py, os.path.join(ROOT, "bench.py"), "--config", args.config, "--steps", str(args.steps), "--warmup", "2",
             "--no-cpu", "--no-peaks", "--no-extras"]
    copy = [py, os.path.join(ROOT, "bench.py"), "--calibrate-copy"]
    rp = ["rocprofv3", "--output-format", "csv", "-o", "run"]

    # the same command without the profiler: its event-timed step, to set beside the profiled kernel average
    run(bench, 120, f"{out}/plain.log")
    plain = json.loads([l for l in open(f"{out}/plain.log") if l.startswith("{")][-1])
    run(rp + ["--kernel-trace", "--stats", "-d", f"{out}/trace", "--"] + bench, 300, f"{out}/trace.log")
    stats = csv_rows(f"{out}/trace", "kernel_stats.csv")
    stats.sort(key=lambda r: -float(r["TotalDurationNs"]))
    top = next(r for r in stats if "k_conv" in r["Name"])  # the conv kernel (the step's dominant kernel)
    kname = top["Name"]
    m = re.search(r"(k_conv\w*)", kname)  # the kernel's base name, e.g. k_conv_wide_dma
    key = m.group(1) if m else "k_conv"
    figs = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        run(rp + ["--pmc", counter, "-d", f"{out}/{counter}", "--"] + bench, 300, f"{out}/{counter}.log")
        figs[counter] = counter_avg(f"{out}/{counter}", counter, key)
        run(rp + ["--pmc", counter, "-d", f"{out}/copy_{counter}", "--"] + copy, 120, f"{out}/copy_{counter}.log")
        figs["copy_" + counter] = counter_avg(f"{out}/copy_{counter}", counter, "copy")
    fetch_factor = COPY_BYTES / 1024.0 / figs["copy_FETCH_SIZE"][0]
    write_factor = COPY_BYTES / 1024.0 / figs["copy_WRITE_SIZE"][0]
    fetch_b = figs["FETCH_SIZE"][0] * 1024.0 * fetch_factor
    write_b = figs["WRITE_SIZE"][0] * 1024.0 * write_factor
    res = {"config": args.config, "kernel": kname, "avg_ns": float(top["AverageNs"]), "calls": int(top["Calls"]),
           "fetch_KiB": figs["FETCH_SIZE"][0], "write_KiB": figs["WRITE_SIZE"][0],
           "copy_fetch_KiB": figs["copy_FETCH_SIZE"][0], "copy_write_KiB": figs["copy_WRITE_SIZE"][0],
           "copy_bytes": COPY_BYTES, "fetch_factor": fetch_factor, "write_factor": write_factor,
           "traffic_bytes": fetch_b + write_b, "plain_ms_per_step": plain["ms_per_step"]}
    prof = args.profiles_dir
    os.makedirs(prof, exist_ok=True)
    with open(os.path.join(prof, f"traffic_{args.config}.json"), "w") as f:
        json.dump(res, f, indent=1)
    rel = lambda cmd: " ".join(os.path.relpath(c, ROOT) if c.startswith(ROOT) else
                               ("python3" if c == py else c) for c in cmd)
    md = [f"# {key} on workload {args.config}", "",
          "Commands (run from the repository root on an MI355X box, each under `timeout -s KILL`):", "",
          "```", "rocprofv3 " + " ".join(rp[1:]) + " --kernel-trace --stats -d <out>/trace -- " + rel(bench),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc FETCH_SIZE -d <out>/FETCH_SIZE -- " + rel(bench),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc WRITE_SIZE -d <out>/WRITE_SIZE -- " + rel(bench),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc FETCH_SIZE -d <out>/copy_FETCH_SIZE -- " + rel(copy),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc WRITE_SIZE -d <out>/copy_WRITE_SIZE -- " + rel(copy),
          "```", "(generated by `python bench_profile.py --config " + args.config + "`)", "",
          "## Kernel time (--kernel-trace --stats, top kernels by total time)", "",
          "| kernel | calls | average us | total us | % |", "|---|---|---|---|---|"]
    for r in stats[:8]:
        md.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                  f"{float(r['TotalDurationNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    md += ["", f"Without the profiler the same command times a step (weight repack + this kernel, HIP events on the "
           f"library's stream) at {plain['ms_per_step'] * 1e3:.1f} us; the profiled average above is "
           f"{float(top['AverageNs']) / 1e3:.1f} us.", "",
           "## HBM traffic of the dominant kernel (per dispatch)", "",
           f"- FETCH_SIZE {figs['FETCH_SIZE'][0]:.0f} KiB ({figs['FETCH_SIZE'][1]} dispatches), "
           f"WRITE_SIZE {figs['WRITE_SIZE'][0]:.0f} KiB",
           f"- calibration: a {COPY_BYTES >> 20} MiB device copy reads FETCH_SIZE {figs['copy_FETCH_SIZE'][0]:.0f} KiB "
           f"and WRITE_SIZE {figs['copy_WRITE_SIZE'][0]:.0f} KiB -> factors {fetch_factor:.3f} (fetch), "
           f"{write_factor:.3f} (write)",
           f"- traffic = {fetch_b / 1e6:.1f} MB fetched + {write_b / 1e6:.1f} MB written = "
           f"{(fetch_b + write_b) / 1e6:.1f} MB per launch"]
    with open(os.path.join(prof, f"{key}_{args.config}.md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print(json.dumps(res))


if __name__ == "__main__":
    main()
