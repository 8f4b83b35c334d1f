"""Collect the rocprofv3 evidence behind bench.py's roofline numbers (run on the GPU box; needs no GPU itself).

For one workload it runs, each as a child process under its own time limit:
  1. rocprofv3 --kernel-trace --stats          -> per-kernel average durations
  2. rocprofv3 --pmc FETCH_SIZE                -> HBM KiB fetched per dispatch
  3. rocprofv3 --pmc WRITE_SIZE                -> HBM KiB written per dispatch
and the same two counter passes over a plain device-to-device copy of known size (bench.py --calibrate-copy), whose
counter/actual ratio scales the conv kernel's counters into bytes. It writes, under profiles/:
  <kernel>_<config>.md       the commands and the figures behind the documented roofline numbers
  traffic_<config>.json      HBM bytes per launch of the dominant kernel (read by bench.py)

With --upsample it profiles the cascade upsample block of c5 (bench.py --upsample-only): every kernel of the
subdivision, the children's map and the gathered conv, per block -> profiles/upsample_block_<config>.md.
With --kmap it profiles the kernel-map build instead (bench.py --kmap-only): per-kernel time and HBM bytes of every
build kernel -> profiles/kmap_build_<config>.md. With --gemm it profiles the vendor dense bf16 GEMM (bench.py
--gemm-only) with the same clock / MFMA-busy counters -> profiles/gemm_bf16_8192.md.

usage: python bench_profile.py --config c3 [--kmap] [--out DIR]   (raw rocprofv3 output; default: a temp dir)
"""
import argparse
import csv
import glob
import json
import os
import re
import subprocess
import sys
import tempfile

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


KMAP_KERNELS = ("k_brick_runs", "k_brick_mask", "k_table_clear", "k_brick_insert", "k_brick_fill", "k_neighbors_vox",
                "k_rs_count", "k_rs_digit_scan", "k_rs_scatter")


def kmap_profile(args, out, py, rp, copy, prof):
    """Kernel-map build: per-kernel time and HBM bytes of every build kernel, summed per build."""
    builds = args.steps + 1  # bench.py --kmap-only runs one untimed build, then --steps timed ones
    cmd = [py, os.path.join(ROOT, "bench.py"), "--config", args.config, "--steps", str(args.steps), "--kmap-only"]
    run(cmd, 120, f"{out}/plain.log")
    plain = json.loads([l for l in open(f"{out}/plain.log") if l.startswith("{")][-1])
    run(rp + ["--kernel-trace", "--stats", "-d", f"{out}/trace", "--"] + cmd, 300, f"{out}/trace.log")
    per = {}
    for r in csv_rows(f"{out}/trace", "kernel_stats.csv"):
        m = re.search(r"(k_\w+)", r["Name"])
        if m and m.group(1) in KMAP_KERNELS:
            per[m.group(1)] = {"calls": int(r["Calls"]), "avg_ns": float(r["AverageNs"])}
    figs = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        run(rp + ["--pmc", counter, "-d", f"{out}/{counter}", "--"] + cmd, 300, f"{out}/{counter}.log")
        rows = csv_rows(f"{out}/{counter}", "counter_collection.csv")
        for k in per:
            vals = [float(r["Counter_Value"]) for r in rows if r["Counter_Name"] == counter and k in r["Kernel_Name"]]
            per[k][counter] = sum(vals) / max(len(vals), 1)
        run(rp + ["--pmc", counter, "-d", f"{out}/copy_{counter}", "--"] + copy, 120, f"{out}/copy_{counter}.log")
        figs["copy_" + counter] = counter_avg(f"{out}/copy_{counter}", counter, "copy")
    ff = COPY_BYTES / 1024.0 / figs["copy_FETCH_SIZE"][0]
    wf = COPY_BYTES / 1024.0 / figs["copy_WRITE_SIZE"][0]
    kb = plain["kmap_build"]
    md = [f"# Kernel-map build on workload {args.config} (N = {plain['N']})", "",
          "Commands (run from the repository root on an MI355X box, each under `timeout -s KILL`):", "",
          "```", "rocprofv3 " + " ".join(rp[1:]) + " --kernel-trace --stats -d <out>/trace -- " + rel(cmd, py),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc FETCH_SIZE -d <out>/FETCH_SIZE -- " + rel(cmd, py),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc WRITE_SIZE -d <out>/WRITE_SIZE -- " + rel(cmd, py),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc FETCH_SIZE -d <out>/copy_FETCH_SIZE -- " + rel(copy, py),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc WRITE_SIZE -d <out>/copy_WRITE_SIZE -- " + rel(copy, py),
          "```", f"(generated by `python bench_profile.py --kmap --config {args.config}`; {builds} builds per command)",
          "", f"Counter scale factors from a {COPY_BYTES >> 20} MiB device copy: fetch {ff:.3f}, write {wf:.3f}.", "",
          "| kernel | dispatches per build | average us | us per build | MB fetched + written per dispatch | GB/s |",
          "|---|---|---|---|---|---|"]
    tot_us = tot_b = 0.0
    for k in KMAP_KERNELS:
        if k not in per:
            continue
        d = per[k]
        cpb = d["calls"] / builds
        b = (d.get("FETCH_SIZE", 0.0) * ff + d.get("WRITE_SIZE", 0.0) * wf) * 1024.0
        us = d["avg_ns"] / 1e3
        tot_us += us * cpb
        tot_b += b * cpb
        md.append(f"| `{k}` | {cpb:g} | {us:.1f} | {us * cpb:.1f} | {b / 1e6:.1f} | {b / (us * 1e-6) / 1e9:.0f} |")
    md += ["", f"Sum of the build kernels: {tot_us:.1f} us and {tot_b / 1e6:.1f} MB of HBM traffic per build "
           f"({tot_b / (tot_us * 1e-6) / 1e9:.0f} GB/s over the kernels' time).",
           f"Without the profiler the same command times a build (HIP events, median) at {kb['ms'] * 1e3:.1f} us; "
           f"algorithmic bytes {kb['algorithmic_bytes'] / 1e6:.1f} MB -> {kb['achieved_GBps']:.0f} GB/s = "
           f"{100 * kb['frac_of_hbm_peak']:.1f}% of the 8 TB/s HBM peak."]
    with open(os.path.join(prof, f"kmap_build_{args.config}.md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print(json.dumps({"config": args.config, "kernels": per, "sum_us": tot_us, "sum_bytes": tot_b, "plain": kb}))


def upsample_profile(args, out, py, rp, prof):
    """Cascade upsample block (bench.py --upsample-only): every kernel of subdivide_build and of the gathered conv on
    the fresh cache (first-call schedules included), summed per block."""
    blocks = args.steps + 1  # bench.py --upsample-only runs one untimed block, then --steps timed ones
    cmd = [py, os.path.join(ROOT, "bench.py"), "--config", args.config, "--steps", str(args.steps), "--upsample-only"]
    run(cmd, 120, f"{out}/plain.log")
    plain = json.loads([l for l in open(f"{out}/plain.log") if l.startswith("{")][-1])
    run(rp + ["--kernel-trace", "--stats", "-d", f"{out}/trace", "--"] + cmd, 300, f"{out}/trace.log")
    rows = []
    for r in csv_rows(f"{out}/trace", "kernel_stats.csv"):
        m = re.search(r"(k_\w+)", r["Name"])
        if not m:
            continue  # torch's input generation and copies
        rows.append((m.group(1), int(r["Calls"]), float(r["AverageNs"]), float(r["TotalDurationNs"])))
    agg = {}
    for k, calls, avg, tot in rows:  # template instances of one kernel summed under its name
        a = agg.setdefault(k, [0, 0.0])
        a[0] += calls
        a[1] += tot
    md = [f"# Cascade upsample block on workload {args.config}: {plain['parents']} parents -> {plain['children']} "
          "children", "",
          "Commands (run from the repository root on an MI355X box, each under `timeout -s KILL`):", "",
          "```", "rocprofv3 " + " ".join(rp[1:]) + " --kernel-trace --stats -d <out>/trace -- " + rel(cmd, py), "```",
          f"(generated by `python bench_profile.py --upsample --config {args.config}`; {blocks} blocks per command: "
          "subdivide_build, then the gathered conv on the fresh cache with its first-call schedules)", "",
          "| kernel | dispatches per block | average us | us per block | share |", "|---|---|---|---|---|"]
    tot_us = sum(v[1] for v in agg.values()) / 1e3 / blocks
    for k, (calls, tot) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        per = tot / 1e3 / blocks
        md.append(f"| `{k}` | {calls / blocks:g} | {tot / 1e3 / calls:.1f} | {per:.1f} | {100 * per / tot_us:.1f}% |")
    md += ["", f"Sum of the block's kernels: {tot_us:.1f} us per block.",
           f"Without the profiler the same command times a block (HIP events, median of {args.steps}) at "
           f"{plain['total_ms'] * 1e3:.1f} us: subdivide_build {plain['kmap_ms'] * 1e3:.1f} us, the conv on the fresh "
           f"cache {plain['conv_ms'] * 1e3:.1f} us. The kernel sum can exceed the block time where the spill-tile "
           "kernel of a 64-channel conv runs on a second stream beside the main one; here the conv is 128 -> 64 "
           "(the gathering kernel, one stream)."]
    with open(os.path.join(prof, f"upsample_block_{args.config}.md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print(json.dumps({"config": args.config, "kernels_us_per_block": {k: v[1] / 1e3 / blocks for k, v in agg.items()},
                      "sum_us": tot_us, "plain": plain}))


def rel(cmd, py):
    return " ".join(os.path.relpath(c, ROOT) if c.startswith(ROOT) else ("python3" if c == py else c) for c in cmd)


def gemm_profile(args, out, py, rp, prof):
    """The vendor dense bf16 GEMM (bench.py --gemm-only: 8192^3 torch.mm after the settle phase) under the same
    kernel-trace and MFMA-busy passes as the conv kernels -> profiles/gemm_bf16_8192.md: the sustained MFMA ceiling
    of the box, as a clock and a busy fraction to set beside the conv kernels' own."""
    bench = [py, os.path.join(ROOT, "bench.py"), "--gemm-only", "--steps", str(max(args.steps, 20))]
    run(bench, 120, f"{out}/plain.log")
    plain = json.loads([l for l in open(f"{out}/plain.log") if l.startswith("{")][-1])
    run(rp + ["--kernel-trace", "--stats", "-d", f"{out}/trace", "--"] + bench, 300, f"{out}/trace.log")
    stats = csv_rows(f"{out}/trace", "kernel_stats.csv")
    stats.sort(key=lambda r: -float(r["TotalDurationNs"]))
    top = stats[0]
    kname = top["Name"]
    busy = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "GRBM_GUI_ACTIVE")
    run(rp + ["--pmc"] + list(busy) + ["-d", f"{out}/busy", "--"] + bench, 300, f"{out}/busy.log")
    key = kname[:40]
    figs = {c: counter_avg(f"{out}/busy", c, key) for c in busy}
    ncu = int(os.environ.get("SPCONV_PROFILE_CUS", "256"))
    nxcd = int(os.environ.get("SPCONV_PROFILE_XCDS", "8"))
    avg_ns = float(top["AverageNs"])
    gui = figs["GRBM_GUI_ACTIVE"][0] / nxcd
    clock = gui / avg_ns
    mbusy = figs["SQ_VALU_MFMA_BUSY_CYCLES"][0] / (gui * ncu * 4)
    tf = 2 * 8192 ** 3 / (avg_ns * 1e-9) / 1e12
    rel = lambda cmd: " ".join(os.path.relpath(c, ROOT) if c.startswith(ROOT) else
                               ("python3" if c == py else c) for c in cmd)
    md = ["# Vendor dense bf16 GEMM (8192 x 8192 x 8192, torch.mm) -- the box's sustained MFMA ceiling", "",
          "Commands (run from the repository root on an MI355X box, each under `timeout -s KILL`):", "",
          "```", "rocprofv3 " + " ".join(rp[1:]) + " --kernel-trace --stats -d <out>/trace -- " + rel(bench),
          "rocprofv3 " + " ".join(rp[1:]) + " --pmc " + " ".join(busy) + " -d <out>/busy -- " + rel(bench), "```",
          "(generated by `python bench_profile.py --gemm`)", "",
          "| kernel | calls | average us | total us | % |", "|---|---|---|---|---|"]
    for r in stats[:4]:
        md.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                  f"{float(r['TotalDurationNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    md += ["", f"Without the profiler the same command (settled, then {max(args.steps, 20)} timed calls) times a GEMM at "
           f"{plain['gemm_ms'] * 1e3:.1f} us = {plain['bf16_gemm_TFLOPs']:.0f} TFLOP/s; the profiled average over "
           f"every call (settle included) is {avg_ns / 1e3:.1f} us = {tf:.0f} TFLOP/s.", "",
           "| counter | value per dispatch |", "|---|---|"]
    for c in busy:
        md.append(f"| {c} | {figs[c][0]:.4g} |")
    md += ["", f"- engine clock over the dispatch: GRBM_GUI_ACTIVE / {nxcd} XCDs / duration = {clock:.3f} GHz",
           f"- MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {nxcd} x {ncu} CUs x 4 SIMDs) = "
           f"{100 * mbusy:.1f}%",
           f"- waves waiting on an instruction dependency (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES): "
           f"{100 * figs['SQ_WAIT_INST_ANY'][0] / max(figs['SQ_WAVE_CYCLES'][0], 1.0):.1f}%",
           f"- dense bf16 peak at that clock: 256 CUs x 4 SIMDs x 1024 flop/clk x {clock:.3f} GHz = "
           f"{ncu * 4 * 1024 * clock / 1e3:.0f} TFLOP/s (the 2500 TFLOP/s spec assumes 2.4 GHz)"]
    with open(os.path.join(prof, "gemm_bf16_8192.md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print(json.dumps({"kernel": kname, "avg_ns": avg_ns, "clock_GHz": clock, "mfma_busy": mbusy, "TFLOPs": tf,
                      "plain": plain}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c3")
    ap.add_argument("--kmap", action="store_true", help="profile the kernel-map build instead of the conv step")
    ap.add_argument("--gemm", action="store_true", help="profile the vendor dense bf16 GEMM ceiling instead")
    ap.add_argument("--upsample", action="store_true",
                    help="profile the cascade upsample block of a subdivision workload (--config c5) instead")
    ap.add_argument("--out", default=os.path.join(tempfile.gettempdir(), "spconv_prof"))
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--profiles-dir", default=os.path.join(ROOT, "profiles"),
                    help="where the summary and traffic_<config>.json go (on a GPU box: somewhere that is copied back)")
    args = ap.parse_args()
    out = os.path.join(args.out, ("kmap_" if args.kmap else "") + args.config)
    os.makedirs(out, exist_ok=True)
    py = sys.executable
    bench = [py, os.path.join(ROOT, "bench.py"), "--config", args.config, "--steps", str(args.steps), "--warmup", "2",
             "--no-cpu", "--no-peaks", "--no-extras"]
    copy = [py, os.path.join(ROOT, "bench.py"), "--calibrate-copy"]
    rp = ["rocprofv3", "--output-format", "csv", "-o", "run"]
    if args.kmap:
        os.makedirs(args.profiles_dir, exist_ok=True)
        return kmap_profile(args, out, py, rp, copy, args.profiles_dir)
    if args.upsample:
        out = os.path.join(args.out, "upsample_" + args.config)
        os.makedirs(out, exist_ok=True)
        os.makedirs(args.profiles_dir, exist_ok=True)
        return upsample_profile(args, out, py, rp, args.profiles_dir)
    if args.gemm:
        out = os.path.join(args.out, "gemm")
        os.makedirs(out, exist_ok=True)
        os.makedirs(args.profiles_dir, exist_ok=True)
        return gemm_profile(args, out, py, rp, args.profiles_dir)

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
    # MFMA pipe and wave-state counters of the dominant kernel (one pass: 4 SQ counters + 1 GRBM counter)
    busy = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "GRBM_GUI_ACTIVE")
    run(rp + ["--pmc"] + list(busy) + ["-d", f"{out}/busy", "--"] + bench, 300, f"{out}/busy.log")
    for c in busy:
        figs[c] = counter_avg(f"{out}/busy", c, key)
    fetch_factor = COPY_BYTES / 1024.0 / figs["copy_FETCH_SIZE"][0]
    write_factor = COPY_BYTES / 1024.0 / figs["copy_WRITE_SIZE"][0]
    fetch_b = figs["FETCH_SIZE"][0] * 1024.0 * fetch_factor
    write_b = figs["WRITE_SIZE"][0] * 1024.0 * write_factor
    res = {"config": args.config, "kernel": kname, "avg_ns": float(top["AverageNs"]), "calls": int(top["Calls"]),
           "fetch_KiB": figs["FETCH_SIZE"][0], "write_KiB": figs["WRITE_SIZE"][0],
           "copy_fetch_KiB": figs["copy_FETCH_SIZE"][0], "copy_write_KiB": figs["copy_WRITE_SIZE"][0],
           "copy_bytes": COPY_BYTES, "fetch_factor": fetch_factor, "write_factor": write_factor,
           "traffic_bytes": fetch_b + write_b, "plain_ms_per_step": plain["ms_per_step"],
           "plain_kernel_ms": plain["roofline"]["kernel_ms"],
           "source_digest": plain["extras"]["source_digest"]}
    ncu = int(os.environ.get("SPCONV_PROFILE_CUS", "256"))
    nxcd = int(os.environ.get("SPCONV_PROFILE_XCDS", "8"))
    avg_ns = float(top["AverageNs"])
    # GRBM_GUI_ACTIVE is summed over the XCDs: per-XCD engine cycles over the dispatch = value / 8.
    # SQ_VALU_MFMA_BUSY_CYCLES is summed over the SIMDs (4 per CU), so it is normalized by 4 x 256 SIMDs.
    gui = figs["GRBM_GUI_ACTIVE"][0] / nxcd
    res["counters"] = {c: figs[c][0] for c in busy}
    res["clock_GHz"] = gui / avg_ns
    res["mfma_busy_frac"] = figs["SQ_VALU_MFMA_BUSY_CYCLES"][0] / (gui * ncu * 4)
    res["wait_frac_of_wave_cycles"] = figs["SQ_WAIT_INST_ANY"][0] / max(figs["SQ_WAVE_CYCLES"][0], 1.0)
    # the same utilisation implied by the algorithmic flops: executed flops / (kernel time x the dense bf16 rate
    # of 256 CUs x 4 SIMDs x 1024 flop/clk at the measured clock)
    rl = plain["roofline"]
    if rl["bound"] == "mfma":
        ex = plain["extras"]["executed_over_active_pairs"]
        flops = plain["extras"]["roofline_detail"]["algorithmic_flops"]
        res["mfma_util_from_flops"] = flops * ex / (avg_ns * 1e-9) / (ncu * 4 * 1024 * gui / avg_ns * 1e9)
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
    md += ["", f"Without the profiler the same command (after its settle phase: untimed launches until the per-launch "
           f"time stops falling) times a step (weight repack + the conv kernels, HIP events on the library's stream) "
           f"at {plain['ms_per_step'] * 1e3:.1f} us and the conv kernels alone at {plain['roofline']['kernel_ms'] * 1e3:.1f} "
           f"us; the profiled average above, over every launch of the run (warm-up and settle included), is "
           f"{float(top['AverageNs']) / 1e3:.1f} us.", "",
           "## HBM traffic of the dominant kernel (per dispatch)", "",
           f"- FETCH_SIZE {figs['FETCH_SIZE'][0]:.0f} KiB ({figs['FETCH_SIZE'][1]} dispatches), "
           f"WRITE_SIZE {figs['WRITE_SIZE'][0]:.0f} KiB",
           f"- calibration: a {COPY_BYTES >> 20} MiB device copy reads FETCH_SIZE {figs['copy_FETCH_SIZE'][0]:.0f} KiB "
           f"and WRITE_SIZE {figs['copy_WRITE_SIZE'][0]:.0f} KiB -> factors {fetch_factor:.3f} (fetch), "
           f"{write_factor:.3f} (write)",
           f"- traffic = {fetch_b / 1e6:.1f} MB fetched + {write_b / 1e6:.1f} MB written = "
           f"{(fetch_b + write_b) / 1e6:.1f} MB per launch",
           f"- compulsory bytes (x, nbr rows, weights, bias, residual, output and order, once each) {plain['extras']['roofline_detail']['compulsory_bytes'] / 1e6:.1f} MB "
           f"-> traffic / compulsory = {(fetch_b + write_b) / plain['extras']['roofline_detail']['compulsory_bytes']:.2f}",
           "", "## MFMA pipe and wave states of the dominant kernel (per dispatch)", "",
           "```", "rocprofv3 " + " ".join(rp[1:]) + " --pmc " + " ".join(busy) + " -d <out>/busy -- " + rel(bench), "```",
           "", "| counter | value |", "|---|---|"]
    for c in busy:
        md.append(f"| {c} | {figs[c][0]:.4g} |")
    md += ["", f"- engine clock over the dispatch: GRBM_GUI_ACTIVE / {nxcd} XCDs / duration = {res['clock_GHz']:.3f} GHz",
           f"- MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {nxcd} x {ncu} CUs x 4 SIMDs) = "
           f"{100 * res['mfma_busy_frac']:.1f}%",
           f"- waves waiting on an instruction dependency (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES): "
           f"{100 * res['wait_frac_of_wave_cycles']:.1f}%"]
    if "mfma_util_from_flops" in res:
        md.append(f"- MFMA utilisation implied by the executed flops (active pairs x "
                  f"{plain['extras']['executed_over_active_pairs']} padding) at that clock: "
                  f"{100 * res['mfma_util_from_flops']:.1f}%")
    md += ["", f"Source digest of the measured library: `{res['source_digest']}` (bench.py reports `traffic` only "
           "while the sources match)."]
    with open(os.path.join(prof, f"{key}_{args.config}.md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print(json.dumps(res))


if __name__ == "__main__":
    main()
