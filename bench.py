"""Benchmark of the MI355X sparse-conv hot path on one GPU.

A step is one fused submanifold-conv launch over the whole synthetic workload (default: config c3, 256^3 grid,
~390k shell voxels, Cin=Cout=256 bf16, fused bias+SiLU), with the kernel map already built (the decoders reuse one
map for every conv of a level). Inputs are resident in HBM before timing starts. The kernel-map build (hash +
neighbours + sort + block masks) is timed separately and reported under "extras".

value = effective TFLOP/s = 2 * P * Ci * Co / time, P = active (row, offset) pairs, centre included; the masked
implicit GEMM's padding work is not counted. The cpu_baseline leg times the CPU oracle (the same operator, fp32
accumulation, multithreaded) on a bounded sample of rows of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "trellis2-cuda_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    try:  # cgroup v2 quota
        q, p = open("/sys/fs/cgroup/cpu.max").read().split()
        if q != "max":
            n = min(n, max(1, int(int(q) / int(p))))
    except (OSError, ValueError):
        pass
    return max(1, min(n, 16))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured copy / GEMM ceilings")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the upsample-block and ConvNeXt-tail extras (profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device-to-device copy (the counter calibration used by bench_profile.py)")
    ap.add_argument("--kmap-only", action="store_true",
                    help="only time the kernel-map build of the workload (--steps builds; the profiling command of the "
                         "kernel-map summary)")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every box has one GPU).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import spconv_amd as sp
    from spconv_amd import workloads as W

    dev = torch.device("cuda:0")
    sp.load_library()
    sp.set_stream(torch.cuda.current_stream())
    cfg = W.CONFIGS[args.config]
    t0 = time.time()
    coords = W.shell_coords(cfg)
    gen_s = time.time() - t0
    if cfg.subdivide:  # c5: parents at C=128 -> kept children are the conv's rows
        par = torch.from_numpy(coords).to(dev)
        lg = W.keep_logits(len(coords), cfg.keep_frac, cfg.seed)
        child, _ = sp.subdivide(par, torch.from_numpy(lg.view(np.int16)).to(dev).view(torch.float16))
        tc = child.contiguous()
    else:
        tc = torch.from_numpy(coords).to(dev)
    n = tc.shape[0]
    ci, co = cfg.ci, cfg.co
    g = torch.Generator(device=dev)
    g.manual_seed(cfg.seed)
    x = torch.randn((n, ci), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((co, 27, ci), generator=g, device=dev) / (27 * ci) ** 0.5).to(torch.bfloat16)
    b = torch.randn((co,), generator=g, device=dev) * 0.1
    res = torch.randn((n, co), generator=g, device=dev).to(torch.bfloat16) if "res" in cfg.epilogue else None
    act = sp.ACT_SILU if "silu" in cfg.epilogue else sp.ACT_NONE
    y = torch.empty((n, co), dtype=torch.bfloat16, device=dev)

    # kernel-map build, timed separately (median after a warm-up)
    stream = torch.cuda.current_stream()
    map_ms = []
    for i in range(1 + (args.steps if args.kmap_only else 5)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        cache = sp.build_neighbors(tc)
        e1.record(stream)
        torch.cuda.synchronize()
        if i:
            map_ms.append(e0.elapsed_time(e1))
    # algorithmic bytes of one build (once each): coords 16 B/voxel, table init + insert 12 B/slot at the reference's
    # capacity (pow2 >= 2N), nbr 108 B/voxel, mask + decoded mask 8, sort in/out 8
    cap = 1
    while cap < 2 * n:
        cap *= 2
    map_bytes = n * (16 + 108 + 8 + 8) + cap * 12
    map_med = float(np.median(map_ms))
    kmap = {"ms": round(map_med, 4), "algorithmic_bytes": map_bytes,
            "achieved_GBps": round(map_bytes / (map_med * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(map_bytes / (map_med * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    if args.kmap_only:
        print(json.dumps({"workload": cfg.name, "N": n, "builds": len(map_ms), "kmap_build": kmap}), flush=True)
        return
    nbr, gray, srt = cache.tensors()
    nbr_np = nbr.cpu().numpy()
    P = int((nbr_np != -1).sum())
    B1 = sp.spconv_cfg(n, ci, co)[0]
    # MFMA padding: the kernels skip an offset per group of rows (32 sorted rows in the wide kernel, 16 rows of the
    # 65536-row windowed order in the narrow one), so executed pairs = sum over groups of rows x |OR of masks|
    narrow = co == 64 and ci <= 128
    halo = co == 64 and ci == 64 and not os.environ.get("SPCONV_NO_HALO")  # 256-row windows (halo kernel)
    gsz = 16 if narrow else 32
    order = srt.cpu().numpy().astype(np.int64)
    if narrow:
        order = order[np.argsort(order >> (8 if halo else 16), kind="stable")]
    gm = gray.cpu().numpy().astype(np.int64)[order]
    ng = (n + gsz - 1) // gsz
    pad = np.zeros(ng * gsz, np.int64)
    pad[:n] = gm
    orm = np.bitwise_or.reduce(pad.reshape(ng, gsz), axis=1)
    cnt = sum((orm >> v) & 1 for v in range(27))
    executed_pairs = int((cnt * np.minimum(gsz, n - np.arange(ng) * gsz)).sum())

    def step():
        sp.subm_conv_fused(x, w, b, cache, residual=res, act=act, out=y)

    # the first call also builds the cache's memoized schedules for this layer shape (tile tables, halo lists)
    torch.cuda.synchronize()
    t_first = time.perf_counter()
    step()
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t_first) * 1e3
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = e0.elapsed_time(e1) / args.steps

    flops = 2.0 * P * ci * co
    tflops = flops / (ms * 1e-3) / 1e12
    comp_bytes = n * ci * 2 + n * 27 * 4 + 27 * ci * co * 2 + co * 4 + (n * co * 2 if res is not None else 0) \
        + n * co * 2 + n * 4
    gbs = comp_bytes / (ms * 1e-3) / 1e9
    mvox = n / (ms * 1e-3) / 1e6
    wide = ci >= 256 or co >= 256
    traffic = None
    tfile = os.path.join(ROOT, "profiles", f"traffic_{cfg.name}.json")
    if os.path.exists(tfile):  # HBM bytes per launch measured by bench_profile.py (FETCH_SIZE + WRITE_SIZE)
        traffic = round(json.load(open(tfile))["traffic_bytes"])
    if wide:
        roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic}
    else:
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic}

    # measured ceilings on this box, for context next to the spec peaks the roofline uses: a 1 GiB device copy
    # (read + write bytes / time) and a large dense bf16 GEMM through the vendor BLAS
    def timed(f, reps):
        f()
        torch.cuda.synchronize()
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record(stream)
        for _ in range(reps):
            f()
        eb.record(stream)
        torch.cuda.synchronize()
        return ea.elapsed_time(eb) / reps
    measured = None
    if not args.no_peaks:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        copy_gbs = 2 * (1 << 30) / (timed(lambda: dst.copy_(src), 5) * 1e-3) / 1e9
        del src, dst
        ga = torch.randn((8192, 8192), device=dev).to(torch.bfloat16)
        gb = torch.randn((8192, 8192), device=dev).to(torch.bfloat16)
        gemm_tf = 2 * 8192 ** 3 / (timed(lambda: torch.mm(ga, gb), 10) * 1e-3) / 1e12
        del ga, gb
        measured = {"hbm_copy_GBps": round(copy_gbs, 1), "bf16_gemm_TFLOPs": round(gemm_tf, 1),
                    "frac_of_measured": round((tflops / gemm_tf) if wide else (gbs / copy_gbs), 4)}

    e2e = None
    if cfg.subdivide and not args.no_extras:
        # cascade upsample block end to end: subdivide -> rehash + kernel map -> conv of the children, which read
        # their parents' rows through the c2s map (no gathered child features are written)
        lgt = torch.from_numpy(lg.view(np.int16)).to(dev).view(torch.float16)
        xp = torch.randn((len(coords), ci), generator=g, device=dev).to(torch.bfloat16)
        parts = {"subdivide": [], "kmap": [], "conv": [], "total": []}
        for i in range(4):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            ev[0].record(stream)
            ch, src = sp.subdivide(par, lgt)
            ev[1].record(stream)
            c2 = sp.build_neighbors(ch.contiguous())
            ev[2].record(stream)
            sp.subm_conv_gathered(xp, src, 3, w, b, c2, residual=res, act=act, out=y)
            ev[3].record(stream)
            torch.cuda.synchronize()
            if i:
                parts["subdivide"].append(ev[0].elapsed_time(ev[1]))
                parts["kmap"].append(ev[1].elapsed_time(ev[2]))
                parts["conv"].append(ev[2].elapsed_time(ev[3]))
                parts["total"].append(ev[0].elapsed_time(ev[3]))
        e2e = {k + "_ms": round(float(np.median(v)), 4) for k, v in parts.items()}
        # the reference block's second half on the same children (src/sdec.cu:76-84): conv1's output h1 [n, 8*Co]
        # (random here) -> child rows -> LayerNorm -> SiLU -> conv2 (Co -> Co) -> skip add from the parents' x
        co2 = co
        h1 = torch.randn((len(coords) * 8, co2), generator=g, device=dev).to(torch.bfloat16)
        w2 = (torch.randn((co2, 27, co2), generator=g, device=dev) * 0.05).to(torch.bfloat16)
        b2 = torch.zeros(co2, device=dev)
        y2 = torch.empty((len(ch), co2), dtype=torch.bfloat16, device=dev)

        def half_gathered_rows():
            sp.subm_conv_fused(sp.gather_ln_act(h1, src, 0), w2, b2, c2, out=y2)
            sp.add_skip(y2, xp, src)

        def half_fused_skip():
            sp.subm_conv_skip(sp.gather_ln_act(h1, src, 0), w2, b2, c2, xp, src, out=y2)

        def half_gathered_conv():
            sp.subm_conv_gathered(sp.gather_ln_act(h1), src, 0, w2, b2, c2, out=y2)
            sp.add_skip(y2, xp, src)

        def torch_preact():
            torch.nn.functional.silu(torch.nn.functional.layer_norm(h1[src.long()].float(), (co2,), eps=1e-6)).to(
                torch.bfloat16)
        e2e["second_half"] = {
            "children": len(ch), "Co": co2,
            "gather_ln_silu_then_conv_ms": round(timed(half_gathered_rows, 10), 4),
            "gather_ln_silu_then_conv_skip_fused_ms": round(timed(half_fused_skip, 10), 4),
            "ln_silu_parents_then_gathered_conv_ms": round(timed(half_gathered_conv, 10), 4),
            "gather_ln_silu_ms": round(timed(lambda: sp.gather_ln_act(h1, src, 0), 20), 4),
            "torch_gather_ln_silu_ms": round(timed(torch_preact, 20), 4),
            "add_skip_ms": round(timed(lambda: sp.add_skip(y2, xp, src), 20), 4)}

    # the decoder's ConvNeXt tail on this layer's output rows (LayerNorm + affine -> Linear 4C + SiLU -> Linear C ->
    # + x, reference src/sdec.cu:60-66), fused, against torch's unfused sequence on the same tensors
    tail = None
    if co in (64, 128, 256) and not args.no_extras:
        hx = torch.randn((n, co), generator=g, device=dev).to(torch.bfloat16)
        xx = torch.randn((n, co), generator=g, device=dev).to(torch.bfloat16)
        gm, bt = torch.ones(co, device=dev), torch.zeros(co, device=dev)
        w1 = (torch.randn((4 * co, co), generator=g, device=dev) / co ** 0.5).to(torch.bfloat16)
        w2 = (torch.randn((co, 4 * co), generator=g, device=dev) / (2 * co)).to(torch.bfloat16)
        b1, b2 = torch.zeros(4 * co, device=dev), torch.zeros(co, device=dev)
        yt = torch.empty_like(hx)
        t_f = timed(lambda: sp.convnext_mlp(hx, xx, gm, bt, w1, b1, w2, b2, out=yt), 10)

        def torch_tail():
            a = torch.nn.functional.layer_norm(hx.float(), (co,), gm, bt, 1e-6).to(torch.bfloat16)
            a = torch.nn.functional.silu(torch.nn.functional.linear(a, w1, b1.to(torch.bfloat16)))
            return torch.nn.functional.linear(a, w2, b2.to(torch.bfloat16)) + xx
        t_t = timed(torch_tail, 5)
        tail = {"rows": n, "C": co, "fused_ms": round(t_f, 4), "torch_ms": round(t_t, 4),
                "fused_GBps": round(3 * n * co * 2 / (t_f * 1e-3) / 1e9, 1),
                "fused_TFLOPs": round(16 * n * co * co / (t_f * 1e-3) / 1e12, 1)}
        del hx, xx, yt

    cpu = None
    if not args.no_cpu:
        import oracle
        nt = cpu_threads()
        onbr = nbr_np.view(np.uint32)
        xs = x.float().cpu().numpy()
        ws = w.float().cpu().numpy()
        bs = b.cpu().numpy()
        rs = res.float().cpu().numpy() if res is not None else None
        rng = np.random.default_rng(0)
        k = 256
        while True:  # grow the pilot until it runs long enough to time, then scale to the requested duration
            rows = rng.choice(n, size=min(n, k), replace=False)
            t = time.perf_counter()
            oracle.conv(xs, ws, bs, onbr, res=rs, act=act, rows=rows, nthreads=nt)
            pilot = time.perf_counter() - t
            if pilot > 0.5 or k >= n:
                break
            k *= 4
        k = int(min(n, max(256, k * args.cpu_seconds / max(pilot, 1e-3))))
        rows = rng.choice(n, size=k, replace=False)
        t = time.perf_counter()
        oracle.conv(xs, ws, bs, onbr, res=rs, act=act, rows=rows, nthreads=nt)
        cs = time.perf_counter() - t
        pairs = int((nbr_np[rows] != -1).sum())
        cpu = {"value": round(2.0 * pairs * ci * co / cs / 1e12, 5), "unit": "TFLOP/s", "cores": nt,
               "kind": "port",
               "sample": f"{k} random rows of {n} ({pairs} active pairs), fp32 oracle conv, {cs:.1f}s",
               "mvox_per_s": round(k / cs / 1e6, 4)}

    out = {
        "metric": "sparse-conv effective TFLOPS + Mvoxels/s at 256^3 C=256 bf16; % MFMA/HBM peak",
        "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded union-of-shapes shell, random N(0,1) features)",
        "config": {"workload": f"{cfg.name}: {cfg.grid}^3 shell N={n} Ci={ci} Co={co} bf16 {cfg.epilogue}",
                   "N": n, "Ci": ci, "Co": co, "active_pairs": P},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extras": {"mvox_per_s": round(mvox, 2), "compulsory_GBps": round(gbs, 1),
                   "kmap_build_ms": round(map_med, 4), "kmap_build": kmap, "first_call_ms": round(first_ms, 3),
                   "coord_gen_s": round(gen_s, 2),
                   "executed_over_active_pairs": round(executed_pairs / max(P, 1), 4), "skip_group_rows": gsz, "wall_s": round(wall, 3),
                   "upsample_block_e2e": e2e, "convnext_tail": tail, "measured_peaks": measured},
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
