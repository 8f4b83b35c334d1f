"""Benchmark of the MI355X sparse-conv hot path on one GPU.

A step is one fused submanifold-conv call (weight repack + conv launch) over the whole synthetic workload, with
the kernel map already built (the decoders reuse one map for every conv of a level). Inputs are resident in HBM
before timing starts. The headline workload is config c3 (256^3 grid, ~390k shell voxels, Cin=Cout=256 bf16,
fused bias+SiLU); the default run also measures c2, c4 and c5 the same way (under "extras.configs") and times the
CPU oracle on c1 (the CPU-only 32 -> 32 fp32 config).

value = effective TFLOP/s = 2 * P * Ci * Co / step time, P = active (row, offset) pairs, centre included; the
masked implicit GEMM's padding work is not counted. Roofline per config: MFMA-bound (bf16 dense peak) for the
wide layers c2/c3, HBM-bound (compulsory bytes) for c4/c5. The kernel-map build is timed separately, and the
first call (map + the memoized schedules + first conv) is reported beside the steady step. The cpu_baseline leg
times the CPU oracle (the same operator, fp32 accumulation, multithreaded over the host cores the process may
use) on a bounded random sample of rows of the same workload.
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
METRIC = "sparse-conv effective TFLOPS + Mvoxels/s at 256^3 C=256 bf16; % MFMA/HBM peak"


def host_cpu():
    """Host cores this process may use: the affinity set, capped by the cgroup v2 quota; plus what the machine
    reports, for the record (the two can differ widely in containers)."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    quota_raw, quota = None, None
    try:
        quota_raw = open("/sys/fs/cgroup/cpu.max").read().strip()
        q, p = quota_raw.split()
        if q != "max":
            quota = int(q) / int(p)
    except (OSError, ValueError):
        pass
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    n = aff if quota is None else min(aff, max(1, int(quota)))
    return {"threads": max(1, n), "hardware_concurrency": os.cpu_count(), "affinity": aff, "cpu_max": quota_raw,
            "model": model}


def gemm_ceiling(torch, settle_s, reps):
    """The vendor BLAS's dense bf16 GEMM (8192^3, torch.mm) after the same settle as the conv steps (batches of 10
    until at least settle_s seconds have passed and a batch is no faster than the one before), then `reps` timed
    calls: the sustained MFMA ceiling of this box to set beside the conv kernels."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    ga = torch.randn((8192, 8192), device=dev).to(torch.bfloat16)
    gb = torch.randn((8192, 8192), device=dev).to(torch.bfloat16)
    gc = torch.empty((8192, 8192), device=dev, dtype=torch.bfloat16)

    def batch(k):
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record(stream)
        for _ in range(k):
            torch.mm(ga, gb, out=gc)
        eb.record(stream)
        torch.cuda.synchronize()
        return ea.elapsed_time(eb) / k
    batch(2)
    t0, prev = time.perf_counter(), None
    while True:
        cur = batch(10)
        el = time.perf_counter() - t0
        if (el >= settle_s and prev is not None and cur >= 0.995 * prev) or el >= 5 * max(settle_s, 0.2):
            break
        prev = cur
    ms = batch(reps)
    del ga, gb, gc
    return {"gemm_ms": round(ms, 4), "bf16_gemm_TFLOPs": round(2 * 8192 ** 3 / (ms * 1e-3) / 1e12, 1)}


def cpu_conv_baseline(oracle, np, x, w, b, res, act, nbr_u32, seconds, cpu):
    """Times the oracle conv (fp32, multithreaded over output rows) on a random row sample sized to ~`seconds`."""
    n = nbr_u32.shape[0]
    ci, co = w.shape[2], w.shape[0]
    nt = cpu["threads"]
    rng = np.random.default_rng(0)
    k = 256
    while True:  # grow the pilot until it runs long enough to time, then scale to the requested duration
        rows = rng.choice(n, size=min(n, k), replace=False)
        t = time.perf_counter()
        oracle.conv(x, w, b, nbr_u32, res=res, act=act, rows=rows, nthreads=nt)
        pilot = time.perf_counter() - t
        if pilot > 0.5 or k >= n:
            break
        k *= 4
    k = int(min(n, max(256, k * seconds / max(pilot, 1e-3))))
    rows = rng.choice(n, size=k, replace=False)
    t = time.perf_counter()
    oracle.conv(x, w, b, nbr_u32, res=res, act=act, rows=rows, nthreads=nt)
    cs = time.perf_counter() - t
    pairs = int((nbr_u32[rows] != 0xFFFFFFFF).sum())
    return {"value": round(2.0 * pairs * ci * co / cs / 1e12, 5), "unit": "TFLOP/s", "cores": nt, "kind": "port",
            "sample": f"{k} random rows of {n} ({pairs} active pairs), fp32 oracle conv {ci}->{co}, {cs:.2f}s",
            "mvox_per_s": round(k / cs / 1e6, 4), "hardware_concurrency": cpu["hardware_concurrency"],
            "affinity": cpu["affinity"], "cpu_max": cpu["cpu_max"], "cpu_model": cpu["model"]}


def traffic_for(cfg_name, digest):
    """HBM bytes per launch of the config's conv kernel, from bench_profile.py's FETCH_SIZE + WRITE_SIZE runs --
    only when the figure was measured on the current sources (else None: a stale figure is not reported)."""
    tfile = os.path.join(ROOT, "profiles", f"traffic_{cfg_name}.json")
    if not os.path.exists(tfile):
        return None, None
    t = json.load(open(tfile))
    if t.get("source_digest") != digest:
        return None, t.get("source_digest")
    return round(t["traffic_bytes"]), digest


def measure(name, args, torch, np, sp, W, cpu, want_cpu, cpu_seconds, extras):
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    cfg = W.CONFIGS[name]
    t0 = time.time()
    coords = W.shell_coords(cfg)
    gen_s = time.time() - t0
    lg = None
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

    def step_on(cache):
        sp.subm_conv_fused(x, w, b, cache, residual=res, act=act, out=y)

    # first call on a fresh cache, host-timed with syncs: kernel-map build, then the first conv (which also builds
    # the cache's memoized schedules for this layer shape: tile tables, halo lists), then a second conv. The first
    # such sequence of the process also grows the device memory pool and loads code objects ("process_cold"); the
    # per-cache cost a decoder pays at every level is the same sequence on a second fresh cache ("warm").
    def first_call():
        torch.cuda.synchronize()
        ta = time.perf_counter()
        cc = sp.build_neighbors(tc)
        torch.cuda.synchronize()
        tb = time.perf_counter()
        step_on(cc)
        torch.cuda.synchronize()
        tcv = time.perf_counter()
        step_on(cc)
        torch.cuda.synchronize()
        td = time.perf_counter()
        return cc, {"kmap_ms": round((tb - ta) * 1e3, 3), "first_conv_ms": round((tcv - tb) * 1e3, 3),
                    "second_conv_ms": round((td - tcv) * 1e3, 3), "map_and_first_conv_ms": round((tcv - ta) * 1e3, 3),
                    "schedule_overhead_ms": round(((tcv - tb) - (td - tcv)) * 1e3, 3)}
    cache, cold = first_call()
    del cache
    cache, first = first_call()
    first["process_cold"] = cold

    # kernel-map build alone, HIP events on the library's stream (median after a warm-up)
    map_ms = []
    for i in range(1 + (args.steps if args.kmap_only else 5)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        c2 = sp.build_neighbors(tc)
        e1.record(stream)
        torch.cuda.synchronize()
        del c2
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
        return {"workload": cfg.name, "N": n, "builds": len(map_ms), "kmap_build": kmap}

    nbr, gray, srt = cache.tensors()
    nbr_np = nbr.cpu().numpy()
    P = int((nbr_np != -1).sum())
    # MFMA padding: the kernels skip an offset per group of rows (32 sorted rows in the wide kernel, 16 rows of the
    # windowed order in the narrow / halo ones), so executed pairs = sum over groups of rows x |OR of masks|
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
        step_on(cache)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # settle: the clock under a sustained conv load falls for the first few hundred ms (power management), so keep
    # launching in batches until at least --settle seconds have passed and a batch is no faster than the one before;
    # the timed steps then run at the clock a long run sees (and that a profiler run of the same command averages)
    settle = {"batches": 0, "seconds": 0.0, "batch_ms": []}
    t_settle = time.perf_counter()
    prev = None
    while True:
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record(stream)
        for _ in range(20):
            step()
        eb.record(stream)
        torch.cuda.synchronize()
        cur = ea.elapsed_time(eb) / 20
        settle["batches"] += 1
        settle["batch_ms"].append(round(cur, 4))
        el = time.perf_counter() - t_settle
        if (el >= args.settle and prev is not None and cur >= 0.995 * prev) or el >= 5 * max(args.settle, 0.2):
            break
        prev = cur
    settle["seconds"] = round(time.perf_counter() - t_settle, 3)
    settle["batch_ms"] = settle["batch_ms"][:3] + settle["batch_ms"][-3:]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = e0.elapsed_time(e1) / args.steps
    # the conv kernels alone (HIP events the library records on its stream around each call's conv kernels: the
    # per-call weight repack falls outside), the same number of steps right after
    sp.kernel_timing(True)
    for _ in range(args.steps):
        step()
    sp.kernel_timing(False)
    kts = sp.kernel_times()
    kernel_ms = float(np.mean(kts)) if kts else ms

    flops = 2.0 * P * ci * co
    tflops = flops / (ms * 1e-3) / 1e12
    k_tflops = flops / (kernel_ms * 1e-3) / 1e12
    comp_bytes = n * ci * 2 + n * 27 * 4 + 27 * ci * co * 2 + co * 4 + (n * co * 2 if res is not None else 0) \
        + n * co * 2 + n * 4
    gbs = comp_bytes / (ms * 1e-3) / 1e9
    k_gbs = comp_bytes / (kernel_ms * 1e-3) / 1e9
    wide = ci >= 256 or co >= 256
    traffic, tdig = traffic_for(cfg.name, args.digest)
    # achieved / frac: per conv-kernel launch (algorithmic work / the kernels' event-timed duration); the *_step
    # figures divide by the whole step (weight repack included) instead
    if wide:
        roof = {"bound": "mfma", "achieved": round(k_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(k_tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "achieved_step": round(tflops, 2), "frac_step": round(tflops / PEAK_BF16_TFLOPS, 4)}
    else:
        roof = {"bound": "hbm", "achieved": round(k_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(k_gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                "achieved_step": round(gbs, 1), "frac_step": round(gbs / PEAK_HBM_GBS, 4)}
    roof["kernel_ms"] = round(kernel_ms, 5)
    roof["step_ms"] = round(ms, 5)
    roof["algorithmic_flops"] = flops
    roof["compulsory_bytes"] = comp_bytes
    if traffic is not None:
        roof["traffic_over_compulsory"] = round(traffic / comp_bytes, 3)
    elif tdig:
        roof["traffic_note"] = f"profiles/traffic_{cfg.name}.json was measured on sources {tdig}, not these"

    out = {"workload": f"{cfg.name}: {cfg.grid}^3 shell N={n} Ci={ci} Co={co} bf16 {cfg.epilogue}",
           "N": n, "Ci": ci, "Co": co, "active_pairs": P, "ms_per_step": round(ms, 5),
           "kernel_ms": round(kernel_ms, 5), "settle": settle,
           "tflops": round(tflops, 3), "mvox_per_s": round(n / (ms * 1e-3) / 1e6, 2), "compulsory_GBps": round(gbs, 1),
           "roofline": roof, "kmap_build": kmap, "first_call": first,
           "executed_over_active_pairs": round(executed_pairs / max(P, 1), 4), "skip_group_rows": gsz,
           "coord_gen_s": round(gen_s, 2), "wall_s": round(wall, 3)}

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

    if cfg.subdivide and extras:
        # cascade upsample block end to end: subdivide -> rehash + kernel map -> conv of the children, which read
        # their parents' rows through the c2s map (no gathered child features are written)
        lgt = torch.from_numpy(lg.view(np.int16)).to(dev).view(torch.float16)
        xp = torch.randn((len(coords), ci), generator=g, device=dev).to(torch.bfloat16)
        parts = {"subdivide": [], "kmap": [], "conv": [], "total": [], "synced_total": []}
        for i in range(6):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
            ev[0].record(stream)
            ch, src, cc = sp.subdivide_build(par, lgt)
            ev[1].record(stream)
            sp.subm_conv_gathered(xp, src, 3, w, b, cc, residual=res, act=act, out=y)
            ev[2].record(stream)
            # the same block with the reference's host read of the child count between subdivision and map
            ch2, src2 = sp.subdivide(par, lgt)
            ev[3].record(stream)
            cc2 = sp.build_neighbors(ch2.contiguous())
            sp.subm_conv_gathered(xp, src2, 3, w, b, cc2, residual=res, act=act, out=y)
            ev[4].record(stream)
            torch.cuda.synchronize()
            if i:
                parts["subdivide"].append(ev[2].elapsed_time(ev[3]))
                parts["kmap"].append(ev[0].elapsed_time(ev[1]))
                parts["conv"].append(ev[1].elapsed_time(ev[2]))
                parts["total"].append(ev[0].elapsed_time(ev[2]))
                parts["synced_total"].append(ev[2].elapsed_time(ev[4]))
        e2e = {k + "_ms": round(float(np.median(v)), 4) for k, v in parts.items()}
        e2e["note"] = ("total: subdivide_build (subdivision + children's map, no host sync between them) -> "
                       "subm_conv_gathered on the fresh cache (first-call schedules included); kmap_ms is "
                       "subdivide_build's part, conv_ms the conv's. synced_total: subdivide (host read of the count, "
                       "as the reference) -> build_neighbors -> the same conv; subdivide_ms that path's "
                       "subdivision. HIP events, median of 5")
        # the reference block's second half on the same children (src/sdec.cu:76-84): conv1's output h1 [n, 8*Co]
        # (random here) -> child rows -> LayerNorm -> SiLU -> conv2 (Co -> Co) -> skip add from the parents' x
        co2 = co
        h1 = torch.randn((len(coords) * 8, co2), generator=g, device=dev).to(torch.bfloat16)
        w2 = (torch.randn((co2, 27, co2), generator=g, device=dev) * 0.05).to(torch.bfloat16)
        b2 = torch.zeros(co2, device=dev)
        y2 = torch.empty((len(ch), co2), dtype=torch.bfloat16, device=dev)

        def half_gathered_rows():
            sp.subm_conv_fused(sp.gather_ln_act(h1, src, 0), w2, b2, cc, out=y2)
            sp.add_skip(y2, xp, src)

        def half_fused_skip():
            sp.subm_conv_skip(sp.gather_ln_act(h1, src, 0), w2, b2, cc, xp, src, out=y2)

        def half_one_kernel():  # gather + LayerNorm + SiLU + conv2 + skip in the halo kernel
            sp.subm_conv_preln(h1, w2, b2, cc, src, 0, None, None, 1e-6, sp.ACT_SILU, x_skip=xp, skip_src=src, out=y2)

        def torch_preact():
            torch.nn.functional.silu(torch.nn.functional.layer_norm(h1[src.long()].float(), (co2,), eps=1e-6)).to(
                torch.bfloat16)
        prev_env = os.environ.get("SPCONV_PRELN_FUSED")
        os.environ["SPCONV_PRELN_FUSED"] = "1"  # the one-kernel form is opt-in (read per call)
        try:
            one_kernel_ms = round(timed(half_one_kernel, 10), 4)
        finally:
            if prev_env is None:
                os.environ.pop("SPCONV_PRELN_FUSED", None)
            else:
                os.environ["SPCONV_PRELN_FUSED"] = prev_env
        e2e["second_half"] = {
            "children": len(ch), "Co": co2,
            "gather_ln_silu_then_conv_ms": round(timed(half_gathered_rows, 10), 4),
            "gather_ln_silu_then_conv_skip_fused_ms": round(timed(half_fused_skip, 10), 4),
            "preln_conv_skip_one_kernel_ms": one_kernel_ms,
            "gather_ln_silu_ms": round(timed(lambda: sp.gather_ln_act(h1, src, 0), 20), 4),
            "torch_gather_ln_silu_ms": round(timed(torch_preact, 20), 4),
            "add_skip_ms": round(timed(lambda: sp.add_skip(y2, xp, src), 20), 4)}
        out["upsample_block_e2e"] = e2e
        del h1, xp

    if co in (64, 128, 256) and extras:
        # the decoder's ConvNeXt tail on this layer's output rows (LayerNorm + affine -> Linear 4C + SiLU -> Linear
        # C -> + x, reference src/sdec.cu:60-66), fused, against torch's unfused sequence on the same tensors
        hx = torch.randn((n, co), generator=g, device=dev).to(torch.bfloat16)
        xx = torch.randn((n, co), generator=g, device=dev).to(torch.bfloat16)
        gmm, bt = torch.ones(co, device=dev), torch.zeros(co, device=dev)
        w1 = (torch.randn((4 * co, co), generator=g, device=dev) / co ** 0.5).to(torch.bfloat16)
        w2 = (torch.randn((co, 4 * co), generator=g, device=dev) / (2 * co)).to(torch.bfloat16)
        b1, b2 = torch.zeros(4 * co, device=dev), torch.zeros(co, device=dev)
        yt = torch.empty_like(hx)
        t_f = timed(lambda: sp.convnext_mlp(hx, xx, gmm, bt, w1, b1, w2, b2, out=yt), 10)

        def torch_tail():
            a = torch.nn.functional.layer_norm(hx.float(), (co,), gmm, bt, 1e-6).to(torch.bfloat16)
            a = torch.nn.functional.silu(torch.nn.functional.linear(a, w1, b1.to(torch.bfloat16)))
            return torch.nn.functional.linear(a, w2, b2.to(torch.bfloat16)) + xx
        t_t = timed(torch_tail, 5)
        out["convnext_tail"] = {"rows": n, "C": co, "fused_ms": round(t_f, 4), "torch_ms": round(t_t, 4),
                                "fused_GBps": round(3 * n * co * 2 / (t_f * 1e-3) / 1e9, 1),
                                "fused_TFLOPs": round(16 * n * co * co / (t_f * 1e-3) / 1e12, 1)}
        del hx, xx, yt

    if want_cpu:
        import oracle
        rs = res.float().cpu().numpy() if res is not None else None
        out["cpu_baseline"] = cpu_conv_baseline(oracle, np, x.float().cpu().numpy(), w.float().cpu().numpy(),
                                                b.cpu().numpy(), rs, act, nbr_np.view(np.uint32), cpu_seconds, cpu)
    del x, w, res, y, cache
    return out


# The sparse decoders' conv shapes beyond the five configs: (log2 N, Ci, Co) from the reference's autotune keys
# (assets/flexgemm_autotune.json: ConvNeXt convs C -> C and up-convs C -> 8 * C/2 at each level, N from 2^11 at
# C = 1024 to 2^21 at C = 64).
DECODER_LEVELS = [(11, 1024, 1024), (11, 1024, 4096), (14, 512, 512), (14, 512, 2048), (16, 256, 256),
                  (16, 256, 1024), (19, 128, 128), (19, 128, 512), (21, 64, 64)]


def upsample_only(args, torch, np, sp, W):
    """The cascade upsample block of a subdivision workload (c5) alone, --steps times after one untimed block: c2s
    subdivision + the children's map (subdivide_build, no host sync between them) -> the children's conv on the fresh
    cache, reading the parents' rows through the c2s map (first-call schedules included). The profiling command of
    the upsample-block summary (bench_profile.py --upsample)."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    cfg = W.CONFIGS[args.config]
    if not cfg.subdivide:
        sys.exit(f"--upsample-only needs a subdivision workload (c5), not {args.config}")
    coords = W.shell_coords(cfg)
    par = torch.from_numpy(coords).to(dev)
    lg = W.keep_logits(len(coords), cfg.keep_frac, cfg.seed)
    lgt = torch.from_numpy(lg.view(np.int16)).to(dev).view(torch.float16)
    g = torch.Generator(device=dev)
    g.manual_seed(cfg.seed)
    xp = torch.randn((len(coords), cfg.ci), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((cfg.co, 27, cfg.ci), generator=g, device=dev) / (27 * cfg.ci) ** 0.5).to(torch.bfloat16)
    b = torch.randn((cfg.co,), generator=g, device=dev) * 0.1
    act = sp.ACT_SILU if "silu" in cfg.epilogue else sp.ACT_NONE
    parts = {"kmap": [], "conv": [], "total": []}
    m = 0
    for i in range(1 + args.steps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        ev[0].record(stream)
        ch, src, cc = sp.subdivide_build(par, lgt)
        ev[1].record(stream)
        y = torch.empty((len(ch), cfg.co), dtype=torch.bfloat16, device=dev)
        sp.subm_conv_gathered(xp, src, 3, w, b, cc, act=act, out=y)
        ev[2].record(stream)
        torch.cuda.synchronize()
        m = len(ch)
        if i:
            parts["kmap"].append(ev[0].elapsed_time(ev[1]))
            parts["conv"].append(ev[1].elapsed_time(ev[2]))
            parts["total"].append(ev[0].elapsed_time(ev[2]))
        del ch, src, cc, y
    return {"workload": f"{args.config} upsample block: {len(coords)} parents -> {m} children, "
                        f"{cfg.ci}->{cfg.co} gathered conv", "parents": len(coords), "children": m,
            "blocks": args.steps, **{k + "_ms": round(float(np.median(v)), 4) for k, v in parts.items()},
            "note": "kmap_ms = subdivide_build (subdivision + children's map); conv_ms = the gathered conv on the "
                    "fresh cache, first-call schedules included; HIP events, median"}


def decoder_levels(torch, np, sp, W):
    """Conv kernel time at each decoder level's shape on a seeded shell of ~2^L voxels (the c3 recipe with the grid
    scaled to the voxel count), bias + SiLU, bf16; HIP events around the conv kernels, median of 20 calls."""
    dev = torch.device("cuda:0")
    out = []
    for L, ci, co in DECODER_LEVELS:
        G = max(16, int(256 * ((1 << L) / 390500) ** 0.5))
        cfg = W.Config("level", G, 12, (20 * G / 256, 90 * G / 256), True, 0.8, ci, co, "bf16", "bias+silu", 7000 + L)
        c = torch.from_numpy(W.shell_coords(cfg)).to(dev)
        n = c.shape[0]
        cache = sp.build_neighbors(c)
        P = int((cache.tensors()[0] != -1).sum().item())
        g = torch.Generator(device=dev)
        g.manual_seed(cfg.seed)
        x = torch.randn((n, ci), generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn((co, 27, ci), generator=g, device=dev) / (27 * ci) ** 0.5).to(torch.bfloat16)
        b = torch.randn((co,), generator=g, device=dev) * 0.1
        y = torch.empty((n, co), dtype=torch.bfloat16, device=dev)
        for _ in range(10):
            sp.subm_conv_fused(x, w, b, cache, act=sp.ACT_SILU, out=y)
        sp.kernel_timing(True)
        for _ in range(20):
            sp.subm_conv_fused(x, w, b, cache, act=sp.ACT_SILU, out=y)
        sp.kernel_timing(False)
        kt = float(np.median(sp.kernel_times()))
        fl = 2.0 * P * ci * co
        out.append({"log2N": L, "N": n, "Ci": ci, "Co": co, "active_pairs": P, "kernel_ms": round(kt, 4),
                    "tflops": round(fl / (kt * 1e-3) / 1e12, 1),
                    "frac_of_mfma_peak": round(fl / (kt * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)})
        del cache, x, w, y
    return out


def c1_cpu(np, W, cpu, seconds):
    """Config c1 runs on the CPU only: 32^3 shell, 32 -> 32 fp32 with bias, the oracle's kernel map and conv over
    every row (repeated to fill ~`seconds`)."""
    import oracle
    cfg = W.CONFIGS["c1"]
    c = W.shell_coords(cfg)
    t = time.perf_counter()
    nbr, _, _, _ = oracle.build_neighbors(c)
    map_s = time.perf_counter() - t
    w, b = W.conv_params(cfg)
    x = W.features(len(c), cfg.ci, 1)
    reps, tot = 0, 0.0
    while tot < seconds or reps < 3:
        t = time.perf_counter()
        oracle.conv(x, w, b, nbr, nthreads=cpu["threads"])
        tot += time.perf_counter() - t
        reps += 1
    P = int((nbr != 0xFFFFFFFF).sum())
    s = tot / reps
    return {"workload": f"c1: {cfg.grid}^3 sphere shell N={len(c)} Ci={cfg.ci} Co={cfg.co} fp32 bias (CPU only)",
            "N": len(c), "active_pairs": P, "conv_ms": round(s * 1e3, 4),
            "value": round(2.0 * P * cfg.ci * cfg.co / s / 1e12, 5), "unit": "TFLOP/s",
            "mvox_per_s": round(len(c) / s / 1e6, 3), "kmap_build_ms": round(map_s * 1e3, 3), "cores": cpu["threads"],
            "reps": reps, "kind": "port"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c3")
    ap.add_argument("--settle", type=float, default=1.0,
                    help="seconds of untimed launches after --warmup, until the per-launch time stops falling")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline legs")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU work of the headline cpu_baseline")
    ap.add_argument("--cpu-seconds-extra", type=float, default=4.0, help="CPU work of each other config's baseline")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured copy / GEMM ceilings")
    ap.add_argument("--no-extras", action="store_true",
                    help="only the one config: no other configs, upsample-block or ConvNeXt-tail extras (profiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device-to-device copy (the counter calibration used by bench_profile.py)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only time the vendor dense bf16 GEMM ceiling (8192^3 torch.mm, settled; --steps calls): the "
                         "profiling command of the GEMM reference summary")
    ap.add_argument("--upsample-only", action="store_true",
                    help="only time the cascade upsample block of a subdivision workload (--config c5; --steps "
                         "blocks): the profiling command of the upsample-block summary")
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
    if args.gemm_only:
        import torch
        print(json.dumps(gemm_ceiling(torch, args.settle, args.steps)), flush=True)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every box has one GPU).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import spconv_amd as sp
    from spconv_amd import workloads as W

    sp.load_library()
    sp.set_stream(torch.cuda.current_stream())
    args.digest = sp.source_digest()
    cpu = host_cpu()
    if args.kmap_only:
        print(json.dumps(measure(args.config, args, torch, np, sp, W, cpu, False, 0, False)), flush=True)
        return
    if args.upsample_only:
        print(json.dumps(upsample_only(args, torch, np, sp, W)), flush=True)
        return
    extras = not args.no_extras
    head = measure(args.config, args, torch, np, sp, W, cpu, not args.no_cpu, args.cpu_seconds, extras)

    # measured ceilings on this box, for context next to the spec peaks the roofline uses: a 1 GiB device copy
    # (read + write bytes / time) and a large dense bf16 GEMM through the vendor BLAS
    stream = torch.cuda.current_stream()

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
        dev = torch.device("cuda:0")
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        copy_gbs = 2 * (1 << 30) / (timed(lambda: dst.copy_(src), 5) * 1e-3) / 1e9
        del src, dst
        g = gemm_ceiling(torch, args.settle, 20)
        gemm_tf = g["bf16_gemm_TFLOPs"]
        measured = {"hbm_copy_GBps": round(copy_gbs, 1), "bf16_gemm_TFLOPs": gemm_tf, "bf16_gemm_settled": True}
        r = head["roofline"]
        measured["frac_of_measured"] = round(r["achieved"] / (gemm_tf if r["bound"] == "mfma" else copy_gbs), 4)

    others = {}
    if extras:
        for name in ("c2", "c3", "c4", "c5"):
            if name != args.config:
                torch.cuda.empty_cache()
                others[name] = measure(name, args, torch, np, sp, W, cpu, not args.no_cpu, args.cpu_seconds_extra,
                                       True)
        if not args.no_cpu:
            others["c1"] = c1_cpu(np, W, cpu, args.cpu_seconds_extra)
        torch.cuda.empty_cache()
        levels = decoder_levels(torch, np, sp, W)

    r = head["roofline"]
    cfg = {k: head[k] for k in ("workload", "N", "Ci", "Co", "active_pairs")}
    keep = {k: v for k, v in head.items() if k not in ("roofline", "cpu_baseline", "workload", "N", "Ci", "Co",
                                                         "active_pairs", "ms_per_step", "tflops")}
    out = {
        "metric": METRIC,
        "value": head["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded union-of-shapes shell, random N(0,1) features, N(0,1/(27Ci)) "
                                 "weights)",
        "config": cfg,
        "roofline": {k: r[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel_ms", "step_ms",
                                       "achieved_step", "frac_step")},
        "cpu_baseline": head.get("cpu_baseline"),
        "extras": dict(keep, roofline_detail=r, measured_peaks=measured, configs=others, source_digest=args.digest,
                       host_cpu=cpu, decoder_levels=levels if extras else None),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
