"""Benchmark of the fused residual-add + RMSNorm path on one MI355X.

Workload (BASELINE.json's metric): bf16 fused add+RMSNorm at (4096, H) for
every H of configs[1] (1024 ... 12288 step 1024) and configs[2] (13312 ...
32768).  One step = one call at each of those H, in order.  Inputs are
resident in HBM before timing starts; every H has two buffer sets used
alternately, and one step moves ~3.8 GB, so no call finds its rows in the
256 MB Infinity Cache left over from its previous use.

value      = algorithmic bytes of a step / time of a step (GB/s), where a
             call at (B, H) moves (4*B*H + H) * 2 bytes: input and residual
             read, residual and output written, weight read once.
per_shape  = per-H microseconds per call and GB/s: back-to-back calls over
             rotating buffer sets spanning >= 1 GiB (so every call is cold in
             the Infinity Cache), one HIP event pair around them on the
             stream the kernels run on; the median and p10/p90 over 7 such
             blocks.  Each timed region starts behind a short spin kernel so
             the host's launch rate is not measured.
roofline   = the kernel instantiation with the largest share of the step
             time, against MI355X's 8 TB/s HBM peak.
cpu_baseline = the reference's CPU path: its test's torch formula
               (x + r; torch.rms_norm) in eager mode on the host's usable
               cores, on the whole workload; core count and CPU model stated.
cpu_oracle   = the CPU oracle (a scalar C restatement, OpenMP over rows) on a
               bounded sample of the same shapes.
details    = printed before the bench line, one JSON line per section
             ({"bench_detail": name, "data": ...}): BASELINE.json's other
             configs (decode, fp16, streamer) and the other operators (FP8 /
             MX outputs, out-of-place, plain RMSNorm, rows off the 128-byte
             grid, partial sums), µs/call; a copy moving the fused op's bytes
             at six of the widths, with the fused op's time as a fraction of
             it; the ceiling leg; the CPU baseline per shape.  The bench line
             itself (the last stdout line) stays under HEADLINE_MAX_BYTES.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--full-json PATH]
       python bench.py --sweep STEP [--sweep-max H]   (per-H table sweep, one JSON line per H)
       python bench.py --ab 'H:lpr,vpl,ldsv,block,flags;...' ... [--hot]
                      (forced bench-library configurations against the table's, one JSON line each)
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "µs/call + achieved HBM GB/s, fused add+RMSNorm bf16 (4096,H), H=1K–32K"
PEAK_GBS = 8000.0
B = 4096
H_SWEEP = list(range(1024, 12288 + 1, 1024)) + [13312, 14336, 16384, 20480, 24576, 28672, 32768]
EPS = 1e-6


def fused_bytes(rows, hidden, elem=2):
    return (4 * rows * hidden + hidden) * elem


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_set(torch, rows, hidden, dtype, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn((rows, hidden), generator=g, device=dev, dtype=torch.float32).to(dtype)
    r = torch.randn((rows, hidden), generator=g, device=dev, dtype=torch.float32).to(dtype)
    return x, r


def make_weight(torch, hidden, dtype, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (1 + 0.1 * torch.randn((hidden,), generator=g, device=dev)).to(dtype)


def kernel_key(abi, rows, hidden, dtype_code):
    """The table's configuration for contiguous rows on this device's CUs."""
    c = abi.select_config(rows, hidden, dtype_code, cus=abi.device_cu_count())
    return c.as_tuple()


_SLEEP_CYCLES_PER_MS = None


def prefill(torch, ms):
    """Queue a spin kernel of about `ms` so the host gets ahead of the GPU:
    the launches that follow are queued while it runs, and the timed region
    measures the GPU, not Python's launch rate."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(_SLEEP_CYCLES_PER_MS * ms))


def make_bufs(torch, shapes, nsets_for, dev="cuda:0"):
    bufs = []
    for i, (rows, hidden, dtype, dist) in enumerate(shapes):
        sets = [make_set(torch, rows, hidden, dtype, 1000 * i + s, dev) for s in range(nsets_for(rows, hidden))]
        if dist == "outliers":
            for x, _ in sets:
                g = torch.Generator(device=dev).manual_seed(7 + i)
                m = torch.rand(x.shape, generator=g, device=dev) < 0.01
                x.copy_(torch.where(m, x.float() * 50, x.float()).to(dtype))
        bufs.append((sets, make_weight(torch, hidden, dtype, i, dev)))
    torch.cuda.synchronize()
    return bufs


def time_step(torch, op, shapes, steps, warmup):
    """One step = one call per shape, in order; two buffer sets per shape used
    alternately.  Returns the mean step time (ms) over `steps` timed steps."""
    bufs = make_bufs(torch, shapes, lambda r, h: 2)
    for it in range(warmup):
        for sets, w in bufs:
            x, r = sets[it % 2]
            op(x, w, r, EPS)
    stream = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    prefill(torch, 20)
    t0.record(stream)
    for it in range(steps):
        for sets, w in bufs:
            x, r = sets[(warmup + it) % 2]
            op(x, w, r, EPS)
    t1.record(stream)
    torch.cuda.synchronize()
    del bufs
    torch.cuda.empty_cache()
    return t0.elapsed_time(t1) / steps


def cold_sets(rows, hidden, elem=2, floor=2, span=1 << 30):
    """Buffer sets so that one pass over them spans >= 1 GiB (4x the MALL)."""
    return max(floor, min(256, -(-span // (2 * rows * hidden * elem))))


def spread(samples):
    """(median, p10, p90) of a list of timings."""
    if len(samples) == 1:
        return samples[0], samples[0], samples[0]
    q = statistics.quantiles(samples, n=10, method="inclusive")
    return statistics.median(samples), q[0], q[8]


def time_shapes(torch, op, shapes, calls, warmup, trials=7):
    """Per shape: `trials` timed blocks, each of `calls` back-to-back calls
    over rotating buffer sets spanning >= 1 GiB with one HIP event pair around
    it.  Returns (median, p10, p90) over the trials of µs per call."""
    out = []
    for shape in shapes:
        rows, hidden = shape[0], shape[1]
        bufs = make_bufs(torch, [shape], lambda r, h: cold_sets(r, h))
        sets, w = bufs[0]
        n = len(sets)
        for it in range(warmup):
            x, r = sets[it % n]
            op(x, w, r, EPS)
        stream = torch.cuda.current_stream()
        ncalls = max(calls, n)
        samples = []
        base = warmup
        for _ in range(trials):
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            prefill(torch, 10)
            t0.record(stream)
            for it in range(ncalls):
                x, r = sets[(base + it) % n]
                op(x, w, r, EPS)
            t1.record(stream)
            torch.cuda.synchronize()
            base += ncalls
            samples.append(t0.elapsed_time(t1) * 1e3 / ncalls)
        out.append(spread(samples))
        del bufs, sets
        torch.cuda.empty_cache()
    return out


def usable_cpus():
    """CPUs this process may run on: its affinity set, capped by a cgroup v2
    CPU quota when one is set (a box may show more cores than it grants)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_torch_baseline(torch, shapes=None, reps=3):
    """The reference's CPU path: its test's formula (test/test_hp_rms_norm.py:6-19),
    ``s = x + r; torch.rms_norm(s, (H,), weight=w, eps=eps)``, in torch eager
    mode on the host's usable cores, on the benchmark's own shapes (bf16,
    4096 rows, every H of the sweep) and distributions.  Per shape: 1 warm-up
    call, then the median of `reps` timed calls (time.perf_counter)."""
    threads = usable_cpus()
    torch.set_num_threads(threads)
    shapes = shapes or [(B, h) for h in H_SWEEP]
    per, total_s, total_bytes = [], 0.0, 0
    for i, (rows, h) in enumerate(shapes):
        g = torch.Generator().manual_seed(i)
        x = torch.randn((rows, h), generator=g).to(torch.bfloat16)
        r = torch.randn((rows, h), generator=g).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn((h,), generator=g)).to(torch.bfloat16)

        def call():
            s_ = x + r
            return torch.rms_norm(s_, (h,), weight=w, eps=EPS)
        call()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            call()
            ts.append(time.perf_counter() - t0)
        med = statistics.median(ts)
        per.append({"rows": rows, "hidden": h, "ms_per_call": round(med * 1e3, 2),
                    "gbs": round(fused_bytes(rows, h) / med / 1e9, 2)})
        total_s += med
        total_bytes += fused_bytes(rows, h)
        del x, r, w
    return {"value": round(total_bytes / total_s / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "what": "the reference test's torch formula (test/test_hp_rms_norm.py:6-19), torch eager on the CPU",
            "sample": (f"the full benchmark workload: bf16 ({B}, H) for the {len(shapes)} H of the sweep, "
                       f"{total_bytes / 1e9:.2f} GB algorithmic; per shape 1 warm-up + median of {reps} calls"),
            "torch_threads": torch.get_num_threads(), "os_cpu_count": os.cpu_count(),
            "cpu_model": cpu_model(), "per_shape": per}


def cpu_oracle_baseline(torch, budget_s=10.0):
    """The CPU oracle (a scalar C restatement, OpenMP over rows) on the same
    cores, on a bounded sample: 256 rows of (4096, H) for every H of the sweep."""
    import numpy as np

    from oracle import oracle

    threads = usable_cpus()
    sample_rows = 256
    shapes = [(sample_rows, h) for h in H_SWEEP]
    g = torch.Generator().manual_seed(0)
    data = []
    for rows, h in shapes:
        x = torch.randn((rows, h), generator=g).to(torch.bfloat16)
        r = torch.randn((rows, h), generator=g).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn((h,), generator=g)).to(torch.bfloat16)
        data.append((x, r, w))
    sample_bytes = sum(fused_bytes(rows, h) for rows, h in shapes)

    def bitsnp(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    def one_pass():
        t = 0.0
        for x, r, w in data:
            xo, ro = bitsnp(x).copy(), bitsnp(r).copy()
            t0 = time.perf_counter()
            oracle.fused_add_rmsnorm_(xo, bitsnp(w), ro, EPS, oracle.BF16, threads=threads)
            t += time.perf_counter() - t0
        return t

    one_pass()
    reps, t_start = [], time.perf_counter()
    while len(reps) < 3 or (time.perf_counter() - t_start < budget_s and len(reps) < 200):
        reps.append(one_pass())
    med = statistics.median(reps)
    return {"value": round(sample_bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "what": "the CPU oracle (oracle/hprms_oracle.c, OpenMP over rows)",
            "sample": (f"{sample_rows} rows x each H of the sweep (bf16, {len(shapes)} shapes, "
                       f"{sample_bytes / 1e6:.0f} MB algorithmic per pass), median of {len(reps)} passes")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--full-json", default="", metavar="PATH",
                    help="also write the bench line and every detail section to PATH as one JSON document")
    ap.add_argument("--profile", type=int, default=0, metavar="H",
                    help="profiling driver: only run (4096, H) bf16 calls, then a 1 GiB device copy "
                         "(the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--sweep", type=int, default=0, metavar="STEP",
                    help="only time the fused op at (4096, H) for every H = STEP, 2*STEP, ... <= --sweep-max "
                         "(cold, like per_shape), one JSON line per H, with the kernel it runs")
    ap.add_argument("--sweep-max", type=int, default=32768)
    ap.add_argument("--profile-config", default="",
                    help="with --profile: force lanes_per_row,vec_per_lane,lds_vec_per_lane,block,flags")
    ap.add_argument("--ceiling", default="", metavar="H,H,...",
                    help="only the ceiling leg: the fused op beside the skeleton, copy, read, write and empty "
                         "kernels of the bench library at (4096, H), one JSON line")
    ap.add_argument("--flat", default="", metavar="H,H,...",
                    help="only the flat-stream leg: one and two in-place streams of each workgroup shape and load "
                         "order at the fused op's bytes, one JSON line per H")
    ap.add_argument("--placement", default="", metavar="H,H,...",
                    help="only the placement leg: the fused op and the flat two-stream rewrite with the residual "
                         "at each of --gaps relative to the input, one JSON line per H")
    ap.add_argument("--gaps", default="0,512,4096,8192,16384,65536,262144,1048576,r0",
                    help="with --placement: bytes from the end of x to the start of r (rG: r first)")
    ap.add_argument("--fillmap", action="store_true",
                    help="only the fill-and-drain map at (4096, 4096): empty grid, skeleton and fused op for every "
                         "split of the row into lanes x vectors and rows per workgroup, one JSON line")
    ap.add_argument("--timeline-dump", default="", metavar="DIR",
                    help="with --ceiling: also save each H's raw per-workgroup timeline as DIR/timeline_H.npy")
    ap.add_argument("--ab", nargs="+", default=None, metavar="H:CFG;CFG",
                    help="only an A/B of the fused op at (4096, H) bf16: the table's configuration against "
                         "forced bench-library ones (CFG = lanes_per_row,vec_per_lane,lds_vec_per_lane,block,flags)")
    ap.add_argument("--xcd-sweep", action="store_true",
                    help="only an A/B at every H of the sweep: the table's shape with its row groups in each "
                         "xcd_runs order (runs of 1, 2, ..., 128 per XCD; flags bits 16-18) against the table")
    ap.add_argument("--ab-runs", default="", metavar="H,H,...",
                    help="only an A/B of the fused op's other forms (plain, out of place, FP8 per row, MXFP8, "
                         "MXFP4, FP8 per 128 elements with rows or columns of scales) at (--ab-rows, H) bf16: the "
                         "table's shape in the default row-group order against runs of 32 and 64 row groups per "
                         "XCD, and the dispatch's own choice")
    ap.add_argument("--hot", action="store_true",
                    help="with --ab: one buffer set, the same every call (resident in the Infinity Cache)")
    ap.add_argument("--ab-rows", type=int, default=B, metavar="ROWS",
                    help="with --ab: rows per call (default 4096)")
    ap.add_argument("--layout", default="0,0", metavar="OFF,PAD",
                    help="with --ab, or --profile of the fused op: input and residual rows start OFF elements "
                         "into rows of H + OFF + PAD elements (rows off the 128-byte grid take the "
                         "configurations' off-grid variants)")
    ap.add_argument("--profile-op", default="fused",
                    choices=("fused", "fp8", "plain", "mxfp8", "mxfp4", "group_rows", "group_columns", "copy",
                             "relu"),
                    help="with --profile: the 16-bit fused op, its FP8 / MX-output forms (group_rows / "
                         "group_columns: FP8 with a scale per 128 elements, rows or column-major scales; "
                         "with --profile-config, forced through the bench library), plain RMSNorm, "
                         "or the streamer (the reference's relu = copy, and the true ReLU)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the op has no cross-GPU step (rows are independent), and this "
              f"build runs on single-GPU boxes; --gpus {args.gpus} is not supported.", file=sys.stderr)
        sys.exit(2)

    import torch

    import hp_rms_norm_amd
    from hp_rms_norm_amd import abi

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    abi.lib()
    op = hp_rms_norm_amd.hp_rms_norm
    if args.profile:
        return profile_driver(torch, abi, op, args)
    if args.sweep:
        return sweep(torch, abi, op, args)
    if args.xcd_sweep:
        # (widths whose table shape at this row count has no such variants in the bench library are left out)
        built = {c.as_tuple() for c in abi.BENCH.kernel_configs(abi.DTYPE_BF16, abi.MODE_FUSED)}
        specs = []
        for h in H_SWEEP:
            c = abi.select_config(args.ab_rows, h, abi.DTYPE_BF16)
            c.flags &= ~(7 << 16)
            if not all(c.as_tuple()[:6] + (c.flags | (v << 16),) in built for v in range(8)):
                log(f"--xcd-sweep: no run-order variants of {c.as_tuple()} for H = {h}")
                continue
            base = ",".join(str(v) for v in (c.lanes_per_row, c.vec_per_lane, c.lds_vec_per_lane, c.block_threads))
            specs.append(f"{h}:" + ";".join(f"{base},{c.flags | (v << 16)}" for v in range(8)))
        return ab_trials(torch, abi, op, specs, args.hot, rows=args.ab_rows)
    if args.ab_runs:
        return ab_runs_leg(torch, abi, hp_rms_norm_amd, [int(v) for v in args.ab_runs.split(",")], rows=args.ab_rows)
    if args.ab:
        off, pad = (int(v) for v in args.layout.split(","))
        return ab_trials(torch, abi, op, args.ab, args.hot, off, pad, rows=args.ab_rows)
    if args.flat:
        return flat_leg(torch, abi, hp_rms_norm_amd, [int(v) for v in args.flat.split(",")], max(args.steps, 10),
                        args.warmup)
    if args.placement:
        return placement_leg(torch, abi, hp_rms_norm_amd, [int(v) for v in args.placement.split(",")],
                             args.gaps.split(","), max(args.steps, 10), args.warmup)
    if args.fillmap:
        return fill_leg(torch, abi, hp_rms_norm_amd, max(args.steps, 10), args.warmup)
    if args.ceiling:
        hs = [int(v) for v in args.ceiling.split(",")]
        rows = ceiling(torch, abi, hp_rms_norm_amd, hs, max(args.steps, 10), args.warmup,
                       dump=args.timeline_dump or None)
        print(json.dumps({"ceiling_bf16": rows}), flush=True)
        return

    shapes = [(B, h, torch.bfloat16, "bench") for h in H_SWEEP]
    log(f"bench: timing {len(shapes)} shapes x {args.steps} steps (warmup {args.warmup})")
    step_ms = time_step(torch, op, shapes, args.steps, args.warmup)
    step_bytes = sum(fused_bytes(B, h) for h in H_SWEEP)
    value = step_bytes / (step_ms * 1e-3) / 1e9
    log("bench: per-shape timing")
    per_us = time_shapes(torch, op, shapes, args.steps, args.warmup)

    per_shape, by_kernel = [], {}
    for (rows, h, _, _), (us, p10, p90) in zip(shapes, per_us):
        key = kernel_key(abi, rows, h, 0)
        per_shape.append({"rows": rows, "hidden": h, "us_per_call": round(us, 2),
                          "us_p10": round(p10, 2), "us_p90": round(p90, 2),
                          "gbs": round(fused_bytes(rows, h) / (us * 1e-6) / 1e9, 1),
                          "kernel": {"lanes_per_row": key[1], "vec_per_lane": key[2],
                                     "lds_vec_per_lane": key[3], "block": key[4], "flags": key[6]}})
        k = by_kernel.setdefault(key, {"us": 0.0, "bytes": 0, "launches": 0, "hidden": []})
        k["us"] += us
        k["bytes"] += fused_bytes(rows, h)
        k["launches"] += 1
        k["hidden"].append(h)
    dom_key, dom = max(by_kernel.items(), key=lambda kv: kv[1]["us"])
    achieved = dom["bytes"] / (dom["us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBS, 4), "traffic": None,
                "kernel": (f"fused_vec_kernel<bf16, fused, lanes_per_row={dom_key[1]}, vec_per_lane={dom_key[2]}, "
                           f"lds_vec_per_lane={dom_key[3]}, block={dom_key[4]}, flags={dom_key[6]}>"),
                "kernel_hidden": dom["hidden"],
                "avg_launch_us": round(dom["us"] / dom["launches"], 2),
                "algorithmic_bytes_per_launch": dom["bytes"] // dom["launches"]}
    prof = load_traffic(dom_key)
    if prof is not None:
        # HBM bytes per launch: the counter-measured traffic/algorithmic ratio of
        # this kernel (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated on a copy of
        # known size) applied to this kernel's algorithmic bytes per launch here
        roofline["traffic"] = round(prof["ratio"] * roofline["algorithmic_bytes_per_launch"])
        roofline["traffic_source"] = {k: prof[k] for k in ("profiled_shape", "hbm_bytes_per_launch_profiled",
                                                           "algorithmic_bytes_per_launch_profiled", "ratio",
                                                           "source")}

    extra = {}
    if not args.no_extra:
        extra = run_extra(torch, hp_rms_norm_amd, args)
        fused_us = {p["hidden"]: p["us_per_call"] for p in per_shape}
        for c in extra.get("copy_same_bytes_bf16", []):
            if c["hidden"] in fused_us:
                c["fused_us_per_call"] = fused_us[c["hidden"]]
                c["fused_over_copy"] = round(fused_us[c["hidden"]] / c["us_per_call"], 3)

    cpu = None
    cpu_oracle = None
    if not args.no_cpu:
        log("bench: CPU baseline (torch eager formula)")
        cpu = cpu_torch_baseline(torch)
        log("bench: CPU oracle")
        cpu_oracle = cpu_oracle_baseline(torch)

    details = detail_lines(extra, cpu)
    line = headline(value=value, steps=args.steps, warmup=args.warmup, step_ms=step_ms, step_bytes=step_bytes,
                    per_shape=per_shape, roofline=roofline, cpu=cpu, cpu_oracle=cpu_oracle,
                    details=[d["bench_detail"] for d in details])
    if args.full_json:
        with open(args.full_json, "w") as f:
            json.dump({"headline": line, "details": details}, f)
    for d in details:
        print(json.dumps(d), flush=True)
    print(json.dumps(line), flush=True)


# The bench line (the last line on stdout) stays well below what a driver
# keeps of a run's output; everything else goes on the lines before it.
HEADLINE_MAX_BYTES = 8192


def kernel_name(k):
    """A per_shape kernel dict as 'lanes x vectors (in LDS) /block flags F'."""
    lds = f" ({k['lds_vec_per_lane']})" if k.get("lds_vec_per_lane") else ""
    return f"{k['lanes_per_row']}x{k['vec_per_lane']}{lds}/{k['block']} f{k['flags']}"


def headline(*, value, steps, warmup, step_ms, step_bytes, per_shape, roofline, cpu, cpu_oracle, details=()):
    """The bench line: the metric, the per-shape figures (hidden, µs with
    p10/p90, GB/s, kernel), the dominant kernel's roofline and the CPU
    baselines without their per-shape lists.  Raises if it would exceed
    HEADLINE_MAX_BYTES."""
    cpu_keys = ("value", "unit", "cores", "kind", "what", "sample", "torch_threads", "os_cpu_count", "cpu_model")
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(step_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "fused add+RMSNorm bf16 (4096, H), H in configs[1] (1024..12288 step 1024) "
                               "and configs[2] (13312..32768); one step = one call per H",
                   "rows": B, "hidden": H_SWEEP, "eps": EPS,
                   "inputs": "input, residual ~ N(0,1), weight ~ N(1,0.1), generated on device",
                   "buffer_sets_per_shape": 2, "bytes_per_step": step_bytes,
                   "per_shape_timing": "back-to-back calls over buffer sets spanning >= 1 GiB"},
        "per_shape": [{"hidden": p["hidden"], "us": p["us_per_call"], "us_p10_p90": [p["us_p10"], p["us_p90"]],
                       "gbs": p["gbs"], "kernel": kernel_name(p["kernel"])} for p in per_shape],
        "roofline": roofline,
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in cpu_keys if k in cpu},
        "cpu_oracle": cpu_oracle,
        "details_on_earlier_lines": list(details),
    }
    n = len(json.dumps(line).encode())
    if n > HEADLINE_MAX_BYTES:
        raise RuntimeError(f"bench line of {n} bytes exceeds {HEADLINE_MAX_BYTES}")
    return line


def detail_lines(extra, cpu):
    """The measurements that do not go into the bench line, one JSON object
    per section ({"bench_detail": name, "data": ...}), printed before it."""
    out = [{"bench_detail": k, "data": v} for k, v in extra.items()]
    if cpu is not None and "per_shape" in cpu:
        out.append({"bench_detail": "cpu_baseline_per_shape", "data": cpu["per_shape"]})
    return out


def time_rotating(torch, call, n, steps, warmup):
    """µs per call of call(i % n) over max(steps, n) back-to-back calls."""
    for i in range(warmup):
        call(i % n)
    ncalls = max(steps, n)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    prefill(torch, 10)
    e0.record()
    for i in range(ncalls):
        call(i % n)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / ncalls


def ab_trials(torch, abi, op, specs, hot, off=0, pad=0, trials=7, rows=B):
    """A/B of the fused op at (rows, H) bf16 (rows = 4096 by default): the table's configuration and
    forced configurations of the bench library, timed in one process in
    `trials` interleaved rounds (the order reversed every other round); each
    timing is back-to-back calls between one HIP event pair, over buffer sets
    spanning >= 1 GiB (cold) or over one set (hot: resident in the 256 MB
    Infinity Cache after the first call).  Rows start `off` elements into rows
    of H + off + pad elements.  One JSON line per configuration: the median µs
    per call and its ratio to the table's."""
    built = {c.as_tuple() for c in abi.BENCH.kernel_configs(abi.DTYPE_BF16, abi.MODE_FUSED)}
    plan = []
    for spec in specs:
        h, _, cfgs = spec.partition(":")
        h = int(h)
        forced = []
        for c in filter(None, cfgs.split(";")):
            lpr, vpl, ldsv, block, flags = (int(v) for v in c.split(","))
            cfg = abi.Config(2 if ldsv else 1, lpr, vpl, ldsv, block, 0, flags)
            if cfg.as_tuple() not in built or lpr * vpl < h // 8:
                raise SystemExit(f"--ab: {c} is not a bench-library configuration that covers H = {h}")
            forced.append((c, cfg))
        plan.append((h, forced))
    stream = torch.cuda.current_stream().cuda_stream
    for h, forced in plan:
        stride = h + off + pad
        n = 1 if hot else cold_sets(rows, stride)
        bufs = [torch.empty((2, rows, stride), dtype=torch.bfloat16, device="cuda:0").normal_() for _ in range(n)]
        sets = [b[:, :, off:off + h] for b in bufs]
        w = (1 + 0.1 * torch.randn(h, device="cuda:0")).to(torch.bfloat16)
        base = abi.select_config(rows, h, abi.DTYPE_BF16)

        def table_call(i):
            op(sets[i][0], w, sets[i][1], EPS)

        def forced_call(cfg):
            return lambda i: abi.BENCH.fused_add_rmsnorm(sets[i][0].data_ptr(), w.data_ptr(), sets[i][1].data_ptr(),
                                                         rows, h, stride, stride, abi.DTYPE_BF16, EPS, stream, cfg)
        runs = [("table", table_call)] + [(c, forced_call(cfg)) for c, cfg in forced]
        res = {k: [] for k, _ in runs}
        for t in range(trials):
            for k, call in (runs if t % 2 == 0 else runs[::-1]):
                res[k].append(time_rotating(torch, call, n, max(40, 2 * n), 3))
        tab = statistics.median(res["table"])
        for k, v in res.items():
            m = statistics.median(v)
            cfg = "table " + ",".join(str(x) for x in (base.lanes_per_row, base.vec_per_lane, base.lds_vec_per_lane,
                                                        base.block_threads, base.flags)) if k == "table" else k
            print(json.dumps({"hidden": h, "rows": rows, "row_offset": off, "row_stride": stride, "hot": hot,
                              "cfg": cfg, "us": round(m, 2),
                              "gbs": round(fused_bytes(rows, h) / m / 1e3, 1), "vs_table": round(m / tab - 1, 4),
                              "spread": round((max(v) - min(v)) / m, 4)}), flush=True)
        del sets, bufs
        torch.cuda.empty_cache()


def ab_runs_leg(torch, abi, ops, hiddens, rows=B, trials=7):
    """The fused op's other forms at (rows, H) bf16, cold: the table's shape
    with its row groups in the default order, in runs of 32 and of 64 per XCD
    (flags bits 16-18 = 5, 6; where the bench library builds them), and the
    dispatch's own choice (through the torch ops), timed in `trials`
    interleaved rounds (order reversed every other round).  One JSON line per
    form and H: the median µs of each and each run length's ratio to the
    default order."""
    stream = torch.cuda.current_stream().cuda_stream
    forms = (("plain", 1), ("out_of_place", 3), ("fp8", 2), ("mxfp8", 5), ("mxfp4", 6), ("group128_rows", 7),
             ("group128_columns", 7))
    for h in hiddens:
        n = cold_sets(rows, h)
        sets = [make_set(torch, rows, h, torch.bfloat16, 7700 + i, "cuda:0") for i in range(n)]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")
        q8 = [torch.empty(rows, h, dtype=torch.uint8, device="cuda:0") for _ in range(n)]
        q4 = [torch.empty(rows, h // 2, dtype=torch.uint8, device="cuda:0") for _ in range(n)]
        o16 = [torch.empty(rows, h, dtype=torch.bfloat16, device="cuda:0") for _ in range(n)]
        ro16 = [torch.empty(rows, h, dtype=torch.bfloat16, device="cuda:0") for _ in range(n)]
        s_row = torch.empty(rows, dtype=torch.float32, device="cuda:0")
        s_mx = torch.empty(rows, h // 32, dtype=torch.uint8, device="cuda:0")
        s_g = torch.empty(rows, h // 128, dtype=torch.float32, device="cuda:0")
        s_gc = torch.empty(h // 128, rows, dtype=torch.float32, device="cuda:0")
        for name, mode in forms:
            out = q4 if mode == 6 else o16 if mode in (1, 3) else q8
            aux = [ro16[i] for i in range(n)] if mode == 3 else [None] * n
            sc, ss, gs = {2: (s_row, 0, 0), 5: (s_mx, h // 32, 1), 6: (s_mx, h // 32, 1)}.get(
                mode, (s_gc, 1, rows) if name.endswith("columns") else (s_g, h // 128, 1))

            def table(i, out=out, aux=aux, sc=sc, mode=mode, name=name):
                x, r = sets[i]
                if mode == 1:
                    ops.rms_norm(out[i], x, w, EPS)
                elif mode == 3:
                    ops.fused_add_rms_norm_out(out[i], aux[i], x, w, r, EPS)
                elif mode == 2:
                    ops.hp_rms_norm_fp8(out[i].view(torch.float8_e4m3fn), sc, x, w, r, EPS)
                elif mode in (5, 6):
                    ops.hp_rms_norm_mx(out[i], sc, x, w, r, EPS, ops.MXFP8 if mode == 5 else ops.MXFP4)
                else:
                    ops.hp_rms_norm_fp8_group(out[i].view(torch.float8_e4m3fn), sc.t() if name.endswith("columns")
                                              else sc, x, w, r, EPS)

            def forced(cfg, out=out, aux=aux, sc=sc, ss=ss, gs=gs, mode=mode):
                def call(i):
                    a = aux[i].data_ptr() if mode == 3 else 0 if mode == 1 else sc.data_ptr()
                    abi.BENCH.bench_form_config(mode, out[i].data_ptr(), a, ss, gs, sets[i][0].data_ptr(),
                                                w.data_ptr(), sets[i][1].data_ptr(), rows, h, abi.DTYPE_BF16, EPS,
                                                cfg, stream)
                return call
            base = abi.select_config(rows, h, abi.DTYPE_BF16, mode)
            built = {c.as_tuple() for c in abi.BENCH.kernel_configs(abi.DTYPE_BF16, mode)}
            default = abi.Config(*base.as_tuple())
            default.flags &= ~(7 << 16)
            calls = [("default", forced(default))]
            for v in (5, 6):
                c = abi.Config(*default.as_tuple())
                c.flags |= v << 16
                if c.as_tuple() in built:
                    calls.append((f"runs{1 << v}", forced(c)))
            if len(calls) == 1:
                print(json.dumps({"ab_runs": name, "hidden": h, "rows": rows, "shape": default.as_tuple(),
                                  "skipped": "no runs variant built for this shape"}), flush=True)
                continue
            calls.append(("table", table))
            res = {k: [] for k, _ in calls}
            for t in range(trials):
                for k, call in (calls if t % 2 == 0 else calls[::-1]):
                    res[k].append(time_rotating(torch, call, n, max(40, 2 * n), 3))
            med = {k: round(statistics.median(v), 2) for k, v in res.items()}
            print(json.dumps({"ab_runs": name, "hidden": h, "rows": rows, "shape": default.as_tuple()[1:5],
                              "flags": default.flags, "us": med,
                              "over_default": {k: round(med[k] / med["default"], 4) for k in med if k != "default"},
                              "spread": {k: round((max(v) - min(v)) / statistics.median(v), 4)
                                         for k, v in res.items()}}), flush=True)
        del sets, q8, q4, o16, ro16
        torch.cuda.empty_cache()


def profile_driver(torch, abi, op, args):
    """A short, fixed workload for rocprofv3 counter runs: `steps` cold calls
    of (4096, H) bf16, then `steps` copies of a 1 GiB bf16 tensor."""
    hidden = args.profile
    if args.profile_config:
        lpr, vpl, ldsv, block, flags = (int(v) for v in args.profile_config.split(","))
        cfg = abi.Config(2 if ldsv else 1, lpr, vpl, ldsv, block, 0, flags)
        stream = torch.cuda.current_stream().cuda_stream

        def op(x, w, r, eps):  # noqa: F811  (the forced configuration, through the C ABI)
            abi.fused_add_rmsnorm(x.data_ptr(), w.data_ptr(), r.data_ptr(), x.shape[0], x.shape[1],
                                  x.stride(0), r.stride(0), abi.DTYPE_BF16, eps, stream, cfg)
    if args.profile_op == "fp8":
        import hp_rms_norm_amd
        q = torch.empty(B, hidden, dtype=torch.float8_e4m3fn, device="cuda:0")
        sc = torch.empty(B, 1, dtype=torch.float32, device="cuda:0")

        def op(x, w, r, eps):  # noqa: F811  (FP8 output; the input row is only read)
            hp_rms_norm_amd.hp_rms_norm_fp8(q, sc, x, w, r, eps)
    if args.profile_op == "plain":
        import hp_rms_norm_amd
        o = torch.empty(B, hidden, dtype=torch.bfloat16, device="cuda:0")

        def op(x, w, r, eps):  # noqa: F811  (plain RMSNorm of the input row; r unused)
            hp_rms_norm_amd.rms_norm(o, x, w, eps)
    if args.profile_op in ("mxfp8", "mxfp4"):
        import hp_rms_norm_amd
        fmt = hp_rms_norm_amd.MXFP8 if args.profile_op == "mxfp8" else hp_rms_norm_amd.MXFP4
        q = torch.empty(B, hidden if fmt == hp_rms_norm_amd.MXFP8 else hidden // 2, dtype=torch.uint8,
                        device="cuda:0")
        sc = torch.empty(B, hidden // 32, dtype=torch.uint8, device="cuda:0")

        def op(x, w, r, eps):  # noqa: F811  (MX output; the input row is only read)
            hp_rms_norm_amd.hp_rms_norm_mx(q, sc, x, w, r, eps, fmt)
    if args.profile_op in ("group_rows", "group_columns"):
        # FP8 with a scale per 128 elements, rows of scales or column-major ones; with
        # --profile-config, that configuration forced through the bench library
        import hp_rms_norm_amd
        q = torch.empty(B, hidden, dtype=torch.float8_e4m3fn, device="cuda:0")
        cols = args.profile_op == "group_columns"
        sc = torch.empty(hidden // 128, B, dtype=torch.float32, device="cuda:0").t() if cols else \
            torch.empty(B, hidden // 128, dtype=torch.float32, device="cuda:0")
        gcfg = cfg if args.profile_config else None
        gstream = torch.cuda.current_stream().cuda_stream

        def op(x, w, r, eps):  # noqa: F811  (the input row is only read)
            if gcfg is None:
                hp_rms_norm_amd.hp_rms_norm_fp8_group(q, sc, x, w, r, eps)
            else:
                abi.BENCH.bench_form_config(7, q.data_ptr(), sc.data_ptr(), sc.stride(0), sc.stride(1),
                                            x.data_ptr(), w.data_ptr(), r.data_ptr(), x.shape[0], x.shape[1],
                                            abi.DTYPE_BF16, eps, gcfg, gstream)
    if args.profile_op in ("copy", "relu"):
        import hp_rms_norm_amd
        stream_fn = hp_rms_norm_amd.relu if args.profile_op == "copy" else hp_rms_norm_amd.relu_max0

        def op(x, w, r, eps):  # noqa: F811  (streamer: reads x, writes r; w and eps unused)
            stream_fn(r, x)
    off, pad = (int(v) for v in args.layout.split(","))
    if (off, pad) == (0, 0):
        us = time_shapes(torch, op, [(B, hidden, torch.bfloat16, "bench")], args.steps, args.warmup, trials=1)[0][0]
    else:
        # rows at element offset `off` of rows of hidden + off + pad elements
        stride = hidden + off + pad
        bases = [make_set(torch, B, stride, torch.bfloat16, 9500 + i, "cuda:0") for i in range(cold_sets(B, stride))]
        sets = [(x[:, off:off + hidden], r[:, off:off + hidden]) for x, r in bases]
        w = make_weight(torch, hidden, torch.bfloat16, 1, "cuda:0")
        us = time_rotating(torch, lambda i: op(sets[i][0], w, sets[i][1], EPS), len(sets), args.steps,
                           args.warmup)
        del bases, sets
    n = 1 << 29
    src = torch.empty(n, dtype=torch.bfloat16, device="cuda:0").normal_()
    dst = torch.empty_like(src)
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile: (4096, {hidden}) layout {off},{pad}: {us:.2f} us/call; then {args.steps} copies of "
        f"{2 * n} bytes")


def sweep(torch, abi, op, args):
    """Every H = STEP, 2*STEP, ... at 4096 rows: µs/call (median of 3 timed
    blocks over rotating buffer sets spanning >= 1 GiB) and GB/s, with the
    kernel the table chooses, one JSON line per H.  The buffers are views of
    one pool, so the sweep allocates once."""
    per_max = B * args.sweep_max
    pool = torch.empty(max(2 * per_max, (1 << 30) // 2 * 2), dtype=torch.bfloat16, device="cuda:0").normal_()
    w_all = make_weight(torch, args.sweep_max, torch.bfloat16, 0, "cuda:0")
    for h in range(args.sweep, args.sweep_max + 1, args.sweep):
        per = B * h
        n = max(2, min(cold_sets(B, h), pool.numel() // (2 * per)))
        sets = [(pool[2 * i * per:(2 * i + 1) * per].view(B, h), pool[(2 * i + 1) * per:(2 * i + 2) * per].view(B, h))
                for i in range(n)]
        w = w_all[:h]
        us = statistics.median(time_rotating(torch, lambda i: op(sets[i][0], w, sets[i][1], EPS), n, args.steps,
                                             args.warmup) for _ in range(3))
        key = kernel_key(abi, B, h, 0)
        print(json.dumps({"rows": B, "hidden": h, "us_per_call": round(us, 2),
                          "gbs": round(fused_bytes(B, h) / (us * 1e-6) / 1e9, 1),
                          "kernel": {"lanes_per_row": key[1], "vec_per_lane": key[2], "lds_vec_per_lane": key[3],
                                     "block": key[4], "flags": key[6]}}), flush=True)


SKEL_FLAG_MASK = 1 | 2 | 8 | 16 | 128   # the cache-policy and load-order bits the skeleton kernels take


def timeline_summary(tl, events_us):
    """Per-workgroup {start, end} realtime ticks (10 ns) of one launch ->
    when the workgroups started and ended relative to the first start."""
    import numpy as np
    t = np.asarray(tl, dtype=np.int64)
    t0 = t[:, 0].min()
    start = (t[:, 0] - t0) * 0.01
    end = (t[:, 1] - t0) * 0.01
    dur = end - start
    q = lambda a, p: round(float(np.percentile(a, p)), 2)  # noqa: E731
    xcc = t[:, 3] & 0xF
    per_xcd_end = [round(float(end[xcc == i].max()), 2) for i in range(8) if (xcc == i).any()]
    return {"workgroups": int(t.shape[0]), "events_us": round(events_us, 2),
            "span_us": round(float(end.max()), 2),
            "outside_span_us": round(events_us - float(end.max()), 2),
            "start_us_p50_p90_max": [q(start, 50), q(start, 90), q(start, 100)],
            "end_us_min_p10_p50_p90": [q(end, 0), q(end, 10), q(end, 50), q(end, 90)],
            "wg_us_p10_p50_p90": [q(dur, 10), q(dur, 50), q(dur, 90)],
            "last_end_per_xcd_us": per_xcd_end,
            "wgs_per_xcd": [int((xcc == i).sum()) for i in range(8)]}


def ceiling(torch, abi, ops, hs, steps, warmup, trials=5, dump=None):
    """The fused op beside kernels that move its bytes without its arithmetic
    (hprms_ceiling.hip, bench library), at (4096, H) bf16, cold (rotating
    buffer sets spanning >= 1 GiB), interleaved over `trials` rounds, median
    µs per call:
      fused     the product op (the table's kernel)
      skeleton  the op's data movement with the table row's shape and cache
                policy, no fp32 arithmetic, no weight
      copy      one read and one write stream of the op's 4*B*H*2 bytes
      read      the op's two read streams only (2*B*H*2 bytes)
      write     the op's two write streams only (2*B*H*2 bytes)
      empty     the table row's grid of empty workgroups
      inplace_1stream / inplace_2stream / copy_2stream
                the op's bytes as flat 4 KiB-per-workgroup streams: one tensor
                rewritten in place, x and r rewritten in place, x and r
                copied to two other tensors
      inplace_2stream_off16 / _off64
                x and r rewritten in place from 16 / 64 bytes past their
                starts, so every wave's 1 KiB access shares its first and
                last 128-byte line with its neighbours
    and one timeline launch of the table's kernel (per-workgroup start/end)."""
    import numpy as np
    bench = abi.BENCH
    BL = bench.lib()
    stream = torch.cuda.current_stream().cuda_stream
    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    out = []
    for h in hs:
        n = cold_sets(B, h)
        bufs = [torch.empty((2, B, h), dtype=torch.bfloat16, device="cuda:0").normal_() for _ in range(n)]
        w = make_weight(torch, h, torch.bfloat16, 0, "cuda:0")
        cfg = abi.select_config(B, h, abi.DTYPE_BF16, cus=abi.device_cu_count())
        rpb = cfg.block_threads // cfg.lanes_per_row
        grid = (B + rpb - 1) // rpb
        nb = B * h * 2   # bytes of one [B, H] tensor
        sflags = cfg.flags & SKEL_FLAG_MASK

        def chk(rc, what):
            if rc != 0:
                raise RuntimeError(f"{what}: status {rc}")
        kinds = {
            "fused": lambda i: ops.hp_rms_norm(bufs[i][0], w, bufs[i][1], EPS),
            "skeleton": lambda i: chk(BL.hprms_ceil_skeleton(bufs[i][0].data_ptr(), bufs[i][1].data_ptr(), B, h,
                                                             cfg.lanes_per_row, cfg.vec_per_lane,
                                                             cfg.block_threads, sflags, stream), "skeleton"),
            "copy": lambda i: chk(BL.hprms_ceil_copy(bufs[(i + 1) % n].data_ptr(), bufs[i].data_ptr(), 2 * nb,
                                                     stream), "copy"),
            "read": lambda i: chk(BL.hprms_ceil_read(bufs[i][0].data_ptr(), bufs[i][1].data_ptr(), nb,
                                                     sink.data_ptr(), stream), "read"),
            "write": lambda i: chk(BL.hprms_ceil_write(bufs[i][0].data_ptr(), bufs[i][1].data_ptr(), nb, stream),
                                   "write"),
            "empty": lambda i: chk(BL.hprms_ceil_empty(grid, cfg.block_threads, stream), "empty"),
            "inplace_1stream": lambda i: chk(BL.hprms_ceil_streams(0, bufs[i].data_ptr(), None, None, None, nb,
                                                                   stream), "inplace_1stream"),
            "inplace_2stream": lambda i: chk(BL.hprms_ceil_streams(1, bufs[i][0].data_ptr(), bufs[i][1].data_ptr(),
                                                                   None, None, nb, stream), "inplace_2stream"),
            "copy_2stream": lambda i: chk(BL.hprms_ceil_streams(2, bufs[i][0].data_ptr(), bufs[i][1].data_ptr(),
                                                                bufs[(i + 1) % n][0].data_ptr(),
                                                                bufs[(i + 1) % n][1].data_ptr(), nb, stream),
                                          "copy_2stream"),
        }
        for off in (16, 64):
            kinds[f"inplace_2stream_off{off}"] = (
                lambda i, off=off: chk(BL.hprms_ceil_streams(1, bufs[i][0].data_ptr() + off,
                                                             bufs[i][1].data_ptr() + off, None, None, nb - 128,
                                                             stream), f"inplace_2stream_off{off}"))
        samples = {k: [] for k in kinds}
        for t in range(trials):
            for k, fn in (kinds.items() if t % 2 == 0 else reversed(list(kinds.items()))):
                samples[k].append(time_rotating(torch, fn, n, steps, warmup))
        us = {k: statistics.median(v) for k, v in samples.items()}
        nbytes = {"fused": fused_bytes(B, h), "skeleton": 4 * nb, "copy": 4 * nb, "read": 2 * nb, "write": 2 * nb,
                  "inplace_1stream": 4 * nb, "inplace_2stream": 4 * nb, "copy_2stream": 4 * nb,
                  "inplace_2stream_off16": 4 * (nb - 128), "inplace_2stream_off64": 4 * (nb - 128)}
        row = {"hidden": h, "rows": B,
               "kernel": {"lanes_per_row": cfg.lanes_per_row, "vec_per_lane": cfg.vec_per_lane,
                          "lds_vec_per_lane": cfg.lds_vec_per_lane, "block": cfg.block_threads,
                          "flags": cfg.flags, "grid": grid, "skeleton_flags": sflags},
               "us_per_call": {k: round(v, 2) for k, v in us.items()},
               "gbs": {k: round(nbytes[k] / (us[k] * 1e-6) / 1e9, 1) for k in nbytes},
               "fused_over_skeleton": round(us["fused"] / us["skeleton"], 3),
               "fused_over_copy": round(us["fused"] / us["copy"], 3)}
        # one timeline launch of the table's kernel on a cold buffer set (in the default row-group
        # order: the instrumented kernels have no runs-per-XCD variants)
        tcfg = abi.Config(*cfg.as_tuple())
        tcfg.flags = (cfg.flags & ~(7 << 16)) | 512
        tl = torch.zeros((grid, 4), dtype=torch.int64, device="cuda:0")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

        def timeline_launch(k):
            return BL.hprms_bench_fused_timeline(bufs[k][0].data_ptr(), w.data_ptr(), bufs[k][1].data_ptr(), B, h,
                                                 abi.DTYPE_BF16, EPS, ctypes.byref(tcfg), tl.data_ptr(), stream)
        # the instrumented kernel's first launch loads its code: once untimed, on another set
        rc = timeline_launch(n - 1)
        for k in range(1, n):  # leave set 0 the least recently used
            kinds["fused"](k)
        torch.cuda.synchronize()
        prefill(torch, 5)
        if rc == 0:
            e0.record()
            rc = timeline_launch(0)
            e1.record()
        torch.cuda.synchronize()
        if rc == 0:
            tlh = tl.cpu().numpy()
            row["timeline"] = timeline_summary(tlh, e0.elapsed_time(e1) * 1e3)
            if dump:
                np.save(os.path.join(dump, f"timeline_{h}.npy"), tlh)
        else:
            row["timeline"] = {"skipped": bench.last_error()}
        log("ceiling", json.dumps(row))
        out.append(row)
        del bufs, tl
        torch.cuda.empty_cache()
    return out


def interleaved(torch, kinds, n, steps, warmup, trials):
    """Median µs per call of each kind (a function of the buffer-set index),
    timed in `trials` interleaved rounds, the order reversed every other one."""
    samples = {k: [] for k in kinds}
    items = list(kinds.items())
    for t in range(trials):
        for k, fn in (items if t % 2 == 0 else items[::-1]):
            samples[k].append(time_rotating(torch, fn, n, steps, warmup))
    return {k: statistics.median(v) for k, v in samples.items()}


def chk(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: status {rc}")


FLAT_SHAPES = [(64, 1), (128, 1), (256, 1), (512, 1), (1024, 1), (256, 2), (512, 2), (1024, 2), (256, 4), (1024, 4)]
# the shapes also built with the workgroups in xcd_order's maps 1 and 2 (hprms_ceil_flat orders 4 and 5)
FLAT_MAPPED = [(256, 1), (512, 1), (1024, 1), (256, 2), (1024, 4)]


def flat_leg(torch, abi, ops, hs, steps, warmup, trials=5):
    """The fused op's bytes at (4096, H) as flat in-place streams of each
    workgroup shape (hprms_ceil_flat): one stream `a` of 2*B*H*2 bytes, and
    two streams `x`, `r` of B*H*2 bytes each (adjacent in one allocation) in
    four load orders (o0-o3), and for FLAT_MAPPED shapes with the workgroups
    in xcd_order's maps 1 and 2 (o4, o5); beside them the fused op and a
    copy.  Cold (rotating buffer sets spanning >= 1 GiB).  One JSON line per
    H."""
    BL = abi.BENCH.lib()
    stream = torch.cuda.current_stream().cuda_stream
    for h in hs:
        nb = B * h * 2
        n = cold_sets(B, h)
        bufs = [torch.empty((2, B, h), dtype=torch.bfloat16, device="cuda:0").normal_() for _ in range(n)]
        w = make_weight(torch, h, torch.bfloat16, 0, "cuda:0")
        kinds = {"fused": lambda i: ops.hp_rms_norm(bufs[i][0], w, bufs[i][1], EPS),
                 "copy": lambda i: chk(BL.hprms_ceil_copy(bufs[(i + 1) % n].data_ptr(), bufs[i].data_ptr(), 2 * nb,
                                                          stream), "copy")}
        for blk, vpl in FLAT_SHAPES:
            kinds[f"one_{blk}x{vpl}"] = (lambda i, blk=blk, vpl=vpl: chk(
                BL.hprms_ceil_flat(0, blk, vpl, 0, bufs[i].data_ptr(), None, nb, stream), "flat"))
            for order in range(4) if (blk, vpl) not in FLAT_MAPPED else range(6):
                kinds[f"two_{blk}x{vpl}_o{order}"] = (lambda i, blk=blk, vpl=vpl, order=order: chk(
                    BL.hprms_ceil_flat(1, blk, vpl, order, bufs[i][0].data_ptr(), bufs[i][1].data_ptr(), nb,
                                       stream), "flat"))
            if (blk, vpl) in FLAT_MAPPED:
                for order in (4, 5):
                    kinds[f"one_{blk}x{vpl}_o{order}"] = (lambda i, blk=blk, vpl=vpl, order=order: chk(
                        BL.hprms_ceil_flat(0, blk, vpl, order, bufs[i].data_ptr(), None, nb, stream), "flat"))
        us = interleaved(torch, kinds, n, steps, warmup, trials)
        nbytes = {k: (fused_bytes(B, h) if k == "fused" else 4 * nb) for k in kinds}
        print(json.dumps({"flat_hidden": h, "rows": B, "us": {k: round(v, 2) for k, v in us.items()},
                          "gbs": {k: round(nbytes[k] / (us[k] * 1e-6) / 1e9, 1) for k in us}}), flush=True)
        del bufs
        torch.cuda.empty_cache()


def placement_leg(torch, abi, ops, hs, gaps, steps, warmup, trials=5):
    """The fused op and the flat two-stream rewrite (256 lanes x 1 vector,
    alternating loads) with the residual placed relative to the input inside
    one allocation: gap "G" puts r G bytes after the end of x, "rG" puts r
    first and x G bytes after it.  Cold, interleaved over the gaps.  One JSON
    line per H."""
    BL = abi.BENCH.lib()
    stream = torch.cuda.current_stream().cuda_stream
    for h in hs:
        nb = B * h * 2
        n = cold_sets(B, h)
        w = make_weight(torch, h, torch.bfloat16, 0, "cuda:0")
        kinds, keep = {}, []
        for gap in gaps:
            rfirst = gap.startswith("r")
            g = int(gap[1:] if rfirst else gap)
            if g % 512:
                raise SystemExit(f"--gaps: {gap} is not a multiple of 512 bytes")
            sets = []
            for _ in range(n):
                raw = torch.empty(2 * nb + g, dtype=torch.uint8, device="cuda:0")
                lo = raw[:nb].view(torch.bfloat16).view(B, h)
                hi = raw[nb + g:].view(torch.bfloat16).view(B, h)
                x, r = (hi, lo) if rfirst else (lo, hi)
                x.normal_()
                r.normal_()
                sets.append((x, r))
            keep.append(sets)
            kinds[f"fused_{gap}"] = lambda i, s=sets: ops.hp_rms_norm(s[i][0], w, s[i][1], EPS)
            kinds[f"flat2_{gap}"] = lambda i, s=sets: chk(
                BL.hprms_ceil_flat(1, 256, 1, 0, s[i][0].data_ptr(), s[i][1].data_ptr(), nb, stream), "flat")
        us = interleaved(torch, kinds, n, steps, warmup, trials)
        print(json.dumps({"placement_hidden": h, "rows": B, "gaps": gaps,
                          "us": {k: round(v, 2) for k, v in us.items()}}), flush=True)
        del keep, kinds
        torch.cuda.empty_cache()


FILL_SHAPES = [(64, 8, 64), (64, 8, 128), (64, 8, 256), (64, 8, 512), (128, 4, 128), (128, 4, 256), (128, 4, 512),
               (256, 2, 256), (256, 2, 512), (512, 1, 512)]


def fill_leg(torch, abi, ops, steps, warmup, trials=7, h=4096):
    """Fill-and-drain map at (4096, 4096) bf16: for every split of a row into
    lanes x vectors in workgroups of one to eight rows (grids of 512 to 4096
    workgroups of 64 to 512 lanes), the empty grid, the skeleton (the op's
    data movement, no arithmetic) and the fused op forced to that shape (nt,
    residual loads first, weight with the row: flags 131); beside them the
    table's op and a copy of the same bytes.  Cold, interleaved.  One JSON
    line."""
    BB = abi.BENCH
    BL = BB.lib()
    stream = torch.cuda.current_stream().cuda_stream
    nb = B * h * 2
    n = cold_sets(B, h)
    bufs = [torch.empty((2, B, h), dtype=torch.bfloat16, device="cuda:0").normal_() for _ in range(n)]
    w = make_weight(torch, h, torch.bfloat16, 0, "cuda:0")
    kinds = {"table": lambda i: ops.hp_rms_norm(bufs[i][0], w, bufs[i][1], EPS),
             "copy": lambda i: chk(BL.hprms_ceil_copy(bufs[(i + 1) % n].data_ptr(), bufs[i].data_ptr(), 2 * nb,
                                                      stream), "copy")}
    for lpr, vpl, blk in FILL_SHAPES:
        grid = B // (blk // lpr)
        tag = f"{lpr}x{vpl}/{blk}"
        cfg = abi.Config(1, lpr, vpl, 0, blk, 0, 131)
        kinds[f"empty {tag}"] = lambda i, g=grid, b=blk: chk(BL.hprms_ceil_empty(g, b, stream), "empty")
        kinds[f"skeleton {tag}"] = lambda i, lpr=lpr, vpl=vpl, blk=blk: chk(
            BL.hprms_ceil_skeleton(bufs[i][0].data_ptr(), bufs[i][1].data_ptr(), B, h, lpr, vpl, blk, 131, stream),
            "skeleton")
        kinds[f"fused {tag}"] = lambda i, cfg=cfg: BB.fused_add_rmsnorm(
            bufs[i][0].data_ptr(), w.data_ptr(), bufs[i][1].data_ptr(), B, h, h, h, abi.DTYPE_BF16, EPS, stream, cfg)
    # every row resident in one round: 128 x 4 held to 8 waves per SIMD (flags +256; the compiler then
    # keeps 64 VGPRs and spills), so the 2048 two-row workgroups fit the chip's wave slots at once
    every = abi.Config(1, 128, 4, 0, 256, 0, 391)
    kinds["fused 128x4/256 at 8 waves per SIMD"] = lambda i: BB.fused_add_rmsnorm(
        bufs[i][0].data_ptr(), w.data_ptr(), bufs[i][1].data_ptr(), B, h, h, h, abi.DTYPE_BF16, EPS, stream, every)
    us = interleaved(torch, kinds, n, steps, warmup, trials)
    grids = {f"{lpr}x{vpl}/{blk}": B // (blk // lpr) for lpr, vpl, blk in FILL_SHAPES}
    print(json.dumps({"fill_hidden": h, "rows": B, "grids": grids, "us": {k: round(v, 2) for k, v in us.items()}}),
          flush=True)
    del bufs
    torch.cuda.empty_cache()


def load_traffic(key):
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 --pmc summary (profiles/), when one exists for this kernel."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            t = json.load(f)
        return t.get("lpr{}_vpl{}_lds{}_b{}".format(key[1], key[2], key[3], key[4]))
    except (OSError, ValueError):
        return None


def run_extra(torch, ops, args):
    """BASELINE.json's other configs, µs/call (median over timed calls)."""
    out = {}
    steps = max(10, args.steps)
    # decode shapes with 1% outliers x50
    dec = [(b, h, torch.bfloat16, "outliers") for b in (1, 8, 32, 128, 512) for h in (4096, 8192)]
    us = time_shapes(torch, ops.hp_rms_norm, dec, steps, args.warmup)
    out["decode_bf16"] = [{"rows": b, "hidden": h, "us_per_call": round(u, 2), "us_p10": round(p10, 2),
                           "us_p90": round(p90, 2)} for (b, h, _, _), (u, p10, p90) in zip(dec, us)]
    # the same decode shapes replayed from a HIP graph (64 calls per replay over 8 buffer sets):
    # the per-call time a serving loop that captures its step sees, without Python's launch cost
    graph = []
    for (b, h, dt, dist) in dec:
        bufs = make_bufs(torch, [(b, h, dt, dist)], lambda r, hh: 8)
        sets, w = bufs[0]
        s_ = torch.cuda.Stream()
        s_.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s_):
            for x, r in sets:
                ops.hp_rms_norm(x, w, r, EPS)
        torch.cuda.current_stream().wait_stream(s_)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(64):
                x, r = sets[i % 8]
                ops.hp_rms_norm(x, w, r, EPS)
        for _ in range(3):
            g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        graph.append({"rows": b, "hidden": h, "us_per_call": round(e0.elapsed_time(e1) * 1e3 / 640, 2)})
        del g, bufs, sets
    torch.cuda.empty_cache()
    out["decode_bf16_hip_graph"] = graph
    # the decode shapes and two mid-size batches with the batch-invariant mode on (every call
    # takes its width's large-batch shape), beside the default mode's time for the same shape
    mid = [(1024, 4096, torch.bfloat16, "bench"), (2048, 2048, torch.bfloat16, "bench")]
    default_us = {(b, h): u for (b, h, _, _), (u, _, _) in zip(dec, us)}
    for (b, h, _, _), (u, _, _) in zip(mid, time_shapes(torch, ops.hp_rms_norm, mid, steps, args.warmup)):
        default_us[(b, h)] = u
    previous = ops.set_batch_invariant(True)
    try:
        inv = time_shapes(torch, ops.hp_rms_norm, dec + mid, steps, args.warmup)
    finally:
        ops.set_batch_invariant(previous)
    out["batch_invariant_mode_bf16"] = [
        {"rows": b, "hidden": h, "us_per_call": round(u, 2), "default_mode_us_per_call": round(default_us[(b, h)], 2)}
        for (b, h, _, _), (u, _, _) in zip(dec + mid, inv)]
    # fp16 non-power-of-two hidden
    f16 = [(B, 5120, torch.float16, "bench"), (B, 7168, torch.float16, "bench")]
    us = time_shapes(torch, ops.hp_rms_norm, f16, steps, args.warmup)
    out["fp16"] = [{"rows": b, "hidden": h, "us_per_call": round(u, 2), "us_p10": round(p10, 2),
                    "us_p90": round(p90, 2), "gbs": round(fused_bytes(b, h) / (u * 1e-6) / 1e9, 1)}
                   for (b, h, _, _), (u, p10, p90) in zip(f16, us)]
    # fused add+RMSNorm with FP8 output (reads x, r, w; writes r and H bytes + a scale per row)
    fp8 = []
    for h in (4096, 8192, 16384, 32768):
        n = cold_sets(B, h)
        sets = [make_set(torch, B, h, torch.bfloat16, 7000 + i, "cuda:0") for i in range(n)]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")
        qs = [torch.empty(B, h, dtype=torch.float8_e4m3fn, device="cuda:0") for _ in range(n)]
        sc = torch.empty(B, 1, dtype=torch.float32, device="cuda:0")
        for i in range(args.warmup):
            ops.hp_rms_norm_fp8(qs[i % n], sc, sets[i % n][0], w, sets[i % n][1], EPS)
        ncalls = max(steps, n)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        prefill(torch, 10)
        e0.record()
        for i in range(ncalls):
            ops.hp_rms_norm_fp8(qs[i % n], sc, sets[i % n][0], w, sets[i % n][1], EPS)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / ncalls
        # the same with each row's maximum bounded above (a bound most rows reach)
        ub = torch.tensor([2.0], dtype=torch.float32, device="cuda:0")

        def call_ub(i, qs=qs, sets=sets, w=w, sc=sc, ub=ub):
            ops.hp_rms_norm_fp8_ub(qs[i], sc, sets[i][0], w, sets[i][1], ub, EPS)
        us_ub = time_rotating(torch, call_ub, n, steps, args.warmup)
        nbytes = 7 * B * h + 2 * h + 4 * B
        fp8.append({"rows": B, "hidden": h, "us_per_call": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                    "bytes_per_call": nbytes, "us_per_call_scale_ub": round(us_ub, 2)})
        del sets, qs
        torch.cuda.empty_cache()
    out["fp8_output_bf16"] = fp8
    # the FP8 output with one given scale for every row: no row maximum, no scales written
    fp8s = []
    for h in (4096, 8192, 16384, 32768):
        n = cold_sets(B, h)
        sets = [make_set(torch, B, h, torch.bfloat16, 7200 + i, "cuda:0") for i in range(n)]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")
        qs = [torch.empty(B, h, dtype=torch.float8_e4m3fn, device="cuda:0") for _ in range(n)]
        sc = torch.full((1,), 0.02, dtype=torch.float32, device="cuda:0")

        def call(i, sets=sets, qs=qs, sc=sc, w=w):
            ops.hp_rms_norm_fp8_static(qs[i], sc, sets[i][0], w, sets[i][1], EPS)
        us = time_rotating(torch, call, n, steps, args.warmup)
        nbytes = 7 * B * h + 2 * h + 4
        fp8s.append({"rows": B, "hidden": h, "us_per_call": round(us, 2),
                     "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes_per_call": nbytes})
        del sets, qs
        torch.cuda.empty_cache()
    out["fp8_static_output_bf16"] = fp8s
    # the FP8 output with one float32 scale per 128 elements (per-token-group quantisation)
    fp8g = []
    for h in (4096, 8192, 16384, 32768):
        n = cold_sets(B, h)
        sets = [make_set(torch, B, h, torch.bfloat16, 7300 + i, "cuda:0") for i in range(n)]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")
        qs = [torch.empty(B, h, dtype=torch.float8_e4m3fn, device="cuda:0") for _ in range(n)]
        sc = torch.empty(B, h // 128, dtype=torch.float32, device="cuda:0")
        # the column-major (token-minor) scale layout some block-scaled GEMMs read
        sc_cols = torch.empty(h // 128, B, dtype=torch.float32, device="cuda:0").t()

        def call(i, sets=sets, qs=qs, sc=sc, w=w):
            ops.hp_rms_norm_fp8_group(qs[i], sc, sets[i][0], w, sets[i][1], EPS)

        def call_cols(i, sets=sets, qs=qs, sc=sc_cols, w=w):
            ops.hp_rms_norm_fp8_group(qs[i], sc, sets[i][0], w, sets[i][1], EPS)
        us = time_rotating(torch, call, n, steps, args.warmup)
        us_cols = time_rotating(torch, call_cols, n, steps, args.warmup)
        nbytes = 7 * B * h + 2 * h + 4 * B * (h // 128)
        fp8g.append({"rows": B, "hidden": h, "us_per_call": round(us, 2),
                     "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes_per_call": nbytes,
                     "us_per_call_column_major_scales": round(us_cols, 2)})
        del sets, qs
        torch.cuda.empty_cache()
    out["fp8_group128_output_bf16"] = fp8g
    # OCP MX outputs (MXFP8 / MXFP4): reads x, r; writes r, the elements and one scale byte per 32
    mx = []
    for fmt, name in ((ops.MXFP8, "mxfp8"), (ops.MXFP4, "mxfp4")):
        for h in (4096, 8192, 16384, 32768):
            n = cold_sets(B, h)
            sets = [make_set(torch, B, h, torch.bfloat16, 7500 + i, "cuda:0") for i in range(n)]
            w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")
            qs = [torch.empty(B, h if fmt == ops.MXFP8 else h // 2, dtype=torch.uint8, device="cuda:0")
                  for _ in range(n)]
            sc = torch.empty(B, h // 32, dtype=torch.uint8, device="cuda:0")

            def call(i, sets=sets, qs=qs, sc=sc, w=w, fmt=fmt):
                ops.hp_rms_norm_mx(qs[i], sc, sets[i][0], w, sets[i][1], EPS, fmt)
            us = time_rotating(torch, call, n, steps, args.warmup)
            nbytes = 6 * B * h + (B * h if fmt == ops.MXFP8 else B * h // 2) + B * h // 32 + 2 * h
            mx.append({"format": name, "rows": B, "hidden": h, "us_per_call": round(us, 2),
                       "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes_per_call": nbytes})
            del sets, qs
            torch.cuda.empty_cache()
    out["mx_output_bf16"] = mx
    # out-of-place fused op (input and residual only read): the same 4 rows of bytes per row
    oop = []
    for h in (4096, 8192, 16384, 32768):
        n = cold_sets(B, h, floor=2, span=1 << 30)
        sets = [make_set(torch, B, h, torch.bfloat16, 8000 + i, "cuda:0") for i in range(n)]
        outs = [(torch.empty_like(x), torch.empty_like(r)) for x, r in sets]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")

        def call(i, sets=sets, outs=outs, w=w):
            ops.fused_add_rms_norm_out(outs[i][0], outs[i][1], sets[i][0], w, sets[i][1], EPS)
        us = time_rotating(torch, call, n, steps, args.warmup)
        oop.append({"rows": B, "hidden": h, "us_per_call": round(us, 2),
                    "gbs": round(fused_bytes(B, h) / (us * 1e-6) / 1e9, 1)})
        del sets, outs
        torch.cuda.empty_cache()
    out["out_of_place_bf16"] = oop
    # plain RMSNorm (no residual): one read and one write of the row
    plain = []
    for h in (4096, 8192, 16384, 32768):
        n = cold_sets(B, h, floor=2, span=1 << 30)
        sets = [make_set(torch, B, h, torch.bfloat16, 9000 + i, "cuda:0")[0] for i in range(n)]
        outs = [torch.empty_like(x) for x in sets]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")

        def call(i, sets=sets, outs=outs, w=w):
            ops.rms_norm(outs[i], sets[i], w, EPS)
        us = time_rotating(torch, call, n, steps, args.warmup)
        nbytes = 2 * B * h * 2 + 2 * h
        plain.append({"rows": B, "hidden": h, "us_per_call": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)})
        del sets, outs
        torch.cuda.empty_cache()
    out["plain_rmsnorm_bf16"] = plain
    # rows off the 128-byte grid: odd widths (the tail variants; from 4104 elements shifted rows),
    # row starts 2 bytes off 16-byte alignment (shifted from 4104), and 16-byte aligned rows with
    # a stride of hidden + 8 (the unaligned variants, rotated); beside them rows on the grid at
    # strides of hidden + 64 and + 128 (the table's kernels at a pitch other than hidden)
    una = []
    for h, off, pad in ((999, 0, 0), (2049, 0, 0), (4097, 0, 0), (8191, 0, 0), (16391, 0, 0), (32775, 0, 0),
                        (4096, 1, 8), (16384, 1, 8), (32768, 1, 8), (16384, 0, 8), (32768, 0, 8),
                        (16384, 0, 64), (32768, 0, 64), (32768, 0, 128)):
        stride = h + off + pad
        n = cold_sets(B, stride)
        bases = [make_set(torch, B, stride, torch.bfloat16, 9500 + i, "cuda:0") for i in range(n)]
        sets = [(x[:, off:off + h], r[:, off:off + h]) for x, r in bases]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")

        def call(i, sets=sets, w=w):
            ops.hp_rms_norm(sets[i][0], w, sets[i][1], EPS)
        us = time_rotating(torch, call, n, steps, args.warmup)
        una.append({"rows": B, "hidden": h, "row_start_offset_bytes": 2 * off, "row_stride": stride,
                    "us_per_call": round(us, 2), "gbs": round(fused_bytes(B, h) / (us * 1e-6) / 1e9, 1)})
        del bases, sets
        torch.cuda.empty_cache()
    out["unaligned_rows_bf16"] = una
    # partial sums + fused op: P parts read, residual read and written, output written
    red = []
    h = 8192
    for nparts in (2, 4, 8):
        per_set = (nparts + 2) * B * h * 2
        n = max(2, -(-(1 << 30) // per_set))
        g = torch.Generator(device="cuda:0").manual_seed(nparts)
        sets = [([torch.randn(B, h, device="cuda:0", generator=g).to(torch.bfloat16) for _ in range(nparts)],
                 torch.randn(B, h, device="cuda:0", generator=g).to(torch.bfloat16),
                 torch.empty(B, h, dtype=torch.bfloat16, device="cuda:0")) for _ in range(n)]
        w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")

        def call(i, sets=sets, w=w):
            parts, r, o = sets[i]
            ops.reduce_add_rms_norm(o, parts, w, r, EPS)
        us = time_rotating(torch, call, n, steps, args.warmup)
        nbytes = (nparts + 3) * B * h * 2 + 2 * h
        red.append({"parts": nparts, "rows": B, "hidden": h, "us_per_call": round(us, 2),
                    "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes_per_call": nbytes})
        del sets
        torch.cuda.empty_cache()
    out["reduce_parts_bf16"] = red
    # the same form at decode sizes (a tensor-parallel step's all-reduce with a few rows): the
    # latency rows load every part before adding them; the fused op beside them (0 parts)
    redd = []
    for h in (4096, 8192):
        for rows in (1, 32):
            g = torch.Generator(device="cuda:0").manual_seed(h + rows)
            w = make_weight(torch, h, torch.bfloat16, 1, "cuda:0")
            for nparts in (0, 2, 8):
                sets = [([torch.randn(rows, h, device="cuda:0", generator=g).to(torch.bfloat16)
                          for _ in range(max(nparts, 1))],
                         torch.randn(rows, h, device="cuda:0", generator=g).to(torch.bfloat16),
                         torch.empty(rows, h, dtype=torch.bfloat16, device="cuda:0")) for _ in range(16)]

                def call(i, sets=sets, w=w, nparts=nparts):
                    parts, r, o = sets[i]
                    if nparts:
                        ops.reduce_add_rms_norm(o, parts, w, r, EPS)
                    else:
                        ops.hp_rms_norm(parts[0], w, r, EPS)
                us = time_rotating(torch, call, len(sets), steps, args.warmup)
                redd.append({"parts": nparts, "rows": rows, "hidden": h, "us_per_call": round(us, 2)})
                del sets
    out["reduce_parts_decode_bf16"] = redd
    # streamer (the reference "relu" = copy, and the true ReLU) at (4096, 14336)
    rows, h = B, 14336
    res = []
    for dtype in (torch.bfloat16, torch.float16):
        n = cold_sets(rows, h)
        sets = [torch.randn(rows, h, device="cuda:0").to(dtype) for _ in range(n)]
        outs = [torch.empty_like(t) for t in sets]
        for name, fn in (("copy", ops.relu), ("relu", ops.relu_max0)):
            for i in range(args.warmup):
                fn(outs[i % n], sets[i % n])
            ncalls = max(steps, n)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            prefill(torch, 10)
            e0.record()
            for i in range(ncalls):
                fn(outs[i % n], sets[i % n])
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / ncalls
            res.append({"op": name, "dtype": str(dtype).replace("torch.", ""), "rows": rows, "hidden": h,
                        "us_per_call": round(us, 2), "gbs": round(2 * rows * h * 2 / (us * 1e-6) / 1e9, 1)})
        del sets, outs
    out["streamer"] = res
    torch.cuda.empty_cache()
    # the vendor stack's own bandwidth on the same box, 1 GiB operands (reference points)
    n = 1 << 29
    a = torch.empty(n, dtype=torch.bfloat16, device="cuda:0").normal_()
    b = torch.empty_like(a)
    ceil = {}
    for name, fn, nbytes in (("torch_copy_gbs", lambda: b.copy_(a), 4 * n),
                             ("torch_fill_gbs", lambda: b.fill_(1.0), 2 * n),
                             ("torch_sum_gbs", lambda: a.sum(), 2 * n)):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        prefill(torch, 5)
        e0.record()
        for _ in range(10):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ceil[name] = round(nbytes / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9, 1)
    out["vendor_stack_bandwidth"] = ceil
    del a, b
    torch.cuda.empty_cache()
    # a copy that moves the fused op's bytes at (B, H): the streamer over (B, 2H), one read
    # and one write of 2·B·H elements; the time any one kernel launch needs to stream that
    # many bytes on this stack (main() sets the fused op's time beside it)
    same = []
    for h in (1024, 2048, 4096, 8192, 16384, 32768):
        n = cold_sets(B, 2 * h)
        srcs = [torch.randn(B, 2 * h, device="cuda:0").to(torch.bfloat16) for _ in range(n)]
        dsts = [torch.empty_like(t) for t in srcs]

        def call(i, srcs=srcs, dsts=dsts):
            ops.relu(dsts[i], srcs[i])
        us = statistics.median(time_rotating(torch, call, n, steps, args.warmup) for _ in range(3))
        nbytes = 4 * B * h * 2
        same.append({"hidden": h, "copy_shape": [B, 2 * h], "copy_bytes": nbytes, "us_per_call": round(us, 2),
                     "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)})
        del srcs, dsts
        torch.cuda.empty_cache()
    out["copy_same_bytes_bf16"] = same
    # the reference's published harness is not in its repository; for comparison
    # with those numbers, the same shapes with one buffer set reused every call
    # (working sets up to 256 MB then sit in the Infinity Cache)
    hot = []
    for h in (1024, 4096, 8192, 16384, 32768):
        shape = (B, h, torch.bfloat16, "bench")
        bufs = make_bufs(torch, [shape], lambda r, hh: 1)
        (x, r), w = bufs[0][0][0], bufs[0][1]
        for _ in range(args.warmup):
            ops.hp_rms_norm(x, w, r, EPS)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        prefill(torch, 5)
        e0.record()
        for _ in range(steps):
            ops.hp_rms_norm(x, w, r, EPS)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        hot.append({"rows": B, "hidden": h, "us_per_call": round(us, 2),
                    "gbs": round(fused_bytes(B, h) / (us * 1e-6) / 1e9, 1)})
        del bufs, x, r
        torch.cuda.empty_cache()
    out["same_buffers_every_call"] = hot
    # the op beside kernels that move its bytes without its arithmetic (bench library)
    from hp_rms_norm_amd import abi
    out["ceiling_bf16"] = ceiling(torch, abi, ops, [4096, 8192, 12288, 16384, 32768], steps, args.warmup, trials=3)
    return out


if __name__ == "__main__":
    main()
