#!/usr/bin/env python
"""Benchmark of the gfx950 rasterizer: forward + backward on one MI355X.

Workload: 1,000,000 fp32 Gaussians, 1920x1080, SH degree
3, forward with depth and alpha outputs plus the manual backward, upstream
gradients ~N(0,1) on colour, depth and alpha, camera direction re-drawn per
iteration from the seed.  One step = one forward + backward through the
public ``GaussianRasterizer`` and ``torch.autograd.backward``.

Prints ONE JSON line on stdout (everything else goes to stderr) with the
metric Gaussians/s = N / t(fwd+bwd), the per-stage times measured live with
HIP events on the launch stream, the HBM-roofline fraction of the dominant
kernel and of the whole iteration, and the CPU baseline (the C oracle on
this host's cores, one fwd+bwd of the same scene).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from collections import defaultdict
from contextlib import contextmanager
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, GB/s
METRIC = "fwd+bwd ms/iter & Gaussians/s @1M Gaussians 1080p SH3; % HBM roofline"


def log(*args):
    print(*args, file=sys.stderr, flush=True)


class StageTimer:
    """Records a pair of HIP events around each pipeline stage on the current stream."""

    def __init__(self):
        import torch

        self.torch = torch
        self.enabled = False
        self.events = defaultdict(list)
        self.notes = defaultdict(list)

    @contextmanager
    def __call__(self, name):
        if not self.enabled:
            yield
            return
        torch = self.torch
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        try:
            yield
        finally:
            end.record()
            self.events[name].append((start, end))

    def chain(self, names):
        """len(names) + 1 events for a C entry point to record between its
        stages; stage names[i] spans events i..i+1.  Each event is recorded
        once here so that its HIP event exists; the C side records it again
        at the stage boundary."""
        if not self.enabled:
            return None
        import ctypes

        torch = self.torch
        events = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
        for e in events:
            e.record()
        for name, a, b in zip(names, events[:-1], events[1:]):
            self.events[name].append((a, b))
        return (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events])

    def note(self, key, value):
        if self.enabled:
            self.notes[key].append(value)

    def mean_ms(self, steps: int) -> dict:
        """Mean time per step of each stage (a stage that runs twice in a step counts twice)."""
        return {name: sum(s.elapsed_time(e) for s, e in pairs) / steps for name, pairs in self.events.items()}


def sort_passes(tiles: int) -> int:
    """Passes of the 64-bit (tile << 32 | depth) key sort, 8 bits each."""
    return math.ceil((32 + math.ceil(math.log2(tiles))) / 8)


def algorithmic_bytes(N: int, R: float, P: int, T: int, dataflow: str) -> dict:
    """Bytes crossing each stage boundary once (the SH3, depth-on accounting of the
    reference dataflow): preprocess 112N + SH 228N, scan 8N, duplicate 44N + 12R
    (64-bit key + value) or 44N + 8R (tile id + value), ranges 8R + 8T, render
    44R + 24P + 8T, render backward 44R + 28P + 40N + 8T, SH + preprocess
    backward 624N.  Sorts: the one 64-bit key sort moves 24R per pass over
    ceil((32 + ceil(log2 T)) / 8) passes; the depth-then-tile dataflow moves 16N
    per pass over 4 passes for the depth sort and 16R per pass over
    ceil(log2 T / 8) passes for the tile sort."""
    out = {
        "preprocess": 340.0 * N,
        "scan": 8.0 * N,
        "ranges": 8.0 * R + 8.0 * T,
        "render": 44.0 * R + 24.0 * P + 8.0 * T,
        "render_bwd": 44.0 * R + 28.0 * P + 40.0 * N + 8.0 * T,
        "preprocess_bwd": 624.0 * N,
    }
    if dataflow == "warp_radix":
        out["duplicate"] = 44.0 * N + 12.0 * R
        out["sort"] = sort_passes(T) * 24.0 * R
    else:
        out["duplicate"] = 44.0 * N + 8.0 * R
        out["depth_sort"] = 4 * 16.0 * N
        out["sort"] = math.ceil((T - 1).bit_length() / 8) * 16.0 * R
    return out


def read_traffic(stage: str):
    """HBM bytes per launch of a stage from the committed rocprofv3 PMC summary, if present."""
    path = ROOT / "profiles" / "traffic_config2.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 2 and parts[0] == f"{stage}:":
            try:
                return float(parts[1])
            except ValueError:
                return None
    return None


def measure_copy_bandwidth(device, nbytes: int = 1 << 30, reps: int = 5) -> float:
    """Achievable HBM bandwidth (GB/s, read + write bytes) of a plain device copy of
    nbytes, timed with HIP events on the current stream."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device=device).fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    end.synchronize()
    seconds = start.elapsed_time(end) * 1e-3 / reps
    del src, dst
    return 2.0 * nbytes / seconds / 1e9


# Kernel-name prefix -> pipeline stage, for the rocprofv3 PMC summary.
STAGE_OF_KERNEL = (
    ("gs::preprocess_fwd_kernel", "preprocess"),
    ("gs::scan_", "scan"),
    ("gs::zero_info_kernel", "scan"),
    ("gs::depth_keys_kernel", "depth_sort"),
    ("gs::duplicate_keys_kernel", "duplicate"),
    ("gs::duplicate_tiles_kernel", "duplicate"),
    ("gs_sort::", "sort"),
    ("gs_seg::", "sort"),
    ("gs::zero_ranges_kernel", "ranges"),
    ("gs::tile_ranges_kernel", "ranges"),
    ("gs::tile_ranges_u32_kernel", "ranges"),
    ("gs::render_fwd_kernel", "render"),
    ("gs::render_bwd_kernel", "render_bwd"),
    ("gs::preprocess_bwd_kernel", "preprocess_bwd"),
)


def _stage_of(kernel_name: str):
    name = kernel_name.replace("void ", "", 1)
    for prefix, stage in STAGE_OF_KERNEL:
        if name.startswith(prefix):
            return stage
    return None


# The profiling commands behind the committed summaries (from the repository
# root R on the GPU box, each pass a run of its own); the summaries repeat
# them so that each file says how it was made.
_PROFILE_PREAMBLE = "#   cd /tmp && export TMPDIR=/tmp"
def _stats_commands(config: int) -> list[str]:
    c = f"c{config}"
    cfg = "" if config == 2 else f"--config {config} "
    return [
        _PROFILE_PREAMBLE,
        f"#   rocprofv3 --kernel-trace --stats --output-format csv -d $R/gpurun_out/prof_{c} -o {c} -- \\",
        f"#       python3 $R/bench.py {cfg}--steps 10 --warmup 3 --no-cpu-baseline > $R/gpurun_out/prof_{c}/bench.json \\",
        f"#       2> $R/gpurun_out/prof_{c}/bench.err",
        f"#   python3 bench.py --stats-summary gpurun_out/prof_{c}/{c}_kernel_stats.csv "
        f"profiles/kernel_stats_config{config}.txt \\",
        f"#       gpurun_out/prof_{c}/bench.err" + ("" if config == 2 else f" --profile-config {config}"),
    ]


PROFILE_COMMANDS = {
    "stats": _stats_commands(2),
    "pmc": [
        _PROFILE_PREAMBLE,
        "#   rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/gpurun_out/pmc_c2 -o fetch -- \\",
        "#       python3 $R/bench.py --steps 3 --warmup 1 --no-cpu-baseline --no-stage-timing",
        "#   rocprofv3 --pmc WRITE_SIZE --output-format csv -d $R/gpurun_out/pmc_c2 -o write -- \\",
        "#       python3 $R/bench.py --steps 3 --warmup 1 --no-cpu-baseline --no-stage-timing",
        "#   python3 bench.py --pmc-summary gpurun_out/pmc_c2/fetch_counter_collection.csv \\",
        "#       gpurun_out/pmc_c2/write_counter_collection.csv profiles/traffic_config2.txt",
    ],
    "sq": [
        _PROFILE_PREAMBLE,
        "#   rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_INSTS_LDS SQ_ACTIVE_INST_LDS \\",
        "#       SQ_LDS_BANK_CONFLICT SQ_WAVE_CYCLES SQ_BUSY_CYCLES --output-format csv -d $R/gpurun_out/sq_c2 -o sq -- \\",
        "#       python3 $R/bench.py --steps 3 --warmup 1 --no-cpu-baseline --no-stage-timing",
        "#   python3 bench.py --sq-summary gpurun_out/sq_c2/sq_counter_collection.csv profiles/sq_counters_config2.txt",
    ],
}


def summarize_pmc(fetch_csv: str, write_csv: str, out_path: str, copy_bytes: int = 1 << 30) -> None:
    """Turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE, then WRITE_SIZE,
    both in KiB per dispatch) into per-stage HBM bytes per launch.  Each counter is
    scaled by what it reads for the calibration copy (the largest device copy, of
    copy_bytes read and copy_bytes written), so the figures are in true bytes."""
    import csv

    def load(path, counter):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        per_stage = defaultdict(float)
        copies = []
        renders = 0
        for r in rows:
            value = float(r["Counter_Value"])
            stage = _stage_of(r["Kernel_Name"])
            if stage is not None:
                per_stage[stage] += value
            if "copyBuffer" in r["Kernel_Name"]:
                copies.append(value)
            if stage == "render":
                renders += 1
        return per_stage, max(copies), renders

    fetch, fetch_copy, iters = load(fetch_csv, "FETCH_SIZE")
    write, write_copy, iters_w = load(write_csv, "WRITE_SIZE")
    f_scale = copy_bytes / fetch_copy
    w_scale = copy_bytes / write_copy
    lines = [
        "# HBM traffic per launch of each stage (bytes), config 2, from rocprofv3 --pmc",
        f"# FETCH_SIZE scale {f_scale:.2f} B/unit, WRITE_SIZE scale {w_scale:.2f} B/unit "
        f"(calibration copy of {copy_bytes} B read + {copy_bytes} B written read "
        f"{fetch_copy:.0f} / {write_copy:.0f} units)",
        f"# iterations averaged: {iters} (fetch run), {iters_w} (write run)",
        "# commands:",
        *PROFILE_COMMANDS["pmc"],
        "# format: '<stage>: <bytes per launch> fetch <bytes> write <bytes>' (bench.py reads the first number)",
    ]
    for stage in sorted(set(fetch) | set(write)):
        fb = fetch.get(stage, 0.0) * f_scale / max(iters, 1)
        wb = write.get(stage, 0.0) * w_scale / max(iters_w, 1)
        lines.append(f"{stage}: {fb + wb:.0f} fetch {fb:.0f} write {wb:.0f}")
    Path(out_path).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def summarize_sq(counter_csv: str, out_path: str) -> None:
    """Per-kernel means per dispatch of the SQ counters in one rocprofv3 --pmc
    counter_collection.csv, with the LDS bank-conflict rate
    (SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS, both in cycles) and VALU
    instructions per wave."""
    import csv

    per = defaultdict(lambda: defaultdict(float))
    dispatches = defaultdict(set)
    for r in csv.DictReader(open(counter_csv)):
        name = r["Kernel_Name"]
        short = name.replace("void ", "", 1).split("(")[0]
        if _stage_of(name) is None:
            continue
        per[short][r["Counter_Name"]] += float(r["Counter_Value"])
        dispatches[short].add(r["Dispatch_Id"])
    counters = sorted({c for d in per.values() for c in d})
    lines = ["# SQ counters per kernel, config 2 (1M Gaussians, 1920x1080, SH3, fwd+bwd), one MI355X",
             "# commands:", *PROFILE_COMMANDS["sq"],
             "# lds_conflict_rate = SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS (cycles per LDS-active cycle)",
             "# SQ counters per dispatch (mean); columns: kernel, dispatches, "
             + ", ".join(counters) + ", lds_conflict_rate, valu_insts_per_wave"]
    for k in sorted(per):
        n = len(dispatches[k])
        d = {c: per[k][c] / n for c in counters}
        lds = d.get("SQ_ACTIVE_INST_LDS", 0.0)
        rate = d.get("SQ_LDS_BANK_CONFLICT", 0.0) / lds if lds else 0.0
        waves = d.get("SQ_WAVES", 0.0)
        vpw = d.get("SQ_INSTS_VALU", 0.0) / waves if waves else 0.0
        lines.append(f"{k} {n} " + " ".join(f"{d[c]:.4g}" for c in counters) + f" {rate:.4f} {vpw:.1f}")
    Path(out_path).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


CONFIG_TITLES = {
    1: "config 1 (100k Gaussians, 800x800, SH3, fwd+bwd)",
    2: "config 2 (1M Gaussians, 1920x1080, SH3, fwd+bwd with depth and alpha)",
    3: "config 3 (5M Gaussians, 1920x1080, SH3, heavy tail of large splats, fwd+bwd)",
    4: "config 4 (flow API, 1M Gaussians, 1280x720, SH3, top-K 20, fwd+bwd)",
}


def summarize_stats(stats_csv: str, out_path: str, bench_err: str | None = None, config: int = 2) -> None:
    """rocprofv3 --kernel-trace --stats kernel_stats.csv -> calls, average / min /
    max duration (us), share of GPU time and name of each kernel, longest first;
    with the profiled bench run's stderr, its own HIP-event stage times too."""
    import csv

    rows = list(csv.DictReader(open(stats_csv)))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = [f"# Kernel time, {CONFIG_TITLES[config]}, one MI355X",
             "# 23 iterations (3 warm-up, 10 timed, 10 with per-stage events) plus bench.py's 1 GiB copy calibration",
             "# commands:", *_stats_commands(config)]
    if bench_err:
        stage_lines = [line.strip() for line in open(bench_err) if line.startswith("[bench]")]
        if stage_lines:
            lines.append("# bench.py's own report in the same run (HIP events under the tracer, same cameras):")
            lines += [f"#   {line}" for line in stage_lines]
    lines.append("# columns: calls, average us, min us, max us, share of GPU time, kernel")
    for r in rows:
        lines.append(f"{int(r['Calls']):5d} {float(r['AverageNs']) / 1e3:10.1f} {float(r['MinNs']) / 1e3:10.1f} "
                     f"{float(r['MaxNs']) / 1e3:10.1f} {float(r['Percentage']):6.2f}%  {r['Name'][:110]}")
    Path(out_path).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def cpu_baseline(scene, grads) -> dict:
    """One fwd+bwd of the same scene with the C oracle on this host's cores."""
    import oracle
    from gswarp_amd import configs

    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "16")), 16)
    oracle.set_num_threads(threads)
    host = configs.scene_to_numpy(scene)
    g = {k: v.detach().cpu().numpy() for k, v in grads.items()}
    t0 = time.perf_counter()
    res = oracle.rasterize(host)
    oracle.rasterize_backward(host, res, g["color"], g["depth"], g["alpha"])
    dt = time.perf_counter() - t0
    n = host["means3D"].shape[0]
    return {
        "value": n / dt,
        "unit": "Gaussians/s",
        "cores": oracle.num_threads(),
        "kind": "port",
        "sample": f"one fwd+bwd of the iteration-0 view of this workload ({n} Gaussians) by the C oracle "
                  f"(oracle/gs_oracle.c, OpenMP), {dt:.2f} s",
        "seconds": dt,
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--config", type=int, default=2, choices=(1, 2, 3, 4))
    parser.add_argument("--count", type=int, default=None, help="override the Gaussian count")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-stage-timing", action="store_true")
    parser.add_argument("--sort-mode", default=None, choices=("warp_depth_stable_tile", "warp_radix", "torch"),
                        help="binning sort mode (default: the API default, warp_depth_stable_tile)")
    parser.add_argument("--pmc-summary", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "OUT"),
                        help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) into OUT and exit")
    parser.add_argument("--sq-summary", nargs=2, metavar=("COUNTER_CSV", "OUT"),
                        help="summarise one rocprofv3 --pmc run of SQ counters into OUT and exit")
    parser.add_argument("--profile-config", type=int, default=2, choices=(1, 2, 3, 4),
                        help="configuration a --stats-summary run profiled (for its header)")
    parser.add_argument("--stats-summary", nargs="+", metavar="PATH",
                        help="KERNEL_STATS_CSV OUT [BENCH_ERR]: summarise one rocprofv3 --kernel-trace --stats "
                             "run into OUT and exit")
    args = parser.parse_args()
    if args.stats_summary:
        summarize_stats(*args.stats_summary, config=args.profile_config)
        return 0
    if args.sq_summary:
        summarize_sq(*args.sq_summary)
        return 0
    if args.pmc_summary:
        summarize_pmc(*args.pmc_summary)
        return 0

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(view-parallel sharding is a design note). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from gswarp_amd import _pipeline, _runtime, configs
    from gswarp_amd.rasterizer import GaussianRasterizationSettings, GaussianRasterizer
    from gswarp_amd.rasterizer_flow import GaussianRasterizationSettings as FlowSettings
    from gswarp_amd.rasterizer_flow import GaussianRasterizer as FlowRasterizer

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.sort_mode:
        _runtime.set_binning_sort_mode(args.sort_mode)
    sort_mode = _runtime.get_binning_sort_mode()
    spec = configs.CONFIGS[args.config]
    t0 = time.perf_counter()
    scene = configs.make_scene(args.config, seed=args.seed, count=args.count, device=device)
    N = scene["means3D"].shape[0]
    W, H = scene["width"], scene["height"]
    P = W * H
    T = ((W + 15) // 16) * ((H + 15) // 16)
    grads = configs.upstream_gradients(args.config, W, H, seed=args.seed, device=device)
    total_steps = args.warmup + args.steps
    if args.config in (2, 3, 4):  # view direction re-drawn per iteration
        cams = [configs.orbit_camera(spec, args.seed, it) for it in range(total_steps)]
    else:
        cams = [scene] * total_steps
    flow = spec.flow
    settings = []
    for cam in cams:
        common = dict(image_height=H, image_width=W, tanfovx=cam["tanfovx"], tanfovy=cam["tanfovy"],
                      bg=scene["bg"], scale_modifier=1.0, viewmatrix=cam["viewmatrix"].to(device),
                      projmatrix=cam["projmatrix"].to(device), sh_degree=spec.sh_degree,
                      campos=cam["campos"].to(device), prefiltered=False, auto_tune=False, auto_tune_verbose=False)
        settings.append(FlowSettings(**common, enable_flow_grad=True, compute_flow_aux=True) if flow
                        else GaussianRasterizationSettings(**common))
    leaves = {k: scene[k].clone().requires_grad_(True) for k in ("means3D", "scales", "rotations", "opacities", "shs")}
    means2D = torch.zeros_like(leaves["means3D"], requires_grad=True)
    log(f"[bench] config {args.config}: N={N} {W}x{H} SH{spec.sh_degree} setup {time.perf_counter() - t0:.1f}s")

    timer = StageTimer()
    _pipeline.STAGE_TIMER = timer
    step_events = []

    def step(i: int, timed: bool):
        for t in (*leaves.values(), means2D):
            t.grad = None
        rast = (FlowRasterizer if flow else GaussianRasterizer)(settings[i])
        e0 = e1 = e2 = None
        if timed:
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record()
        out = rast(leaves["means3D"], means2D, leaves["opacities"], shs=leaves["shs"], scales=leaves["scales"],
                   rotations=leaves["rotations"])
        if timed:
            e1.record()
        if flow:
            outputs, upstream = [out[0], out[9]], [grads["color"], grads["x_mu"]]
        else:
            color, _radii, meta = out
            outputs, upstream = [color, meta.depth, meta.alpha], [grads["color"], grads["depth"], grads["alpha"]]
        torch.autograd.backward(outputs, upstream)
        if timed:
            e2.record()
            step_events.append((e0, e1, e2))

    for i in range(args.warmup):
        step(i, False)
    torch.cuda.synchronize()
    # Headline: the K timed steps run uninstrumented (only the two per-step
    # events around forward and backward).
    t_start = time.perf_counter()
    for i in range(args.warmup, total_steps):
        step(i, True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    fwd_bwd_events = list(step_events)
    # Per-stage breakdown: the same K cameras again with HIP events around
    # every stage (their recording adds host and GPU time, so these steps are
    # not part of the headline figure).
    if not args.no_stage_timing:
        timer.enabled = True
        for i in range(args.warmup, total_steps):
            step(i, False)
        torch.cuda.synchronize()
        timer.enabled = False
    _pipeline.STAGE_TIMER = None
    step_events[:] = fwd_bwd_events

    ms_per_step = 1000.0 * elapsed / args.steps
    fwd_ms = sum(a.elapsed_time(b) for a, b, _ in step_events) / len(step_events)
    bwd_ms = sum(b.elapsed_time(c) for _, b, c in step_events) / len(step_events)
    stage_ms = timer.mean_ms(args.steps) if not args.no_stage_timing else {}
    passes = timer.notes.get("sort_passes", [])
    Rs = timer.notes.get("num_rendered", [])
    R = sum(Rs) / len(Rs) if Rs else float("nan")
    log(f"[bench] {ms_per_step:.3f} ms/step (fwd {fwd_ms:.3f} ms, bwd {bwd_ms:.3f} ms), mean R={R:.0f}")

    roofline = None
    binning_sort = None
    stages = {}
    if stage_ms and Rs:
        dataflows = set(timer.notes.get("binning_dataflow", []))
        algo = algorithmic_bytes(N, R, P, T, "warp_radix" if dataflows == {"packed_key"} else sort_mode)
        for name, ms in sorted(stage_ms.items(), key=lambda kv: -kv[1]):
            gbps = algo[name] / (ms * 1e-3) / 1e9 if name in algo else None
            stages[name] = {"ms": round(ms, 4), "algorithmic_bytes": algo.get(name),
                            "achieved_GBps": None if gbps is None else round(gbps, 1),
                            "hbm_frac": None if gbps is None else round(gbps / HBM_PEAK_GBPS, 4)}
            log(f"[bench]   {name:15s} {ms:8.4f} ms" + ("" if gbps is None else f"  {gbps:8.1f} GB/s"))
        sort_names = [n for n in ("depth_sort", "sort") if n in stage_ms]
        sort_ms = sum(stage_ms[n] for n in sort_names)
        sort_bytes = sum(algo[n] for n in sort_names)
        binning_sort = {"mode": sort_mode, "stages": sort_names, "ms": round(sort_ms, 4),
                        "algorithmic_bytes": sort_bytes,
                        "hbm_frac": round(sort_bytes / (sort_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        binning_sort["dataflow"] = sorted(dataflows)
        log(f"[bench]   binning sort ({sort_mode}, {'/'.join(sorted(dataflows))}) {sort_ms:.4f} ms  "
            f"{binning_sort['hbm_frac'] * 100:.1f}% of HBM peak")
        dominant = max((n for n in stage_ms if n in algo), key=lambda n: stage_ms[n])
        achieved = algo[dominant] / (stage_ms[dominant] * 1e-3) / 1e9
        roofline = {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 5),
                    "traffic": read_traffic(dominant),
                    "algorithmic_bytes_per_launch": algo[dominant]}
    copy_gbps = measure_copy_bandwidth(device)
    log(f"[bench] device copy bandwidth {copy_gbps:.0f} GB/s")
    if roofline is not None:
        roofline["copy_GBps"] = round(copy_gbps, 1)
    iteration_bytes = 1056.0 * N + 252.0 * R + 52.0 * P + 24.0 * T if Rs else None

    result = {
        "metric": METRIC,
        "value": N / (ms_per_step * 1e-3),
        "unit": "Gaussians/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Gaussians and cameras, BASELINE config distributions)",
        "config": {"workload": f"config{args.config}: {spec.description}", "gaussians": N, "width": W,
                   "height": H, "sh_degree": spec.sh_degree, "tiles": T, "mean_num_rendered": R,
                   "mean_sort_passes": (sum(passes) / len(passes)) if passes else None,
                   "binning_dataflow": sorted(set(timer.notes.get("binning_dataflow", []))),
                   "parallelism": "single GPU"},
        "fwd_ms": fwd_ms,
        "bwd_ms": bwd_ms,
        "fwd_bwd_ms": ms_per_step,
        "hbm_copy_GBps": round(copy_gbps, 1),
        "iteration_hbm_frac": None if iteration_bytes is None else
        round(iteration_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 5),
        "stages": stages,
        "binning_sort": binning_sort,
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(scene, grads)  # the scene carries the iteration-0 camera
        log(f"[bench] CPU baseline {result['cpu_baseline']['seconds']:.2f} s on "
            f"{result['cpu_baseline']['cores']} threads")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
