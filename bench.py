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
import re
import sys
import time
from collections import defaultdict
from contextlib import contextmanager
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, GB/s
# VALU issue peak: 256 CUs x 4 SIMDs, one wave64 instruction per SIMD every 2 cycles (the
# 157.3 TFLOP/s fp32 vector rate) at the 2.4 GHz peak engine clock, in wave instructions per
# second.  Measured on one MI355X: fp32 add / mul / fma with VGPR or literal operands issue at
# 2.1-2.8 cycles; with an SGPR operand, and compares, selects, min / max, conversions and DPP, at
# about 4; v_exp_f32, v_rcp_f32 and the lane-swap permutes at about 8.
VALU_SIMDS = 1024
VALU_PEAK_INSTS = VALU_SIMDS * 2.4e9 / 2
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

    # scalar facts of a step (pair count, dataflow, sizes) are kept on every
    # step, so that an uninstrumented run (the profiler's) still reports its R
    ALWAYS = frozenset({"num_rendered", "binning_dataflow", "sort_passes", "bucket_entries", "bucket_valid"})

    def note(self, key, value):
        if self.enabled or key in self.ALWAYS:
            self.notes[key].append(value)

    def mean_ms(self, steps: int) -> dict:
        """Mean time per step of each stage (a stage that runs twice in a step counts twice)."""
        return {name: sum(s.elapsed_time(e) for s, e in pairs) / steps for name, pairs in self.events.items()}


def sort_passes(tiles: int) -> int:
    """Passes of the 64-bit (tile << 32 | depth) key sort, 8 bits each."""
    return math.ceil((32 + math.ceil(math.log2(tiles))) / 8)


def algorithmic_bytes(N: int, R: float, P: int, T: int, dataflow: str, flow_k: int = 0, entries: float = 0.0,
                      valid: float = 0.0, sized_scan: bool = False, sh_coeffs: int = 16) -> dict:
    """Bytes crossing each stage boundary once (the depth-on accounting of the
    reference dataflow): preprocess 112N + SH (36 + 12 K)N with K SH
    coefficients per Gaussian (228N at SH3, 48N at SH0), scan 8N (the two-pass
    scan that sizes the bucketed binning also reads the 16-byte cover words,
    24N; the one-pass scan takes the sizes from the preprocess), duplicate
    44N + 12R (64-bit key + value) or 44N + 8R (tile id + value), ranges
    8R + 8T (4R + 8T over the depth-then-tile dataflow's 32-bit tile ids),
    render 44R + 24P + 8T, render backward 44R + 28P + 40N + 8T, SH +
    preprocess backward (240 + 24 K)N (624N at SH3).  Sorts: the one 64-bit key sort moves 24R per
    pass over ceil((32 + ceil(log2 T)) / 8) passes; the depth-then-tile
    dataflow moves 16N per pass over 4 passes for the depth sort and 16R per
    pass over ceil(log2 T / 8) passes for the tile sort.  The bucketed binning
    (E entries of V Gaussians with a valid cover word) sorts depth as above,
    reads the depth order and the cover words and writes its entries (index +
    64-bit mask) in `bucket`, 20V + 12E, and reads the entries and writes the
    point list and ranges in `bucket_tiles`, 12E + 4R + 8T.  The flow render
    also writes its top-K auxiliaries, 16 K P (id, weight and the two x_mu
    components)."""
    out = {
        "preprocess": (148.0 + 12.0 * sh_coeffs) * N,
        "scan": (24.0 if sized_scan else 8.0) * N,
        "ranges": 8.0 * R + 8.0 * T,
        "render": 44.0 * R + 24.0 * P + 8.0 * T + 16.0 * flow_k * P,
        "render_bwd": 44.0 * R + 28.0 * P + 40.0 * N + 8.0 * T,
        "preprocess_bwd": (240.0 + 24.0 * sh_coeffs) * N,
    }
    if dataflow == "warp_radix":
        out["duplicate"] = 44.0 * N + 12.0 * R
        out["sort"] = sort_passes(T) * 24.0 * R
    elif dataflow == "buckets":
        out["depth_sort"] = 4 * 16.0 * N
        out["bucket"] = 20.0 * valid + 12.0 * entries
        out["bucket_tiles"] = 12.0 * entries + 4.0 * R + 8.0 * T
    else:
        out["duplicate"] = 44.0 * N + 8.0 * R
        out["depth_sort"] = 4 * 16.0 * N
        out["sort"] = math.ceil((T - 1).bit_length() / 8) * 16.0 * R
        out["ranges"] = 4.0 * R + 8.0 * T  # the sorted 32-bit tile ids, not 64-bit keys
    return out


def visited_pairs(n_contrib, width: int, height: int) -> int:
    """Pairs the backward blend reads: each 16x16 tile's list back to front from
    the largest n_contrib of its pixels, summed over the tiles (at most R;
    less where a tile's last entries blend into none of its pixels)."""
    import torch.nn.functional as F

    t = n_contrib.reshape(1, 1, height, width).float()
    return int(F.max_pool2d(t, 16, stride=16, ceil_mode=True).double().sum().item())


def early_stop_share(alpha, width: int, height: int, flow: bool = False) -> float:
    """Share of the forward's pixel slices (8x8 quadrants; 16x4 rows for the
    flow variant) that may have stopped before the end of their tile's list:
    every pixel has alpha > 0.99 (a pixel stops when T would fall below 1e-4,
    and alpha is at most 0.99 per Gaussian, so it stops only with T < 1e-2).
    Where this is 0 the forward reads all R pairs."""
    import torch.nn.functional as F

    a = alpha.reshape(1, 1, height, width)
    window = (4, 16) if flow else (8, 8)
    lowest = -F.max_pool2d(-a, window, stride=window, ceil_mode=True)
    return float((lowest > 0.99).double().mean().item())


def profile_path(kind: str, config: int) -> Path:
    return ROOT / "profiles" / f"{kind}_config{config}.txt"


def profile_provenance(kind: str, config: int):
    """Where a committed profile's figures come from: the file and the mean pair
    count R of the profiled run (its '# profiled run:' header line), or None."""
    path = profile_path(kind, config)
    if not path.exists():
        return None
    out = {"file": str(path.relative_to(ROOT)), "R": None}
    for line in path.read_text().splitlines():
        if line.startswith("# profiled run:"):
            m = re.search(r"mean R=([0-9.]+)", line)
            if m:
                out["R"] = float(m.group(1))
            break
    return out


def read_traffic(stage: str, config: int = 2):
    """HBM bytes per launch of a stage from the committed rocprofv3 PMC summary, if present."""
    path = profile_path("traffic", config)
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


def read_valu_insts(stage: str, config: int = 2):
    """VALU wave instructions per launch of a stage's kernel (the variant with the
    most dispatches) from the committed SQ counter summary, if present."""
    path = profile_path("sq_counters", config)
    if not path.exists():
        return None
    columns, best = None, None
    for line in path.read_text().splitlines():
        if line.startswith("# SQ counters per dispatch"):
            columns = [c.strip() for c in line.split("columns:", 1)[1].split(",")]
            continue
        if line.startswith("#") or columns is None:
            continue
        tokens = line.split()
        values = tokens[-(len(columns) - 1):]
        name = " ".join(tokens[:len(tokens) - len(values)])
        if _stage_of(name, config) != stage:
            continue
        row = dict(zip(columns[1:], values))
        try:
            dispatches, insts = float(row["dispatches"]), float(row["SQ_INSTS_VALU"])
        except (KeyError, ValueError):
            continue
        if best is None or dispatches > best[0]:
            best = (dispatches, insts)
    return None if best is None else best[1]


def profiled_run_line(bench_log: str | None) -> list[str]:
    """The header line naming the profiled bench run's mean pair count, taken
    from that run's own '[bench] ... mean R=' report (stderr)."""
    if not bench_log:
        return []
    for line in open(bench_log, errors="replace"):
        m = re.search(r"\[bench\] .*ms/step.*mean R=([0-9]+)", line)
        if m:
            return [f"# profiled run: mean R={m.group(1)} (bench.py's report: {line.strip()[8:]})"]
    return []


def valu_issue(stage: str, ms: float, config: int = 2):
    """The stage's VALU issue rate against VALU_PEAK_INSTS, from the committed
    instruction count and this run's stage time (slower instruction forms take
    two to four times the issue time of the fastest and are counted once, so a
    mix with them cannot reach 1.0)."""
    insts = read_valu_insts(stage, config)
    if insts is None or ms <= 0:
        return None
    rate = insts / (ms * 1e-3)
    return {"insts_per_launch": insts, "achieved": round(rate / 1e9, 1), "peak": round(VALU_PEAK_INSTS / 1e9, 1),
            "unit": "G wave-instructions/s", "frac": round(rate / VALU_PEAK_INSTS, 4)}


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
    ("gs::render_bwd_whole_kernel", "render_bwd"),
    ("gs::preprocess_bwd_kernel", "preprocess_bwd"),
    ("gs::bucket_depth_keys_kernel", "depth_sort"),
    ("gs::bucket_count_kernel", "bucket"),
    ("gs::bucket_scatter_kernel", "bucket"),
    ("gs::bucket_", "bucket_tiles"),
)

# Configurations whose profiled forwards bin by buckets: their radix-sort
# kernels are the depth sort (the bucketed binning sorts no pairs), and the
# scan kernels also run the bucket counts' scan.
BUCKET_CONFIGS = (3,)


def _stage_of(kernel_name: str, config: int = 2):
    name = kernel_name.replace("void ", "", 1)
    if config in BUCKET_CONFIGS and name.startswith("gs_sort::"):
        return "depth_sort"
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


def _pmc_commands(config: int) -> list[str]:
    c = f"c{config}"
    cfg = "" if config == 2 else f"--config {config} "
    run = f"python3 $R/bench.py {cfg}--steps 3 --warmup 1 --no-cpu-baseline --no-stage-timing"
    return [
        _PROFILE_PREAMBLE,
        f"#   rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/gpurun_out/pmc_{c} -o fetch -- \\",
        f"#       {run} > $R/gpurun_out/pmc_{c}/fetch.json 2> $R/gpurun_out/pmc_{c}/fetch.err",
        f"#   rocprofv3 --pmc WRITE_SIZE --output-format csv -d $R/gpurun_out/pmc_{c} -o write -- \\",
        f"#       {run} > $R/gpurun_out/pmc_{c}/write.json 2> $R/gpurun_out/pmc_{c}/write.err",
        f"#   python3 bench.py --pmc-summary gpurun_out/pmc_{c}/fetch_counter_collection.csv \\",
        f"#       gpurun_out/pmc_{c}/write_counter_collection.csv profiles/traffic_config{config}.txt \\",
        f"#       gpurun_out/pmc_{c}/fetch.err" + ("" if config == 2 else f" --profile-config {config}"),
    ]


def _sq_commands(config: int) -> list[str]:
    c = f"c{config}"
    cfg = "" if config == 2 else f"--config {config} "
    return [
        _PROFILE_PREAMBLE,
        "#   rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_INSTS_LDS SQ_ACTIVE_INST_LDS \\",
        f"#       SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_BUSY_CYCLES --output-format csv -d $R/gpurun_out/sq_{c} -o sq -- \\",
        f"#       python3 $R/bench.py {cfg}--steps 3 --warmup 1 --no-cpu-baseline --no-stage-timing \\",
        f"#       > $R/gpurun_out/sq_{c}/sq.json 2> $R/gpurun_out/sq_{c}/sq.err",
        f"#   python3 bench.py --sq-summary gpurun_out/sq_{c}/sq_counter_collection.csv "
        f"profiles/sq_counters_config{config}.txt gpurun_out/sq_{c}/sq.err"
        + ("" if config == 2 else f" --profile-config {config}"),
    ]


def summarize_pmc(fetch_csv: str, write_csv: str, out_path: str, bench_log: str | None = None,
                  copy_bytes: int = 1 << 30, config: int = 2) -> None:
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
            stage = _stage_of(r["Kernel_Name"], config)
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
        f"# HBM traffic per launch of each stage (bytes), {CONFIG_TITLES[config]}, from rocprofv3 --pmc",
        f"# FETCH_SIZE scale {f_scale:.2f} B/unit, WRITE_SIZE scale {w_scale:.2f} B/unit "
        f"(calibration copy of {copy_bytes} B read + {copy_bytes} B written read "
        f"{fetch_copy:.0f} / {write_copy:.0f} units)",
        f"# iterations averaged: {iters} (fetch run), {iters_w} (write run)",
        *profiled_run_line(bench_log),
        "# commands:",
        *_pmc_commands(config),
        "# format: '<stage>: <bytes per launch> fetch <bytes> write <bytes>' (bench.py reads the first number)",
    ]
    for stage in sorted(set(fetch) | set(write)):
        fb = fetch.get(stage, 0.0) * f_scale / max(iters, 1)
        wb = write.get(stage, 0.0) * w_scale / max(iters_w, 1)
        lines.append(f"{stage}: {fb + wb:.0f} fetch {fb:.0f} write {wb:.0f}")
    Path(out_path).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def summarize_sq(counter_csv: str, out_path: str, bench_log: str | None = None, config: int = 2) -> None:
    """Per-kernel means per dispatch of the SQ counters in one rocprofv3 --pmc
    counter_collection.csv, with the LDS bank-conflict rate in conflict cycles
    per LDS access cycle, SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE -
    SQ_LDS_BANK_CONFLICT) (rocprofv3's LdsBankConflict), and VALU
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
    lines = [f"# SQ counters per kernel, {CONFIG_TITLES[config]}, one MI355X",
             *profiled_run_line(bench_log),
             "# commands:", *_sq_commands(config),
             "# lds_conflict_rate = SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT) "
             "(conflict cycles per LDS access cycle)",
             "# SQ counters per dispatch (mean); columns: kernel, dispatches, "
             + ", ".join(counters) + ", lds_conflict_rate, valu_insts_per_wave"]
    for k in sorted(per):
        n = len(dispatches[k])
        d = {c: per[k][c] / n for c in counters}
        conflict = d.get("SQ_LDS_BANK_CONFLICT", 0.0)
        access = d.get("SQ_LDS_IDX_ACTIVE", 0.0) - conflict
        rate = conflict / access if access > 0 else 0.0
        waves = d.get("SQ_WAVES", 0.0)
        vpw = d.get("SQ_INSTS_VALU", 0.0) / waves if waves else 0.0
        lines.append(f"{k} {n} " + " ".join(f"{d[c]:.4g}" for c in counters) + f" {rate:.4f} {vpw:.1f}")
    Path(out_path).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


CONFIG_TITLES = {
    0: "config 0 (10k Gaussians, 256x256, SH0, forward only)",
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
             *profiled_run_line(bench_err),
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


def signature(tensor) -> dict:
    """numel, finite count, sum, sum of |x| and max |x| of a device tensor, in the
    tensor's own precision (the reference microbenchmark's `_signature`,
    benchmarks/rasterizer_microbench.py:44-53)."""
    import torch

    value = tensor.detach()
    return {"numel": value.numel(), "finite": int(torch.isfinite(value).sum().item()),
            "sum": float(value.sum().item()), "abs_sum": float(value.abs().sum().item()),
            "max_abs": float(value.abs().max().item()) if value.numel() else 0.0}


def signature_difference(left: dict, right: dict) -> dict:
    """Largest absolute and relative difference between two runs' signatures
    over the sum, abs_sum and max_abs fields, relative to max(|right|, 1); inf
    when a tensor's size or finite count differs (the reference's
    `_difference`, benchmarks/rasterizer_microbench.py:145-163)."""
    largest_abs = largest_rel = 0.0
    for name, a in left.items():
        b = right[name]
        if a["numel"] != b["numel"] or a["finite"] != a["numel"] or b["finite"] != b["numel"]:
            return {"max_abs": math.inf, "max_rel": math.inf}
        for field in ("sum", "abs_sum", "max_abs"):
            delta = abs(a[field] - b[field])
            largest_abs = max(largest_abs, delta)
            largest_rel = max(largest_rel, delta / max(abs(b[field]), 1.0))
    return {"max_abs": largest_abs, "max_rel": largest_rel}


def median(values):
    v = sorted(values)
    n = len(v)
    if n == 0:
        return None
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def host_cpu_info() -> dict:
    """The host's CPUs as this process sees them: os.cpu_count(), the CPUs it may
    run on, the cgroup quota, the usable count (the smaller of those two) and
    the model name."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        text = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if text and text[0] != "max":
            quota = float(text[0]) / float(text[1])
    except (OSError, ValueError, IndexError):
        pass
    usable = affinity if quota is None else max(1, min(affinity, math.floor(quota)))
    return {"os_cpu_count": os.cpu_count(), "affinity_cpus": affinity, "cgroup_cpu_quota": quota,
            "usable_cpus": usable, "cpu_model": model}


def cpu_baseline_and_parity(scene, grads, gpu: dict, flow: bool, top_k: int, reps: int = 3,
                            backward: bool = True) -> tuple[dict, dict]:
    """The CPU baseline and the parity check of the iteration-0 view, both from the C oracle.

    Baseline: one untimed warm-up fwd+bwd (the forward alone for a forward-only
    workload) of the same scene, then `reps` timed ones on all usable host CPUs
    and one on a single thread.  Parity: the
    warm-up's forward is the checker for the GPU's outputs of the same view
    (gpu: images, radii, flow ids and leaf gradients captured after the timed
    region), the gradients to the per-element bound of the oracle (its
    rounding bound B, computed outside the timed runs)."""
    import numpy as np

    import oracle
    from gswarp_amd import configs

    info = host_cpu_info()
    threads = info["usable_cpus"]
    oracle.set_num_threads(threads)
    host = configs.scene_to_numpy(scene)
    gc = grads["color"].detach().cpu().numpy()
    zero = np.zeros((1, *gc.shape[1:]), np.float32)
    gd = zero if flow else grads["depth"].detach().cpu().numpy()
    ga = zero if flow else grads["alpha"].detach().cpu().numpy()

    def run():
        res = oracle.rasterize(host, top_k=top_k)
        if backward:
            oracle.rasterize_backward(host, res, gc, gd, ga, flow_double=flow)
        return res

    ref = run()
    seconds = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        seconds.append(time.perf_counter() - t0)
    oracle.set_num_threads(1)
    t0 = time.perf_counter()
    run()
    one_thread = time.perf_counter() - t0
    oracle.set_num_threads(threads)
    n = host["means3D"].shape[0]
    mean = sum(seconds) / len(seconds)
    baseline = {
        "value": n / mean,
        "unit": "Gaussians/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{'fwd+bwd' if backward else 'forward'} of the iteration-0 view of this workload "
                  f"({n} Gaussians) by the C oracle "
                  f"(oracle/gs_oracle.c, OpenMP): 1 warm-up, mean of {reps} timed runs on {threads} threads "
                  f"({mean:.2f} s), 1 run on 1 thread ({one_thread:.2f} s)",
        "seconds": mean,
        "seconds_per_rep": [round(t, 3) for t in seconds],
        "value_1thread": n / one_thread,
        "seconds_1thread": one_thread,
        **info,
    }

    t0 = time.perf_counter()
    ref_g = oracle.rasterize_backward(host, ref, gc, gd, ga, flow_double=flow, with_bound=True) if backward else None
    rf = ref["fwd"]
    parity = {"view": "iteration 0 (the scene's camera)",
              "bar": "radii (and flow top-K ids) equal; colour, depth, alpha within 1e-4"
                     + ("; each gradient element within 1e-3 |e| + 1e-5 + 2 B (B: the oracle's bound on its "
                        "fp32 rounding)" if backward else ""),
              "radii_equal": bool(np.array_equal(gpu["radii"], ref["pre"]["radii"]))}
    ok = parity["radii_equal"]
    for key in ("color", "depth", "alpha"):
        err = float(np.abs(gpu[key] - rf[key]).max())
        parity[f"{key}_max_abs_err"] = err
        ok = ok and err <= 1e-4
    if flow:
        parity["topk_ids_equal"] = bool(np.array_equal(gpu["ids"], rf["gs_per_pixel"]))
        ok = ok and parity["topk_ids_equal"]
    grad_report = {}
    for name in ("means3D", "means2D", "opacities", "scales", "rotations", "sh") if backward else ():
        e = ref_g[name].astype(np.float64)
        a = gpu["grads"][name].reshape(e.shape).astype(np.float64)
        diff = np.abs(a - e)
        plain = 1e-3 * np.abs(e) + 1e-5
        tol = plain + 2.0 * ref_g["bound"][name]
        failures = int((diff > tol).sum())
        grad_report[name] = {"failures": failures, "worst_ratio": round(float((diff / tol).max()), 4),
                             "outside_plain_bar": int((diff > plain).sum()), "elements": int(e.size)}
        ok = ok and failures == 0
    if backward:
        parity["gradients"] = grad_report
    parity["ok"] = bool(ok)
    parity["check_seconds"] = round(time.perf_counter() - t0, 2)
    return baseline, parity


# The reference's published full forward + backward runs with precomputed RGB
# (docs/rasterizer.md:315, Warp on one RTX 5090): Gaussians, image side, ms,
# peak MiB, repeated-output max abs difference.
REFERENCE_MICROBENCH = ((262_144, 384, 2.215, 85.8, 5.59e-9), (1_048_576, 640, 4.733, 345.5, 5.96e-8))


def reference_microbench(warmups: int = 20, repeats: int = 100, seed: int = 20260710) -> dict:
    """Context only (not the headline): the reference microbenchmark's workload
    (benchmarks/rasterizer_microbench.py:57-128) at the two sizes it publishes
    figures for: means x, y ~ U[-0.65, 0.65], z ~ U[2, 3], precomputed RGB ~
    U[0, 1), opacity ~ U[0.1, 0.9], scales ~ U[0.025, 0.06], identity
    rotations, identity view and projection, tan(fov) = 1, background
    (0.05, 0.15, 0.25), SH degree 0, warp_depth_stable_tile binning; drawn
    from a device generator seeded seed + count in that order; the loss
    color^2 mean + alpha mean + 0.01 depth mean + 1e-4 (proj_2D^2 mean +
    conic_2D sum + conic_2D_inv sum).  Timing follows the reference: events
    around `repeats` back-to-back steps after `warmups` (lines 166-186), with
    the signature repeatability of two collected steps (lines 172-175) and
    torch's peak allocation over the timed steps."""
    import torch

    from gswarp_amd.rasterizer import GaussianRasterizationSettings, rasterize_gaussians

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    records = []
    for count, side, ref_ms, ref_mib, ref_rep in REFERENCE_MICROBENCH:
        g = torch.Generator(device=device).manual_seed(seed + count)
        means3D = torch.empty((count, 3), dtype=torch.float32, device=device)
        means3D[:, :2].uniform_(-0.65, 0.65, generator=g)
        means3D[:, 2].uniform_(2.0, 3.0, generator=g)
        colors = torch.rand((count, 3), dtype=torch.float32, device=device, generator=g)
        opacities = torch.empty((count, 1), dtype=torch.float32, device=device).uniform_(0.1, 0.9, generator=g)
        scales = torch.empty((count, 3), dtype=torch.float32, device=device).uniform_(0.025, 0.06, generator=g)
        rotations = torch.zeros((count, 4), dtype=torch.float32, device=device)
        rotations[:, 0] = 1.0
        leaves = {"means3D": means3D, "means2D": torch.zeros((count, 3), dtype=torch.float32, device=device),
                  "colors_precomp": colors, "opacities": opacities, "scales": scales, "rotations": rotations}
        for t in leaves.values():
            t.requires_grad_(True)
        empty = torch.empty((0,), dtype=torch.float32, device=device)
        settings = GaussianRasterizationSettings(
            image_height=side, image_width=side, tanfovx=1.0, tanfovy=1.0,
            bg=torch.tensor((0.05, 0.15, 0.25), dtype=torch.float32, device=device), scale_modifier=1.0,
            viewmatrix=torch.eye(4, dtype=torch.float32, device=device),
            projmatrix=torch.eye(4, dtype=torch.float32, device=device), sh_degree=0,
            campos=torch.zeros(3, dtype=torch.float32, device=device), prefiltered=False, auto_tune=False,
            auto_tune_verbose=False, binning_sort_mode="warp_depth_stable_tile")

        def run(collect: bool):
            for t in leaves.values():
                t.grad = None
            color, radii, meta = rasterize_gaussians(
                leaves["means3D"], leaves["means2D"], empty, leaves["colors_precomp"], leaves["opacities"],
                leaves["scales"], leaves["rotations"], empty, settings)
            loss = (color.square().mean() + meta.alpha.mean() + 0.01 * meta.depth.mean()
                    + 1.0e-4 * (meta.proj_2D.square().mean() + meta.conic_2D.sum() + meta.conic_2D_inv.sum()))
            loss.backward()
            if not collect:
                return None
            tensors = {"loss": loss.reshape(1), "color": color, "depth": meta.depth, "alpha": meta.alpha,
                       "proj_2D": meta.proj_2D, "conic_2D": meta.conic_2D, "conic_2D_inv": meta.conic_2D_inv}
            tensors.update({f"grad.{k}": v.grad for k, v in leaves.items()})
            return int((radii > 0).sum().item()), {k: signature(v) for k, v in tensors.items()}

        for _ in range(warmups):
            run(False)
        torch.cuda.synchronize()
        visible, first = run(True)
        _, second = run(True)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(device)
        host = []
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(repeats):
            h0 = time.perf_counter()
            run(False)
            host.append(time.perf_counter() - h0)
        end.record()
        end.synchronize()
        ms = start.elapsed_time(end) / repeats
        peak = torch.cuda.max_memory_allocated(device) / 2.0 ** 20
        rep = signature_difference(second, first)
        records.append({"gaussians": count, "image": f"{side}x{side}", "visible_gaussians": visible,
                        "fwd_bwd_ms": round(ms, 4), "host_step_median_ms": round(1e3 * median(host), 4),
                        "peak_allocated_mib": round(peak, 1), "repeatability": rep,
                        "reference_rtx5090_warp": {"fwd_bwd_ms": ref_ms, "peak_allocated_mib": ref_mib,
                                                   "repeat_max_abs": ref_rep}})
        log(f"[bench] reference microbench {count} Gaussians {side}x{side}: {ms:.3f} ms fwd+bwd "
            f"(reference 5090/Warp {ref_ms} ms), {visible} visible, peak {peak:.1f} MiB, "
            f"repeat max abs {rep['max_abs']:.3g}")
        del leaves, means3D, colors, opacities, scales, rotations
        torch.cuda.empty_cache()
    return {"mode": "reference microbenchmark workloads (context only, not the headline metric)",
            "warmups": warmups, "repeats": repeats, "seed": seed, "dtype": "f32",
            "data": "synthetic, the reference microbenchmark's distributions (device generator)",
            "records": records}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--config", type=int, default=2, choices=(0, 1, 2, 3, 4))
    parser.add_argument("--count", type=int, default=None, help="override the Gaussian count")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-stage-timing", action="store_true")
    parser.add_argument("--sort-mode", default=None, choices=("warp_depth_stable_tile", "warp_radix", "torch"),
                        help="binning sort mode (default: the API default, warp_depth_stable_tile)")
    parser.add_argument("--pmc-summary", nargs="+", metavar="PATH",
                        help="FETCH_CSV WRITE_CSV OUT [BENCH_ERR]: summarise two rocprofv3 --pmc runs "
                             "(FETCH_SIZE, WRITE_SIZE) into OUT and exit")
    parser.add_argument("--sq-summary", nargs="+", metavar="PATH",
                        help="COUNTER_CSV OUT [BENCH_ERR]: summarise one rocprofv3 --pmc run of SQ counters "
                             "into OUT and exit")
    parser.add_argument("--profile-config", type=int, default=2, choices=(0, 1, 2, 3, 4),
                        help="configuration a --stats-summary, --pmc-summary or --sq-summary run profiled")
    parser.add_argument("--reference-microbench", action="store_true",
                        help="context only: time the reference microbenchmark's two published precomputed-RGB "
                             "workloads (256K at 384x384, 1024K at 640x640) and print their JSON line")
    parser.add_argument("--stats-summary", nargs="+", metavar="PATH",
                        help="KERNEL_STATS_CSV OUT [BENCH_ERR]: summarise one rocprofv3 --kernel-trace --stats "
                             "run into OUT and exit")
    args = parser.parse_args()
    if args.reference_microbench:
        print(json.dumps(reference_microbench()), flush=True)
        return 0
    if args.stats_summary:
        summarize_stats(*args.stats_summary, config=args.profile_config)
        return 0
    if args.sq_summary:
        summarize_sq(*args.sq_summary, config=args.profile_config)
        return 0
    if args.pmc_summary:
        summarize_pmc(*args.pmc_summary, config=args.profile_config)
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
    if args.config in BUCKET_CONFIGS:
        # The default mode prepares the bucketed binning after a forward with more
        # than 4 pairs per Gaussian on the device; here every forward, the first
        # warm-up one included, takes that steady-state dataflow, so the profiled
        # launches (which include the warm-up) are all of one dataflow.
        _pipeline.BUCKET_SIZING = "always"
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
    sh_coeffs = (spec.sh_degree + 1) ** 2
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

    backward = spec.backward
    host_times = []  # (forward, backward) host seconds of each timed step

    def step(i: int, timed: bool, events: bool = False):
        for t in (*leaves.values(), means2D):
            t.grad = None
        rast = (FlowRasterizer if flow else GaussianRasterizer)(settings[i])
        e0 = e1 = e2 = None
        if events:
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record()
        h0 = time.perf_counter()
        if backward:
            out = rast(leaves["means3D"], means2D, leaves["opacities"], shs=leaves["shs"], scales=leaves["scales"],
                       rotations=leaves["rotations"])
        else:
            with torch.no_grad():
                out = rast(leaves["means3D"], means2D, leaves["opacities"], shs=leaves["shs"],
                           scales=leaves["scales"], rotations=leaves["rotations"])
        h1 = time.perf_counter()
        if events:
            e1.record()
        if flow:
            outputs, upstream = [out[0], out[9]], [grads["color"], grads["x_mu"]]
            images = {"color": out[0], "radii": out[1], "depth": out[2], "alpha": out[3], "ids": out[7]}
        else:
            color, radii, meta = out
            outputs, upstream = [color, meta.depth, meta.alpha], [grads["color"], grads["depth"], grads["alpha"]]
            images = {"color": color, "radii": radii, "depth": meta.depth, "alpha": meta.alpha}
        h2 = time.perf_counter()
        if backward:
            torch.autograd.backward(outputs, upstream)
        h3 = time.perf_counter()
        if events:
            e2.record()
            step_events.append((e0, e1, e2))
        if timed:
            host_times.append((h1 - h0, h3 - h2))
        return images

    def capture(i: int) -> dict:
        """Outputs and leaf gradients of one untimed step, on the host, with the
        reference microbenchmark's signatures (numel, finite count, sum, sum of
        absolute values, largest absolute value) of each, taken on the device
        in fp32 as it takes them (rasterizer_microbench.py:44-53)."""
        images = step(i, False)
        torch.cuda.synchronize()
        out = {k: v.detach().cpu().numpy() for k, v in images.items()}
        tensors = {f"output.{k}": images[k] for k in ("color", "depth", "alpha")}
        if backward:
            out["grads"] = {k: leaves[k].grad.detach().cpu().numpy() for k in ("means3D", "scales", "rotations",
                                                                             "opacities")}
            out["grads"]["sh"] = leaves["shs"].grad.detach().cpu().numpy()
            out["grads"]["means2D"] = means2D.grad.detach().cpu().numpy()
            tensors.update({f"grad.{k}": leaves[k].grad for k in leaves})
            tensors["grad.means2D"] = means2D.grad
        out["signature"] = {k: signature(v) for k, v in tensors.items()}
        return out

    for i in range(args.warmup):
        step(i, False)
    torch.cuda.synchronize()
    timer.notes.clear()  # the warm-up cameras are not the timed ones
    torch.cuda.reset_peak_memory_stats(device)
    # Headline: the K timed steps run uninstrumented (no events on the
    # stream; only the host clock per call).
    t_start = time.perf_counter()
    for i in range(args.warmup, total_steps):
        step(i, True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    peak_bytes = torch.cuda.max_memory_allocated(device)
    # The forward / backward split: the same K cameras again with HIP events
    # around forward and backward (three per step, not in the headline).
    for i in range(args.warmup, total_steps):
        step(i, False, events=True)
    torch.cuda.synchronize()
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
    visited = [visited_pairs(nc, W, H) for nc in timer.notes.pop("n_contrib", [])]
    R_visited = sum(visited) / len(visited) if visited else None
    stopped = [early_stop_share(a, W, H, flow) for a in timer.notes.pop("alpha", [])]
    early_share = sum(stopped) / len(stopped) if stopped else 0.0
    # Run-to-run repeatability of the iteration-0 view (the float atomics of the
    # backward add in an unspecified order), and its outputs for the parity check.
    first = capture(0)
    second = capture(0)
    repeat = {"images_max_abs_diff": max(float(abs(first[k] - second[k]).max()) for k in ("color", "depth", "alpha"))}
    if backward:
        repeat["grads_max_abs_diff"] = max(float(abs(first["grads"][k] - second["grads"][k]).max())
                                           for k in first["grads"])
        repeat["grads_max_rel_diff"] = max(float((abs(first["grads"][k] - second["grads"][k])
                                                  / (abs(first["grads"][k]) + 1e-30)).max()) for k in first["grads"])
    # the reference's repeatability figure: the same view twice, compared through
    # per-tensor signatures (sum, abs_sum, max_abs) of the images and gradients
    repeat["signature"] = signature_difference(second["signature"], first["signature"])
    log(f"[bench] run-to-run: images {repeat['images_max_abs_diff']:.3g}"
        + (f", gradients {repeat['grads_max_abs_diff']:.3g} max abs" if backward else "")
        + f"; signatures {repeat['signature']['max_abs']:.3g} max abs, {repeat['signature']['max_rel']:.3g} max rel"
        + f"; peak allocated {peak_bytes / 2**30:.2f} GiB")

    ms_per_step = 1000.0 * elapsed / args.steps
    fwd_list = [a.elapsed_time(b) for a, b, _ in step_events]
    bwd_list = [b.elapsed_time(c) for _, b, c in step_events]
    fwd_ms = sum(fwd_list) / len(fwd_list)
    bwd_ms = sum(bwd_list) / len(bwd_list) if backward else None
    # Host time per call (Python dispatch plus, in the forward, the wait for the
    # pair count), as the reference reports a host median beside the GPU time
    # (docs/rasterizer.md:313).  The backward returns once its kernels are queued.
    host = {"fwd_median_ms": round(1e3 * median([h[0] for h in host_times]), 4),
            "bwd_median_ms": round(1e3 * median([h[1] for h in host_times]), 4) if backward else None,
            "gpu_fwd_median_ms": round(median(fwd_list), 4),
            "gpu_bwd_median_ms": round(median(bwd_list), 4) if backward else None}
    stage_ms = timer.mean_ms(args.steps) if not args.no_stage_timing else {}
    passes = timer.notes.get("sort_passes", [])
    Rs = timer.notes.get("num_rendered", [])
    R = sum(Rs) / len(Rs) if Rs else float("nan")
    log(f"[bench] {ms_per_step:.3f} ms/step (fwd {fwd_ms:.3f} ms"
        + (f", bwd {bwd_ms:.3f} ms" if backward else ", forward only") + f"), mean R={R:.0f}")
    log(f"[bench] host medians: fwd {host['fwd_median_ms']:.3f} ms"
        + (f", bwd {host['bwd_median_ms']:.3f} ms" if backward else ""))

    roofline = None
    binning_sort = None
    stages = {}
    if stage_ms and Rs:
        dataflows = set(timer.notes.get("binning_dataflow", []))
        flow_k = _runtime.get_flow_topk() if flow else 0
        Es, Vs = timer.notes.get("bucket_entries", []), timer.notes.get("bucket_valid", [])
        E_mean = sum(Es) / len(Es) if Es else 0.0
        V_mean = sum(Vs) / len(Vs) if Vs else 0.0
        flow_of = ("warp_radix" if dataflows == {"packed_key"} else "buckets" if dataflows == {"buckets"}
                   else sort_mode)
        # the two-pass sizing scan reads the cover words; the one-pass scan does not
        sized_scan = "buckets" in dataflows and not _pipeline.SCAN_ONEPASS
        algo = algorithmic_bytes(N, R, P, T, flow_of, flow_k, E_mean, V_mean, sized_scan, sh_coeffs)
        # The formula counts every pair once per stage.  The backward reads each tile's
        # list only from its largest n_contrib (visited pairs), and the forward stops a
        # slice once all its pixels have stopped: where that happens the formula does not
        # describe the work, and its fraction is not given (the visited figures are).
        visited_algo = (algorithmic_bytes(N, R_visited, P, T, "warp_radix", flow_k, sh_coeffs=sh_coeffs)
                        if R_visited else {})
        formula_applies = {"render": early_share <= 0.01,
                           "render_bwd": R_visited is None or R_visited >= 0.5 * R}
        for name, ms in sorted(stage_ms.items(), key=lambda kv: -kv[1]):
            gbps = algo[name] / (ms * 1e-3) / 1e9 if name in algo else None
            entry = {"ms": round(ms, 4), "algorithmic_bytes": algo.get(name),
                     "achieved_GBps": None if gbps is None else round(gbps, 1),
                     "hbm_frac": None if gbps is None else round(gbps / HBM_PEAK_GBPS, 4)}
            if name == "render_bwd" and R_visited:
                vg = visited_algo[name] / (ms * 1e-3) / 1e9
                entry.update(visited_pairs=round(R_visited), visited_bytes=visited_algo[name],
                             visited_GBps=round(vg, 1), visited_hbm_frac=round(vg / HBM_PEAK_GBPS, 4))
            if name == "render":
                entry["early_stopped_slice_share"] = round(early_share, 4)
            if not formula_applies.get(name, True):
                entry["hbm_frac"] = entry["achieved_GBps"] = None
            traffic = read_traffic(name, args.config)
            if traffic is not None:
                entry["counter_bytes"] = traffic
                entry["counter_hbm_frac"] = round(traffic / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)
            if name == "render_bwd":  # VALU-issue-bound
                valu = valu_issue(name, ms, args.config)
                if valu is not None:
                    entry["valu_issue"] = valu
            stages[name] = entry
            shown = entry.get("visited_GBps") if entry["hbm_frac"] is None else gbps
            note = "" if entry["hbm_frac"] is not None else (" (visited pairs)" if shown else " (formula n/a)")
            log(f"[bench]   {name:15s} {ms:8.4f} ms" + ("" if shown is None else f"  {shown:8.1f} GB/s") + note)
        sort_names = [n for n in ("depth_sort", "sort", "bucket", "bucket_tiles") if n in stage_ms]
        sort_ms = sum(stage_ms[n] for n in sort_names)
        sort_bytes = sum(algo[n] for n in sort_names)
        binning_sort = {"mode": sort_mode, "stages": sort_names, "ms": round(sort_ms, 4),
                        "algorithmic_bytes": sort_bytes,
                        "hbm_frac": round(sort_bytes / (sort_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        counter = [stages[n].get("counter_bytes") for n in sort_names]
        if all(c is not None for c in counter):
            # the bytes the sort kernels actually move (PMC), next to the formula's
            binning_sort["counter_bytes"] = sum(counter)
            binning_sort["counter_hbm_frac"] = round(sum(counter) / (sort_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)
        binning_sort["dataflow"] = sorted(dataflows)
        log(f"[bench]   binning sort ({sort_mode}, {'/'.join(sorted(dataflows))}) {sort_ms:.4f} ms  "
            f"{binning_sort['hbm_frac'] * 100:.1f}% of HBM peak (formula bytes)")
        dominant = max((n for n in stage_ms if n in algo), key=lambda n: stage_ms[n])
        achieved = algo[dominant] / (stage_ms[dominant] * 1e-3) / 1e9
        roofline = {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 5),
                    "traffic": read_traffic(dominant, args.config),
                    "algorithmic_bytes_per_launch": algo[dominant]}
        if roofline["traffic"] is not None:
            # the counters come from a separate profiled run of the same workload: its R
            roofline["traffic_source"] = profile_provenance("traffic", args.config)
        if "visited_GBps" in stages[dominant]:
            roofline["visited_achieved"] = stages[dominant]["visited_GBps"]
            roofline["visited_frac"] = stages[dominant]["visited_hbm_frac"]
        if "valu_issue" in stages[dominant]:
            # the bound that binds: VALU issue (the bytes' fraction is reported as the contract asks)
            roofline["valu_issue"] = stages[dominant]["valu_issue"]
    copy_gbps = measure_copy_bandwidth(device)
    log(f"[bench] device copy bandwidth {copy_gbps:.0f} GB/s")
    if roofline is not None:
        roofline["copy_GBps"] = round(copy_gbps, 1)
    if not Rs:
        iteration_bytes = None
    elif backward:  # the SH3, depth-on fwd+bwd headline formula
        iteration_bytes = 1056.0 * N + 252.0 * R + 52.0 * P + 24.0 * T
    else:  # forward only: preprocess + SH + scan + duplicate, keys, sort, ranges, render
        iteration_bytes = ((112.0 + 36.0 + 12.0 * sh_coeffs + 8.0 + 44.0) * N
                           + (12.0 + 24.0 * sort_passes(T) + 8.0 + 44.0) * R + 24.0 * P + 16.0 * T)

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
        "fwd_bwd_ms": ms_per_step if backward else None,
        "host_ms": host,
        "hbm_copy_GBps": round(copy_gbps, 1),
        "iteration_hbm_frac": None if iteration_bytes is None else
        round(iteration_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 5),
        "stages": stages,
        "binning_sort": binning_sort,
        "roofline": roofline,
        "peak_allocated_bytes": peak_bytes,
        "run_to_run": repeat,
        # figures read from the committed profiles (counter_bytes, roofline.traffic,
        # valu_issue) were measured in these profiled runs, whose mean R may differ
        "profile_sources": {kind: profile_provenance(kind, args.config)
                            for kind in ("traffic", "sq_counters", "kernel_stats")},
        "cpu_baseline": None,
        "parity": None,
    }
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline and parity check (oracle) ...")
        # the scene carries the iteration-0 camera
        top_k = _runtime.get_flow_topk() if flow else 0
        baseline, parity = cpu_baseline_and_parity(scene, grads, first, flow, top_k, backward=backward)
        result["cpu_baseline"], result["parity"] = baseline, parity
        log(f"[bench] CPU baseline {baseline['seconds']:.2f} s on {baseline['cores']} threads, "
            f"{baseline['seconds_1thread']:.2f} s on 1; parity {'ok' if parity['ok'] else 'FAILED'}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
