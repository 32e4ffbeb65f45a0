"""Per-tile cost and active-lane diagnostics of the compositors.

Runs one forward + backward of a workload through ``libgabor_hip_diag.so``
(the same sources built with ``-DGS_DIAGNOSTICS``; build it with
``python -m diff_gabor_splatting_amd.build --diagnostics``) and reports:

* per tile: the point-list length, the records replayed by the backward
  (taken by some pixel), and the wall-clock time of the tile's workgroup in
  the forward and in the backward, as log2 histograms and percentiles;
* per compositor launch: its span (first tile begun to last tile ended), the
  time by which 90% and 99% of tiles had ended, the longest tile, and the
  tail, the time during which fewer than half the peak number of tiles were
  in flight;
* the backward's histogram of taking lanes per processed (record, wave): of
  the 64 lanes of a wave that processes a record (some lane takes it), how
  many take it. The adjoint runs on all 64 lanes either way.

    python -m diff_gabor_splatting_amd.diagnostics --workload config4 --json out.json

Workloads: ``config0`` .. ``config4`` (the benchmark configs, ``workloads.py``)
and ``harness-classic`` / ``harness-neural`` (the benchmark harness's default
scene, all images in one dense call). The per-(record, wave) counting adds
instructions to every processed pair, so times here run above the product
library's (by up to about 15% in the backward); use ``bench.py`` for timing.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import sys
from pathlib import Path

import torch

from . import _native
from .build import DIAGNOSTICS_LIBRARY


def log2_histogram(values: torch.Tensor) -> dict[str, int]:
    """Counts of values in [0, 1), [1, 2), [2, 4), ... keyed by the bin's lower edge."""
    values = values.double().clamp_min(0)
    bins = torch.where(values < 1, torch.zeros_like(values),
                       torch.floor(torch.log2(values.clamp_min(1))) + 1).long()
    counts = torch.bincount(bins)
    return {str(0 if b == 0 else 2 ** (b - 1)): int(c) for b, c in enumerate(counts.tolist())
            if c}


def percentiles(values: torch.Tensor, points=(50, 90, 99, 100)) -> dict[str, float]:
    values = values.double()
    return {f"p{p}": float(torch.quantile(values, p / 100)) for p in points}


def launch_profile(span: torch.Tensor, khz: int) -> dict:
    """Timing statistics of one compositor launch from its tiles' [begin, end]
    wall-clock stamps (ticks at ``khz`` kHz)."""
    begin, end = span[:, 0], span[:, 1]
    t0 = int(begin.min())
    scale = 1000.0 / khz  # microseconds per tick

    def us(ticks):
        return float(ticks) * scale

    duration = (end - begin).double() * scale
    finish = torch.sort(end - t0).values.double() * scale
    # Tiles in flight over time: +1 at each begin, -1 at each end.
    stamps = torch.cat((begin, end)) - t0
    steps = torch.cat((torch.ones_like(begin), -torch.ones_like(end)))
    order = torch.argsort(stamps * 2 + (steps > 0).long(), stable=True)  # ends before begins
    stamps, steps = stamps[order], steps[order]
    flight = torch.cumsum(steps, 0)
    peak = int(flight.max())
    gaps = torch.diff(stamps, append=stamps[-1:]).double() * scale
    tail = float(gaps[flight < peak / 2].sum())
    longest = int(torch.argmax(duration))
    return {
        "span_us": us(int(end.max()) - t0),
        "ended_90pct_us": float(finish[int(0.9 * (finish.numel() - 1))]),
        "ended_99pct_us": float(finish[int(0.99 * (finish.numel() - 1))]),
        "peak_tiles_in_flight": peak,
        "tail_us_below_half_peak": tail,
        "longest_tile_us": float(duration[longest]),
        "longest_tile_began_us": us(int(begin[longest]) - t0),
        "tile_us": percentiles(duration),
        "tile_us_sum": float(duration.sum()),
        "tile_us_log2_histogram": log2_histogram(duration),
    }


def lane_summary(hist: list[int]) -> dict:
    pairs = sum(hist)
    mean = sum(i * h for i, h in enumerate(hist)) / max(pairs, 1)

    def share(upto):
        return sum(hist[1:upto + 1]) / max(pairs, 1)

    return {"record_wave_pairs": pairs, "mean_taking_lanes": mean,
            "share_at_most_8": share(8), "share_at_most_16": share(16),
            "share_at_most_32": share(32), "share_all_64": hist[64] / max(pairs, 1),
            "histogram": hist}


def walk_summary(visits: int, forward_samples: int, lanes: dict) -> dict:
    """(pixel, record) counts of one render: the forward's visits (every list
    record up to the one that stops a pixel, or to the end of its list), the
    samples the forward evaluated in lockstep ((record, wave) pairs times 64
    lanes) and the backward's (its processed pairs times 64, of which the
    taking lanes are the useful share)."""
    hist = lanes["histogram"]
    return {"forward_pixel_record_visits": int(visits),
            "forward_samples_evaluated": int(forward_samples),
            "backward_samples_evaluated": 64 * int(lanes["record_wave_pairs"]),
            "backward_samples_taken": int(sum(k * c for k, c in enumerate(hist)))}


def packing_summary(counters) -> dict:
    """The backward's wave steps now (one record per wave step over the 8x8
    quadrant) and under two packings it could use: each 32-lane half (8x4)
    or each 16-lane block (4x4) walking its own records, at best and in
    list order (see gs_diagnostics_set), as counts and as ratios."""
    steps = int(counters[2])

    def ratio(v):
        return round(int(v) / steps, 4) if steps else None

    return {"wave_steps": steps,
            "halves_at_best": int(counters[3]), "blocks_at_best": int(counters[4]),
            "halves_in_order": int(counters[5]), "blocks_in_order": int(counters[6]),
            "ratio_halves_at_best": ratio(counters[3]),
            "ratio_blocks_at_best": ratio(counters[4]),
            "ratio_halves_in_order": ratio(counters[5]),
            "ratio_blocks_in_order": ratio(counters[6])}


def replay_quadrant_bits(lists, counts, ranges) -> int:
    """Processed (record, wave) pairs the replay lists call for: the quadrant
    bits (28..31) set over every tile's replay entries."""
    counts = counts.long()
    total = int(counts.sum())
    if total == 0:
        return 0
    tile_start = ranges[:, 0].long().repeat_interleave(counts)
    within = torch.arange(total, device=counts.device) - torch.repeat_interleave(
        torch.cumsum(counts, 0) - counts, counts)
    entries = lists[tile_start + within, 1].long()
    bits = (entries >> 28) & 15
    return int(sum(((bits >> q) & 1).sum() for q in range(4)))


def workload_step(name: str, device: torch.device):
    """(description, step) for a named workload; step() runs one forward +
    loss + backward."""
    if name.startswith("config"):
        from . import workloads

        index = int(name[len("config"):])
        *_, step = workloads.prepare(index, device, False)
        return workloads.CONFIGS[index]["name"], step
    if name in ("harness-classic", "harness-neural"):
        from . import benchmark_rasterization as harness

        method = name.split("-")[1]
        work, _ = harness.parse_workload(["--skip-validation"])
        scene = harness.synthesize(work, method, device)
        strategy = harness.Fused(work, method, packed=False)
        params = [v for v in scene.values() if v.requires_grad]

        def step():
            for p in params:
                p.grad = None
            harness.objective(strategy.maps(scene)).backward()

        description = (f"harness {method}: {work.num_primitives} primitives, "
                       f"{work.num_scenes}x{work.num_cameras} images of "
                       f"{work.image_width}x{work.image_height}, fused dense")
        return description, step
    raise ValueError(f"unknown workload {name!r}")


def collect(name: str, device: torch.device | None = None) -> dict:
    """Run one step of the workload through the diagnostics library and
    return the report (see the module docstring)."""
    device = device or torch.device("cuda:0")
    if not DIAGNOSTICS_LIBRARY.exists():
        raise ImportError(f"{DIAGNOSTICS_LIBRARY.name} is not built; run "
                          "`python -m diff_gabor_splatting_amd.build --diagnostics`")
    previous = _native.library_path()
    _native.use_library(DIAGNOSTICS_LIBRARY)
    try:
        return _collect(name, device)
    finally:
        # Later calls in this process render through the product library again.
        _native.use_library(previous)


def _collect(name: str, device: torch.device) -> dict:
    available, khz = ctypes.c_int32(), ctypes.c_int32()
    with torch.cuda.device(device):
        _native._check(_native.lib.gs_diagnostics_query(ctypes.byref(available),
                                                        ctypes.byref(khz)))
    if available.value != 1:
        raise RuntimeError(f"{DIAGNOSTICS_LIBRARY} is not a diagnostics build")
    description, step = workload_step(name, device)
    captured = {}
    original = _native.rasterize_forward

    def spy(*args, **kwargs):
        result = original(*args, **kwargs)
        captured["forward"] = result
        return result

    step()  # warm-up, nothing recorded
    torch.cuda.synchronize(device)
    _native.rasterize_forward = spy
    try:
        step()  # sizes the span buffers (tiles) and keeps the forward's lists
        torch.cuda.synchronize(device)
        tiles = captured["forward"][2].shape[0]
        lanes = torch.zeros(65, dtype=torch.int64, device=device)
        # Begins start at all ones and ends at zero: the kernels keep the
        # earliest begin and the latest end of every workgroup of a tile.
        spans = torch.zeros((2, tiles, 2), dtype=torch.int64, device=device)
        spans[..., 0] = -1
        counters = torch.zeros(8, dtype=torch.int64, device=device)
        with torch.cuda.device(device):
            _native._check(_native.lib.gs_diagnostics_set(
                lanes.data_ptr(), spans[0].data_ptr(), spans[1].data_ptr(), tiles,
                counters.data_ptr()))
            try:
                step()
                torch.cuda.synchronize(device)
            finally:
                _native._check(_native.lib.gs_diagnostics_set(None, None, None, 0, None))
    finally:
        _native.rasterize_forward = original
    _, point_list, ranges, _, _, *replay = captured["forward"]
    ranges = ranges.long()
    lengths = (ranges[:, 1] - ranges[:, 0]).clamp_min(0)
    report = {"workload": description, "tiles": tiles, "wall_clock_khz": khz.value,
              "list_length": {**percentiles(lengths), "log2_histogram": log2_histogram(lengths)},
              "intersections": int(point_list.numel())}
    lists = replay[0] if replay else None
    if lists is not None:
        records, counts = lists[0], lists[1]
        report["replayed_records"] = {**percentiles(counts.long()),
                                      "log2_histogram": log2_histogram(counts.long()),
                                      "total": int(counts.long().sum())}
        report["replay_quadrant_bits"] = replay_quadrant_bits(records, counts, ranges)
    spans = spans.cpu()
    for index, kernel in enumerate(("render_forward", "render_backward")):
        if bool((spans[index, :, 0] >= 0).all()):
            report[kernel] = launch_profile(spans[index], khz.value)
    report["backward_taking_lanes"] = lane_summary(lanes.cpu().tolist())
    counters = counters.cpu().tolist()
    report["forward_walk"] = walk_summary(counters[0], counters[1],
                                          report["backward_taking_lanes"])
    report["backward_packing"] = packing_summary(counters)
    return report


def format_report(report: dict) -> str:
    lines = [f"workload: {report['workload']}",
             f"tiles {report['tiles']}, intersections {report['intersections']}"]
    ll = report["list_length"]
    lines.append(f"list length per tile: p50 {ll['p50']:.0f}, p90 {ll['p90']:.0f}, "
                 f"p99 {ll['p99']:.0f}, max {ll['p100']:.0f}; log2 bins {ll['log2_histogram']}")
    if "replayed_records" in report:
        rr = report["replayed_records"]
        lines.append(f"replayed records per tile: p50 {rr['p50']:.0f}, p90 {rr['p90']:.0f}, "
                     f"p99 {rr['p99']:.0f}, max {rr['p100']:.0f}, total {rr['total']}; "
                     f"log2 bins {rr['log2_histogram']}")
    for kernel in ("render_forward", "render_backward"):
        if kernel not in report:
            continue
        k = report[kernel]
        t = k["tile_us"]
        lines.append(
            f"{kernel}: span {k['span_us']:.1f} us; 90% of tiles ended by "
            f"{k['ended_90pct_us']:.1f} us, 99% by {k['ended_99pct_us']:.1f} us; "
            f"tail below half the peak {k['peak_tiles_in_flight']} tiles in flight "
            f"{k['tail_us_below_half_peak']:.1f} us; longest tile {k['longest_tile_us']:.1f} us "
            f"(began at {k['longest_tile_began_us']:.1f} us); tile us p50 {t['p50']:.2f}, "
            f"p90 {t['p90']:.2f}, p99 {t['p99']:.2f}; sum {k['tile_us_sum']:.0f} us")
        lines.append(f"  tile us log2 bins {k['tile_us_log2_histogram']}")
    lanes = report["backward_taking_lanes"]
    lines.append(
        f"backward taking lanes per processed (record, wave): {lanes['record_wave_pairs']} "
        f"pairs, mean {lanes['mean_taking_lanes']:.1f} of 64; <=8 {lanes['share_at_most_8']:.1%}, "
        f"<=16 {lanes['share_at_most_16']:.1%}, <=32 {lanes['share_at_most_32']:.1%}, "
        f"all 64 {lanes['share_all_64']:.1%}")
    hist = lanes["histogram"]
    lines.append("  by taking lanes (1-8, 9-16, ..., 57-64): "
                 + ", ".join(str(sum(hist[1 + 8 * b: 9 + 8 * b])) for b in range(8)))
    if "forward_walk" in report:
        walk = report["forward_walk"]
        lines.append(
            f"(pixel, record) counts: forward visits {walk['forward_pixel_record_visits']}, "
            f"forward samples evaluated {walk['forward_samples_evaluated']}, backward samples "
            f"evaluated {walk['backward_samples_evaluated']} of which taken "
            f"{walk['backward_samples_taken']}")
    if "backward_packing" in report:
        p = report["backward_packing"]
        lines.append(
            f"backward wave steps {p['wave_steps']}; with 8x4 halves walking their own records "
            f"{p['ratio_halves_at_best']} of them at best, {p['ratio_halves_in_order']} in list "
            f"order; with 4x4 blocks {p['ratio_blocks_at_best']} at best, "
            f"{p['ratio_blocks_in_order']} in list order")
    return "\n".join(lines)


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--workload", action="append", required=True,
                        help="config0..config4, harness-classic or harness-neural (repeatable)")
    parser.add_argument("--json", help="also write the reports to this file")
    args = parser.parse_args(argv)
    reports = {}
    for name in args.workload:
        reports[name] = collect(name)
        print(format_report(reports[name]), flush=True)
        torch.cuda.empty_cache()
    if args.json:
        Path(args.json).write_text(json.dumps(reports, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
