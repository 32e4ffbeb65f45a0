"""Benchmark of the HIP Gabor rasterizer: fwd+bwd ms/iter and Mpix/s on one MI355X.

Default workload is BASELINE config 4: classic Gabor, B=1 C=1, N=1M SH-3
surfels drawn from 64 Gaussian clusters, 1920x1080, all nine output maps in
a mean-square loss, forward + backward through the public API. A step is one
forward + loss + backward over inputs already resident in HBM.

Prints ONE JSON line. Besides the driver's contract fields it carries:
  roofline      for the dominant kernel family (largest share of the timed
                region): algorithmic bytes per launch / average launch time,
                both measured in this run (HIP events on the launch stream);
  cpu_baseline  the CPU oracle (torch fp32, autograd backward) timed on this
                host on config 0 at full frame (the designated CPU config),
                next to the GPU's time for the same workload, plus a
                labelled secondary figure on a crop of config 4;
  per_config    ms/step and Mpix/s of the other BASELINE configs, same run;
  graph_replay  a labelled secondary figure: every config's render and
                backward captured once in a HIP graph and replayed, next to
                its eager step (what the host-bound small configs cost
                without Python, autograd and launch overheads);
  kernels       per-family average milliseconds per step.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import torch

from diff_gabor_splatting_amd.timing import collected_collector, paused_collector
from diff_gabor_splatting_amd.workloads import (CAMERA_KEYS, CONFIGS, crop, loss as _loss,
                                                 loss_groups as _loss_groups, make_scene,
                                                 prepare)

HBM_PEAK_GBS = 8000.0
COPY_BYTES = 1 << 30

RECORD_BYTES_CLASSIC = 4 + 8 + 68 + 4 * 18 + 4  # point list, primitive id, geometry, appearance, opacity
REPLAY_ENTRY_BYTES = 8  # replay entry {pair, position | quadrant bits} instead of the point list


def algorithmic_bytes(kind: str, neural: bool, pixels: int, records: int, rows: int,
                      entry_bytes: int = 4) -> int:
    """Compulsory HBM bytes of one compositor launch.

    pixels: output pixels; records: tile-records the kernel walks, each
    gathering its list entry (`entry_bytes`: 4 B of point list, or 8 B of
    replay entry) + primitive id 8 B + geometry 68 B + appearance 4A B +
    opacity 4 B; rows: visible pairs, whose gradient rows (geometry 68 B,
    appearance 4A B, opacity 4 B) the backward writes once. The forward
    writes maps 36 B + state 12 B + contributors 4 B per pixel; the backward
    reads the same 52 B per pixel.
    """
    appearance = 57 if neural else 18
    record = entry_bytes + 8 + 68 + 4 * appearance + 4
    total = pixels * 52 + records * record
    if kind == "render_backward":
        total += rows * (68 + 4 * appearance + 4)
    return int(total)


def time_steps(step, steps: int, warmup: int, min_ms: float = 0.0,
               pause_collector: bool = False) -> float:
    """Milliseconds per step over `steps` steps after `warmup` untimed ones,
    with the device synchronised on both sides of the timed region. The
    garbage collector runs a full collection before the region and stays
    enabled inside it, as in a training loop (`pause_collector`: it stays
    off inside, which keeps a generation-2 collection of torch's ~170k
    tracked objects, ~40 ms of host time, out of a short region).

    With `min_ms` > 0, a timed region shorter than that is measured again
    over enough steps to fill it (the first region then counts as warm-up):
    a 64x64 config steps in about half a millisecond, and ten of its steps
    time the host's clock ramp more than the step."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    collector = paused_collector if pause_collector else collected_collector
    while True:
        with collector():
            start = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            elapsed = (time.perf_counter() - start) * 1000
        if elapsed >= min_ms:
            return elapsed / steps
        steps = math.ceil(min_ms / max(elapsed / steps, 1e-3))


# Shortest timed region of a secondary (per-config or graph-replay) figure.
MIN_CONFIG_MS = 250.0


def per_config_times(skip: int, steps: int, warmup: int, device, validate: bool) -> dict:
    """ms/step and Mpix/s of every other BASELINE config, measured in this run."""
    out = {}
    for index, cfg in CONFIGS.items():
        if index == skip:
            continue
        *_, step = prepare(index, device, validate)
        ms = time_steps(step, steps, warmup, min_ms=MIN_CONFIG_MS)
        pixels = cfg["scenes"] * cfg["cameras"] * cfg["width"] * cfg["height"]
        out[str(index)] = {"workload": cfg["name"], "ms_per_step": round(ms, 4),
                           "mpix_per_s": round(pixels / (ms / 1000) / 1e6, 3)}
        del step
        torch.cuda.empty_cache()
    return out


def graph_replay_times(steps: int, warmup: int, device, indices=None) -> dict:
    """Every config's render and backward captured once in a HIP graph and
    replayed: ms per replay next to the eager step.

    Inside ``fixed_capacity`` the renderers never synchronise with the host,
    so one capture holds the render, the loss gradient's multi-tensor pass
    and the backward; a replay then costs the kernels alone. The loss's
    reduction stays out of the graph (torch's reduction records a memset
    node, which is not replay-safe here) and the backward receives the loss
    gradient 2 x / n directly, so a replay computes the eager step's
    parameter gradients without the scalar loss itself. The capacity is the
    eager intersection count plus a quarter; every replay is checked not to
    exceed it, and one replay's gradients are compared with eager ones.
    `indices` restricts the configs (all by default).
    """
    from diff_gabor_splatting_amd import fixed_capacity

    out = {}
    for index, cfg in CONFIGS.items():
        if indices is not None and index not in indices:
            continue
        _, values, renderer, options, step = prepare(index, device, False)
        eager_ms = time_steps(step, steps, warmup, min_ms=MIN_CONFIG_MS)
        params = [v for v in values.values() if v.requires_grad]

        def body():
            rgb, alpha, meta = renderer(**values, **options)
            groups = _loss_groups(rgb, alpha, meta, cfg["channels"])
            scale = 2.0 / sum(t.numel() for t in groups)
            return torch.autograd.grad(groups, params, grad_outputs=torch._foreach_mul(
                [t.detach() for t in groups], scale))

        with fixed_capacity(1 << 26) as probe:
            renderer(**values, **options)
        count = probe.check()
        capacity = fixed_capacity(count + count // 4 + 1024)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with capacity, torch.cuda.stream(side):
            for _ in range(2):
                body()
        torch.cuda.current_stream().wait_stream(side)
        capacity.check()
        graph = torch.cuda.CUDAGraph()
        with capacity, torch.cuda.graph(graph):
            grads = body()
        replay_ms = time_steps(graph.replay, steps, warmup, min_ms=MIN_CONFIG_MS)
        capacity.check()  # raises if any replay exceeded the capacity
        expected = body()
        worst = max(float(((g - e).abs().max() / e.abs().max().clamp_min(1e-30)).item())
                    for g, e in zip(grads, expected))
        out[str(index)] = {"workload": cfg["name"], "eager_ms_per_step": round(eager_ms, 4),
                           "replay_ms": round(replay_ms, 4), "capacity": count + count // 4 + 1024,
                           "grad_max_rel_diff_vs_eager": worst}
        del graph, grads, expected, step, values
        torch.cuda.empty_cache()
    return out


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--config", type=int, default=4, choices=sorted(CONFIGS))
    parser.add_argument("--validate", action="store_true",
                        help="run the numerical input checks inside every step")
    parser.add_argument("--cpu-baseline", type=int, default=1,
                        help="1: time the CPU oracle on config 0 (and a crop of config 4)")
    parser.add_argument("--per-config", type=int, default=1,
                        help="1: also time every other config (ms/step), same run")
    parser.add_argument("--graph-replay", type=int, default=1,
                        help="1: also time every config captured in a HIP graph and replayed")
    parser.add_argument("--cpu-crop", type=int, default=32,
                        help="edge in pixels of the secondary config-4 CPU crop (0: skip it)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only copy 1 GiB device-to-device three times and exit: the "
                             "known-size kernel that fixes how rocprof byte counters read")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(
            f"bench.py runs on exactly one GPU (got --gpus {args.gpus}); multi-GPU runs are "
            "not part of this build",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration()
    from diff_gabor_splatting_amd import _native

    cfg = CONFIGS[args.config]
    device = torch.device("cuda:0")
    cpu_values, values, renderer, options, step = prepare(args.config, device, args.validate)
    ms_per_step = time_steps(step, args.steps, args.warmup)
    # Per-family kernel times from HIP events on the launch stream, over the
    # same number of steps run again after the timed region (the events
    # themselves cost host time, so they stay out of the timed steps).
    _native.profile_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    kernels = {}
    for family in _native.PROFILE_FAMILIES:
        total_ms, launches = _native.profile_read(family)
        kernels[family] = {"ms_per_step": total_ms / args.steps, "launches": launches,
                           "avg_launch_ms": total_ms / launches if launches else 0.0}
    _native.profile_enable(False)
    images = cfg["scenes"] * cfg["cameras"]
    pixels = images * cfg["width"] * cfg["height"]
    mpix = pixels / (ms_per_step / 1000) / 1e6

    # Workload statistics of the last step (outside the timed region).
    stats = workload_stats(values, renderer, options)
    dominant = max(("render_forward", "render_backward"), key=lambda f: kernels[f]["ms_per_step"])
    avg_ms = kernels[dominant]["avg_launch_ms"]
    roofline = roofline_entry(dominant, cfg, pixels, stats, avg_ms)
    walk = measured_walk(cfg["name"])
    evals_forward = walk["forward_pixel_record_visits"] if walk else None
    # Surfel-pixel evaluations per second: the forward's visits (each pixel's
    # list records up to the one that stops it, from the diagnostics build's
    # count of this workload) plus the backward's walk as the reference
    # defines it (every tile's 256 pixels up to its largest contributor count).
    evaluations = (None if evals_forward is None else
                   round((evals_forward + stats["evals_backward"]) / (ms_per_step / 1000), 1))
    secondary = secondary_step_times(args, device, ms_per_step)
    result = {
        "metric": "fwd+bwd Mpix/s (1M surfels at 1080p); fwd+bwd ms/iter; HBM roofline",
        "value": round(mpix, 3),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded BASELINE distributions, generated on the CPU)",
        "config": {
            "workload": cfg["name"],
            "surfels_per_scene": cfg["n"],
            "images": images,
            "width": cfg["width"],
            "height": cfg["height"],
            "sh_degree": cfg["sh"],
            "neural": cfg["neural"],
            "packed": cfg["packed"],
            "validate": args.validate,
            "objective": "mean of squares of the listed map channels as one multi-tensor pass "
                         "(value and gradient of torch.cat(maps, -1).square().mean()); the "
                         "reference's literal expression is timed in secondary",
            "garbage_collector": "enabled in the timed region (full collection before it)",
            "tile_intersections": stats["intersections"],
            "visible_pairs": stats["visible"],
            "records_replayed": stats["records_replayed"],
            "surfel_pixel_evaluations_per_s": evaluations,
            "surfel_pixel_evaluations": {
                "forward_visits": evals_forward,
                "backward_reference_walk": stats["evals_backward"],
                "source": walk["source"] if walk else None,
            },
        },
        "roofline": roofline,
        "kernels": {k: round(v["ms_per_step"], 4) for k, v in kernels.items()},
        "secondary": secondary,
        "gpu": torch.cuda.get_device_name(device),
    }
    del values, step
    torch.cuda.empty_cache()
    if args.per_config:
        result["per_config"] = per_config_times(args.config, args.steps, args.warmup, device,
                                                args.validate)
    if args.graph_replay:
        result["graph_replay"] = graph_replay_times(args.steps, args.warmup, device)
    if args.cpu_baseline:
        gpu_config0 = result.get("per_config", {}).get("0", {}).get("ms_per_step")
        if args.config == 0:
            gpu_config0 = round(ms_per_step, 4)
        result["cpu_baseline"] = cpu_baseline(cpu_values if args.config == 4 else None, args,
                                              gpu_config0)
    print(json.dumps(result), flush=True)
    return 0


def copy_calibration() -> int:
    """A plain copy of known size: 1 GiB read and 1 GiB written per launch."""
    source = torch.ones(COPY_BYTES // 4, device="cuda:0")
    target = torch.empty_like(source)
    torch.cuda.synchronize()
    for _ in range(3):
        target.copy_(source)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "launches": 3}), flush=True)
    return 0


# One wave64 VALU instruction issues per SIMD every 4 cycles: 256 CUs x 4
# SIMDs at 2.4 GHz; 64 lanes each. A single-issue model: gfx950 also issues
# some VALU instructions on a second path (SQ_ACTIVE_INST_VALU2), so a kernel
# can exceed it.
VALU_ISSUE_PER_S = 256 * 4 * 2.4e9 / 4
VALU_LANE_OPS_PEAK_T = VALU_ISSUE_PER_S * 64 / 1e12
# MI355X's published FP32 vector peak (packed FMAs on every lane), and the
# non-packed FMA rate this build issues at (packed FP32 is disabled).
FP32_PEAK_TFLOPS = 157.3
FP32_NONPACKED_FMA_TFLOPS = VALU_ISSUE_PER_S * 64 * 2 / 1e12


def measured_valu(kernel: str, workload: str, avg_ms: float):
    """VALU issue of ``kernel`` from the committed rocprof counter summary:
    SQ_INSTS_VALU per launch, the time issuing them takes at one wave64
    instruction per SIMD every 4 cycles, and that time as a fraction of the
    launch time measured in this run; plus the profiled run's own busy
    fractions (4-cycle model and SQ_ACTIVE_INST_VALU, which also charges the
    extra cycles of multi-cycle instructions) and its LDS busy fraction.
    None when no summary covers it."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"{kernel}_valu.json")
    try:
        with open(path) as handle:
            summary = json.load(handle)
    except (OSError, ValueError):
        return None
    if summary.get("kernel") != kernel or summary.get("workload") != workload or not avg_ms:
        return None
    issue_ms = summary["valu_instructions"] / VALU_ISSUE_PER_S * 1e3
    out = {"instructions": summary["valu_instructions"], "issue_ms": round(issue_ms, 4),
           "frac": round(issue_ms / avg_ms, 4),
           "profiled_busy_model": summary.get("busy_model"),
           "profiled_busy_measured": summary.get("busy_measured"),
           "profiled_second_issue_busy": summary.get("second_issue_busy"),
           "profiled_lds_busy": summary.get("lds_busy"),
           "source": summary.get("source")}
    flops = summary.get("fp32_flops_per_wave")
    if flops:
        # SQ_INSTS_VALU_FLOPS_FP32 counts per wave instruction (FMA 2, add,
        # multiply and transcendental 1); 64 lanes each.
        tflops = flops * 64 / (avg_ms / 1e3) / 1e12
        out["fp32"] = {"achieved": round(tflops, 3), "unit": "TFLOP/s",
                       "peak": FP32_PEAK_TFLOPS, "frac": round(tflops / FP32_PEAK_TFLOPS, 4),
                       "nonpacked_fma_peak": round(FP32_NONPACKED_FMA_TFLOPS, 2),
                       "nonpacked_fma_frac": round(tflops / FP32_NONPACKED_FMA_TFLOPS, 4),
                       "instruction_mix": summary.get("fp32_mix")}
    return out


def roofline_entry(kernel: str, cfg: dict, pixels: int, stats: dict, avg_ms: float) -> dict:
    """The dominant compositor's roofline: VALU issue (its bound) as the
    primary figure, HBM beside it.

    VALU: SQ_INSTS_VALU per launch from the committed counter summary of
    this workload, times 64 lanes, over the launch time measured in this
    run, against the non-packed fp32 issue ceiling (one wave64 instruction
    per SIMD every 4 cycles on 256 CUs at 2.4 GHz = 39.3 T lane-ops/s;
    packed FP32 is disabled in this build). That model is single-issue;
    gfx950 issues some VALU instructions on a second path as well
    (SQ_ACTIVE_INST_VALU2, reported beside it), so the fraction can exceed
    1. Beside it, `valu.fp32`: the FP32 flops the counters attribute to the
    kernel (SQ_INSTS_VALU_FLOPS_FP32) against MI355X's published FP32 peak
    and the non-packed FMA rate. HBM: algorithmic bytes of the
    reference's walk (every tile's records up to its largest contributor
    count) and of the walk this kernel performs (the replayed records), the
    measured L2-to-memory traffic and its ratio to both.
    """
    walked = stats["records_backward" if kernel == "render_backward" else "records_forward"]
    reference_bytes = algorithmic_bytes(kernel, cfg["neural"], pixels, walked, stats["visible"])
    replay_bytes = None if stats["records_replayed"] is None else algorithmic_bytes(
        kernel, cfg["neural"], pixels, stats["records_replayed"], stats["visible"],
        entry_bytes=REPLAY_ENTRY_BYTES)
    seconds = avg_ms / 1000 if avg_ms else None
    traffic = measured_traffic(kernel, cfg["name"])
    hbm = {
        "achieved": round(reference_bytes / seconds / 1e9, 2) if seconds else None,
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(reference_bytes / seconds / 1e9 / HBM_PEAK_GBS, 5) if seconds else None,
        "algorithmic_bytes_per_launch": reference_bytes,
        "replay_walk_bytes_per_launch": replay_bytes,
        "achieved_replay_walk": (round(replay_bytes / seconds / 1e9, 2)
                                 if seconds and replay_bytes else None),
        "traffic": traffic,
        "traffic_over_reference_walk": round(traffic / reference_bytes, 3) if traffic else None,
        "traffic_over_replay_walk": (round(traffic / replay_bytes, 3)
                                     if traffic and replay_bytes else None),
    }
    valu = measured_valu(kernel, cfg["name"], avg_ms)
    entry = {"kernel": kernel, "avg_launch_ms": round(avg_ms, 4)}
    if valu is None:
        # No counter summary for this workload: the HBM figures only.
        entry.update(bound="hbm", achieved=hbm["achieved"], peak=HBM_PEAK_GBS, unit="GB/s",
                     frac=hbm["frac"], traffic=traffic, hbm=hbm)
        return entry
    lane_ops = valu["instructions"] * 64 / seconds / 1e12
    entry.update(bound="valu", achieved=round(lane_ops, 3), peak=round(VALU_LANE_OPS_PEAK_T, 4),
                 unit="T VALU lane-ops/s", frac=round(lane_ops / VALU_LANE_OPS_PEAK_T, 4),
                 traffic=traffic, hbm=hbm, valu=valu)
    return entry


def measured_walk(workload: str):
    """(pixel, record) counts of ``workload`` from the committed summary of
    the diagnostics build (``python -m diff_gabor_splatting_amd.diagnostics``),
    or None when no summary covers it. The counts are deterministic: they
    follow from the sorted lists and the forward's float results."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "render_walk_counts.json")
    try:
        with open(path) as handle:
            summaries = json.load(handle)
    except (OSError, ValueError):
        return None
    for summary in summaries.get("workloads", []):
        if summary.get("workload") == workload:
            return {**summary, "source": "profiles/render_walk_counts.json"}
    return None


def secondary_step_times(args, device, headline_ms: float) -> dict:
    """The headline step timed two other ways, labelled: with the collector
    paused inside the timed region, and with the reference benchmark's
    literal objective (torch.cat of the maps, square, mean)."""
    out = {}
    _, _, _, _, step = prepare(args.config, device, args.validate)
    out["collector_paused_ms_per_step"] = round(
        time_steps(step, args.steps, args.warmup, pause_collector=True), 4)
    del step
    _, _, _, _, step = prepare(args.config, device, args.validate, objective="reference")
    out["reference_objective_ms_per_step"] = round(time_steps(step, args.steps, args.warmup), 4)
    out["headline_ms_per_step"] = round(headline_ms, 4)
    del step
    torch.cuda.empty_cache()
    return out


def measured_traffic(kernel: str, workload: str):
    """Bytes per launch of ``kernel`` between L2 and memory, from the
    committed rocprof counter summary of the same bench command.

    The summary holds read bytes (128/64/32 x TCC_EA0_RDREQ_128B/_64B/_32B)
    and written bytes (64 x TCC_EA0_WRREQ_64B + 32 x the other write
    requests, atomics included), a split that a 1 GiB device copy reads back
    exactly. None when no summary covers this workload.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"{kernel}_traffic.json")
    try:
        with open(path) as handle:
            summary = json.load(handle)
    except (OSError, ValueError):
        return None
    if summary.get("kernel") != kernel or summary.get("workload") != workload:
        return None
    return int(summary["read_bytes"] + summary["write_bytes"])


def workload_stats(values, renderer, options):
    """Intersections, visible pairs, records walked and replayed, and the
    backward's surfel-pixel evaluations of one call. The render records
    gradients (the renderers write replay lists only when a backward can
    follow); no backward is run."""
    from diff_gabor_splatting_amd import _native

    captured = {}
    original = _native.rasterize_forward

    def spy(*a, **k):
        out = original(*a, **k)
        captured["out"] = out
        captured["args"] = a
        return out

    _native.rasterize_forward = spy
    try:
        rgb, alpha, meta = renderer(**values, **options)
    finally:
        _native.rasterize_forward = original
    del rgb, alpha, meta
    maps, point_list, ranges, state, contributors = captured["out"][:5]
    replay = captured["out"][5] if len(captured["out"]) > 5 else None
    geometry = captured["args"][0]
    width, height = options["width"], options["height"]
    tw, th = _native.tile_grid(width, height)
    lengths = (ranges[:, 1] - ranges[:, 0]).long()
    images = contributors.shape[0]
    pad_h, pad_w = th * 16 - height, tw * 16 - width
    contrib = torch.nn.functional.pad(contributors, (0, pad_w, 0, pad_h))
    per_tile = contrib.reshape(images, th, 16, tw, 16).permute(0, 1, 3, 2, 4).reshape(-1, 256)
    tile_max = per_tile.max(-1).values.long()
    # The backward as the reference walks it: every tile up to its largest
    # contributor count; with replay lists it gathers only the replayed
    # records (those some pixel took).
    return {
        "intersections": int(point_list.numel()),
        "visible": int((captured["args"][5] > 0).sum()),
        "pairs": int(geometry.shape[0]),
        "records_forward": int(lengths.sum()),
        "records_backward": int(tile_max.sum()),
        "records_replayed": int(replay[1].long().sum()) if replay is not None else None,
        "evals_backward": int(tile_max.sum()) * 256,
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's
    processor string where that is not available."""
    try:
        with open("/proc/cpuinfo") as handle:
            for line in handle:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown CPU"


def cpu_threads() -> int:
    """Every core this process may run on: its CPU affinity, capped by
    OMP_NUM_THREADS when the environment sets a share (on the GPU boxes this
    is the box's CPU share, not the host's full core count)."""
    available = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (
        os.cpu_count() or 1)
    share = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(available, int(share))) if share.isdigit() and int(share) > 0 else available


def oracle_step_seconds(values, cfg, width, height, warmup: int, iterations: int):
    """Seconds per fwd+bwd step of the fp32 torch oracle (autograd backward),
    loss as in the GPU step, after `warmup` untimed steps."""
    import oracle.render as oracle_render

    values = {k: v.clone().requires_grad_(k not in CAMERA_KEYS) for k, v in values.items()}
    function = (oracle_render.rasterize_neural_gabors if cfg["neural"]
                else oracle_render.rasterize_gabors)
    options = dict(width=width, height=height, packed=cfg["packed"])
    if not cfg["neural"]:
        options["sh_degree"] = cfg["sh"]
    params = [v for v in values.values() if v.requires_grad]
    times = []
    for k in range(warmup + iterations):
        start = time.perf_counter()
        maps, _, _ = function(**values, **options)
        loss = maps[..., : cfg["channels"]].square().mean()
        torch.autograd.grad(loss, params)
        if k >= warmup:
            times.append(time.perf_counter() - start)
    return sum(times) / len(times), times


def cpu_baseline(config4_values, args, gpu_config0_ms):
    """The CPU oracle on this host. Primary: config 0 (the designated CPU
    config) at full frame, 2 warm-up and 5 timed fwd+bwd steps. Secondary
    (labelled): one step over a centre crop of config 4 with all its 1M
    surfels projected, which mostly measures per-surfel work."""
    threads = cpu_threads()
    torch.set_num_threads(threads)
    cfg0 = CONFIGS[0]
    seconds, times = oracle_step_seconds(make_scene(0), cfg0, cfg0["width"], cfg0["height"],
                                         warmup=2, iterations=5)
    pixels = cfg0["width"] * cfg0["height"]
    out = {
        "value": round(pixels / seconds / 1e6, 6),
        "unit": "Mpix/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{cfg0['name']}, full frame: fp32 torch oracle forward + autograd backward, "
                   f"2 warm-up + {len(times)} timed steps, {seconds:.3f} s per step "
                   f"(steps {', '.join(f'{t:.3f}' for t in times)} s) on {threads} threads"),
        "ms_per_step": round(seconds * 1000, 2),
        "gpu_ms_per_step_same_workload": gpu_config0_ms,
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
    }
    if config4_values is not None and args.cpu_crop:
        cfg4, edge = CONFIGS[4], args.cpu_crop
        x0, y0 = (cfg4["width"] - edge) // 2, (cfg4["height"] - edge) // 2
        crop_seconds, _ = oracle_step_seconds(crop(config4_values, x0, y0), cfg4, edge, edge,
                                              warmup=0, iterations=1)
        out["secondary_config4_crop"] = {
            "value": round(edge * edge / crop_seconds / 1e6, 6),
            "unit": "Mpix/s",
            "sample": (f"{edge}x{edge} centre crop of config 4 (all {cfg4['n']} surfels "
                       f"projected, SH evaluated and binned), one fwd+bwd step, "
                       f"{crop_seconds:.2f} s; dominated by per-surfel work, not comparable "
                       f"with a full-frame rate"),
        }
    return out


if __name__ == "__main__":
    sys.exit(main())
