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

from diff_gabor_splatting_amd.timing import paused_collector

HBM_PEAK_GBS = 8000.0
COPY_BYTES = 1 << 30
FP32_VALU_PEAK_TFLOPS = 157.3

CONFIGS = {
    0: dict(name="config0: classic SH0, N=1024, 64x64", n=1024, width=64, height=64, scenes=1,
            cameras=1, sh=0, neural=False, packed=False, channels=9),
    1: dict(name="config1: classic SH3, N=100k, 1024x768, rgb+alpha+depth loss", n=100_000,
            width=1024, height=768, scenes=1, cameras=1, sh=3, neural=False, packed=False,
            channels=5),
    2: dict(name="config2: neural SIREN, N=100k, 800x800", n=100_000, width=800, height=800,
            scenes=1, cameras=1, sh=None, neural=True, packed=False, channels=9),
    3: dict(name="config3: classic SH3, 8 scenes x 4 cameras, N=50k/scene, 512x512, packed",
            n=50_000, width=512, height=512, scenes=8, cameras=4, sh=3, neural=False,
            packed=True, channels=9),
    4: dict(name="config4: classic SH3, N=1M surfels, 1920x1080, all 9 maps in loss",
            n=1_000_000, width=1920, height=1080, scenes=1, cameras=1, sh=3, neural=False,
            packed=False, channels=9),
}


def _uniform(generator, shape, low, high):
    return torch.rand(shape, generator=generator) * (high - low) + low


def _log_uniform(generator, shape, low, high):
    return torch.exp(_uniform(generator, shape, math.log(low), math.log(high)))


def _ring_cameras(generator, scenes, cameras, radius=5.0):
    """Rigid world->camera views on a ring around the origin, looking at it."""
    views = torch.zeros(scenes, cameras, 4, 4)
    for s in range(scenes):
        for c in range(cameras):
            yaw = float(_uniform(generator, (), 0.0, 2 * math.pi))
            centre = torch.tensor([radius * math.sin(yaw), 0.0, -radius * math.cos(yaw)])
            forward = -centre / centre.norm()
            down = torch.tensor([0.0, 1.0, 0.0])
            right = torch.linalg.cross(down, forward)
            right = right / right.norm()
            down = torch.linalg.cross(forward, right)
            R = torch.stack([right, down, forward])  # rows: camera axes in world
            views[s, c, :3, :3] = R
            views[s, c, :3, 3] = -R @ centre
            views[s, c, 3, 3] = 1.0
    return views


def make_scene(index: int, seed: int | None = None, n: int | None = None):
    """Seeded CPU tensors of one BASELINE config (see BASELINE.json `configs`)."""
    cfg = CONFIGS[index]
    g = torch.Generator().manual_seed(index if seed is None else seed)
    S, C = cfg["scenes"], cfg["cameras"]
    N = cfg["n"] if n is None else n
    W, H = cfg["width"], cfg["height"]
    if index == 0:
        means = torch.cat([_uniform(g, (S, N, 2), -1, 1), _uniform(g, (S, N, 1), 2, 4)], -1)
    elif index in (1, 2):
        means = torch.cat([_uniform(g, (S, N, 2), -3, 3), _uniform(g, (S, N, 1), 2, 8)], -1)
    elif index == 3:
        means = _uniform(g, (S, N, 3), -2, 2)
    else:
        centres = torch.cat([_uniform(g, (64, 2), -5, 5), _uniform(g, (64, 1), 2, 12)], -1)
        which = torch.randint(0, 64, (S, N), generator=g)
        means = centres[which] + torch.randn(S, N, 3, generator=g) * 0.3
    quats = torch.randn(S, N, 4, generator=g)
    quats = quats / quats.norm(dim=-1, keepdim=True)
    low, high = (0.005, 0.1) if index == 4 else (0.02, 0.2)
    scales = _log_uniform(g, (S, N, 2), low, high)
    opacities = _uniform(g, (S, N), 0.1, 0.9)
    if index == 3:
        views = _ring_cameras(g, S, C)
    else:
        views = torch.eye(4).expand(S, C, 4, 4).clone()
    focal = {0: 80.0, 1: 900.0, 2: 900.0, 3: 600.0, 4: 1500.0}[index]
    cx, cy = (32.0, 32.0) if index == 0 else ((W - 1) / 2, (H - 1) / 2)
    K = torch.tensor([[focal, 0.0, cx], [0.0, focal, cy], [0.0, 0.0, 1.0]])
    values = dict(means=means, quaternions=quats, scales=scales, opacities=opacities,
                  view_matrices=views, intrinsics=K.expand(S, C, 3, 3).clone())
    if cfg["neural"]:
        values.update(
            input_weights=_uniform(g, (S, N, 6, 5), -1 / 5, 1 / 5),
            input_biases=torch.zeros(S, N, 6),
            output_weights=_uniform(g, (S, N, 3, 6), -1 / 30, 1 / 30),
            output_biases=torch.zeros(S, N, 3),
        )
    else:
        k = (cfg["sh"] + 1) ** 2
        weights = _uniform(g, (S, N, 4), 0, 1)
        values.update(
            colors=_uniform(g, (S, N, k, 3), 0, 1),
            secondary_colors=_uniform(g, (S, N, k, 3), 0, 1),
            frequency_weights=weights / weights.sum(-1, keepdim=True),
            frequency_magnitudes=_uniform(g, (S, N, 4), 0, 8),
            phases=_uniform(g, (S, N, 4), 0, 2 * math.pi),
        )
    return values


CAMERA_KEYS = ("view_matrices", "intrinsics")


def crop(values, x0: int, y0: int):
    """The same scene seen through a window whose top-left pixel is (x0, y0)."""
    out = dict(values)
    K = values["intrinsics"].clone()
    K[..., 0, 2] -= x0
    K[..., 1, 2] -= y0
    out["intrinsics"] = K
    return out


class _MeanOfSquares(torch.autograd.Function):
    """Mean of squares over several map groups, taken as one flat vector.

    Forward: one multi-tensor pass for the groups' Euclidean norms (each
    element read once), then a sum of the squared norms over n. Backward:
    one multi-tensor pass writing each group's gradient g * 2 x / n. The
    groups are never concatenated: the compositor's backward takes one
    gradient tensor per map group, so a concatenated copy only costs a
    read and a write of every map element.
    """

    @staticmethod
    def forward(ctx, *groups):
        ctx.save_for_backward(*groups)
        ctx.count = sum(t.numel() for t in groups)
        return torch.stack(torch._foreach_norm(list(groups))).square().sum() / ctx.count

    @staticmethod
    def backward(ctx, grad):
        return tuple(torch._foreach_mul(list(ctx.saved_tensors), grad * (2.0 / ctx.count)))


def _loss(rgb, alpha, meta, channels):
    """Mean of squares of the first `channels` map channels in the reference
    benchmark's order - rgb, alpha, depth, normals, distortion - its objective
    ``torch.cat(maps, -1).square().mean()`` (benchmarks/
    benchmark_rasterization.py:80-82, 133).

    Same value and gradient, less glue: a mean of squares does not depend on
    the order or grouping of the elements, so each group enters as it is
    (`_MeanOfSquares`). Groups past `channels` are left out rather than
    sliced off (a slice adds a zero-filled full-size gradient).
    """
    return _MeanOfSquares.apply(*_loss_groups(rgb, alpha, meta, channels))


def _loss_groups(rgb, alpha, meta, channels):
    """The map groups holding the loss's first `channels` channels (the last
    one sliced when it holds more)."""
    groups, left = [], channels
    for t in (rgb, alpha, meta["accumulated_depth"], meta["normals"], meta["distortion"]):
        if left <= 0:
            break
        k = t.shape[-1]
        groups.append(t if k <= left else t[..., :left])
        left -= k
    return groups


def algorithmic_bytes(kind: str, neural: bool, pixels: int, records: int, pairs: int,
                      rows: int) -> int:
    """Compulsory HBM bytes of one compositor launch.

    pixels: output pixels; records: tile-records the kernel walks (each gathers
    point_list 4 B + primitive id 8 B + geometry 68 B + appearance 4A B +
    opacity 4 B); pairs/rows: gradient rows written once by the backward.
    Forward writes maps 36 B + state 12 B + contributors 4 B per pixel; the
    backward reads the same 52 B per pixel.
    """
    appearance = 57 if neural else 18
    record = 4 + 8 + 68 + 4 * appearance + 4
    total = pixels * 52 + records * record
    if kind == "render_backward":
        total += pairs * 68 + rows * (4 * appearance + 4)
    return int(total)


def prepare(index: int, device, validate: bool):
    """Seeded inputs of one config on the device and a closure running one
    fwd+bwd step on them through the public API."""
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    cfg = CONFIGS[index]
    cpu_values = make_scene(index)
    values = {k: v.to(device).contiguous() for k, v in cpu_values.items()}
    for k, v in values.items():
        v.requires_grad_(k not in CAMERA_KEYS)
    renderer = rasterize_neural_gabors if cfg["neural"] else rasterize_gabors
    options = dict(width=cfg["width"], height=cfg["height"], packed=cfg["packed"],
                   validate=validate)
    if not cfg["neural"]:
        options["sh_degree"] = cfg["sh"]
    params = [v for v in values.values() if v.requires_grad]

    def step():
        for p in params:
            p.grad = None
        rgb, alpha, meta = renderer(**values, **options)
        _loss(rgb, alpha, meta, cfg["channels"]).backward()
        return meta

    return cpu_values, values, renderer, options, step


def time_steps(step, steps: int, warmup: int, min_ms: float = 0.0) -> float:
    """Milliseconds per step over `steps` steps after `warmup` untimed ones,
    with the device synchronised on both sides of the timed region and the
    garbage collector paused inside it.

    With `min_ms` > 0, a timed region shorter than that is measured again
    over enough steps to fill it (the first region then counts as warm-up):
    a 64x64 config steps in about half a millisecond, and ten of its steps
    time the host's clock ramp more than the step."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    while True:
        with paused_collector():
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
    walked = stats["records_backward" if dominant == "render_backward" else "records_forward"]
    algo = algorithmic_bytes(dominant, cfg["neural"], pixels, walked, stats["pairs"],
                             stats["rows"])
    avg_ms = kernels[dominant]["avg_launch_ms"]
    achieved = algo / (avg_ms / 1000) / 1e9 if avg_ms else 0.0
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
            "tile_intersections": stats["intersections"],
            "visible_pairs": stats["visible"],
            "pixel_record_pairs_walked_per_s": round(
                (stats["evals_forward"] + stats["evals_backward"]) / (ms_per_step / 1000), 1
            ),
        },
        "roofline": {
            "kernel": dominant,
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5),
            "traffic": measured_traffic(dominant, cfg["name"]),
            "algorithmic_bytes_per_launch": algo,
            "avg_launch_ms": round(avg_ms, 4),
            "note": "the compositors are bound by VALU issue, not HBM: see valu",
            "valu": measured_valu(dominant, cfg["name"], avg_ms),
        },
        "kernels": {k: round(v["ms_per_step"], 4) for k, v in kernels.items()},
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
# SIMDs at 2.4 GHz.
VALU_ISSUE_PER_S = 256 * 4 * 2.4e9 / 4


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
    return {"instructions": summary["valu_instructions"], "issue_ms": round(issue_ms, 4),
            "frac": round(issue_ms / avg_ms, 4),
            "profiled_busy_model": summary.get("busy_model"),
            "profiled_busy_measured": summary.get("busy_measured"),
            "profiled_lds_busy": summary.get("lds_busy"),
            "source": summary.get("source")}


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
    """Intersections, visible pairs and surfel-pixel evaluation counts of one call."""
    from diff_gabor_splatting_amd import _native

    with torch.no_grad():
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
    maps, point_list, ranges, state, contributors = captured["out"][:5]
    geometry, appearance = captured["args"][0], captured["args"][1]
    width, height = options["width"], options["height"]
    tw, th = _native.tile_grid(width, height)
    lengths = (ranges[:, 1] - ranges[:, 0]).long()
    images = contributors.shape[0]
    pad_h, pad_w = th * 16 - height, tw * 16 - width
    contrib = torch.nn.functional.pad(contributors, (0, pad_w, 0, pad_h))
    per_tile = contrib.reshape(images, th, 16, tw, 16).permute(0, 1, 3, 2, 4).reshape(-1, 256)
    tile_max = per_tile.max(-1).values.long()
    # (pixel, record) pairs walked: the backward walks every tile up to its
    # largest contributor count; the forward at most the whole tile list.
    return {
        "intersections": int(point_list.numel()),
        "visible": int((captured["args"][5] > 0).sum()),
        "pairs": int(geometry.shape[0]),
        "rows": int(appearance.shape[0]),
        "records_forward": int(lengths.sum()),
        "records_backward": int(tile_max.sum()),
        "evals_forward": int(lengths.sum()) * 256,
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
