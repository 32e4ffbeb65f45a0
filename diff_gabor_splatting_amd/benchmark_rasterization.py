"""Loop vs fused-dense vs fused-packed rendering through the public API.

The caller-side methodology of the reference's benchmark
(benchmarks/benchmark_rasterization.py:101-251), on this implementation:
the same command-line options, the same synthetic scene distributions, a
parity gate before any timing (every camera rendered separately against
one fused call, dense and packed, maps and parameter gradients), HIP-event
timing of forward (including the scalar loss) and backward, and a JSON
report with the same keys. Optional kernel profiling uses this library's
own HIP-event counters per kernel family instead of a tracing profiler.

    python -m diff_gabor_splatting_amd.benchmark_rasterization --method both \\
        --num-primitives 10000 --num-cameras 4 --output-json results.json
"""

from __future__ import annotations

import argparse
import json
import platform
import subprocess
from pathlib import Path

import torch

from . import _native
from .rendering import rasterize_gabors, rasterize_neural_gabors

IMPLEMENTATIONS = ("single_view_loop", "fused_dense", "fused_packed")
CAMERA_KEYS = ("view_matrices", "intrinsics", "backgrounds")
NEURAL_FIELDS = (
    ("input_weights", (6, 5), 1 / 5),
    ("input_biases", (6,), 1 / 5),
    ("output_weights", (3, 6), 1 / 30),
    ("output_biases", (3,), 0.1),
)


def make_scene(args: argparse.Namespace, method: str) -> dict:
    """Deterministic synthetic scene (built outside every timed region).

    Distributions follow the reference benchmark (:16-64): means ~ N(0, 0.6)
    with depth U(3, 5), near-identity unit quaternions, scales 0.025,
    opacity 0.3, cameras spread along x, focal length 0.8 x image size.
    """
    device = torch.device("cuda")
    gen = torch.Generator(device=device).manual_seed(args.seed)
    b, n, c = args.num_scenes, args.num_primitives, args.num_cameras
    width, height = args.image_width, args.image_height
    means = torch.randn(b, n, 3, device=device, generator=gen) * 0.6
    means[..., 2] = torch.rand(b, n, device=device, generator=gen) * 2 + 3
    quats = torch.randn(b, n, 4, device=device, generator=gen) * 0.1
    quats[..., 0] += 1
    quats = quats / quats.norm(dim=-1, keepdim=True)
    views = torch.eye(4, device=device).repeat(b, c, 1, 1)
    if c > 1:
        views[..., 0, 3] = torch.linspace(-0.2, 0.2, c, device=device)
    intrinsics = torch.zeros(b, c, 3, 3, device=device)
    intrinsics[..., 0, 0] = width * 0.8
    intrinsics[..., 1, 1] = height * 0.8
    intrinsics[..., 0, 2] = (width - 1) / 2
    intrinsics[..., 1, 2] = (height - 1) / 2
    intrinsics[..., 2, 2] = 1.0
    scene = dict(
        means=means,
        quaternions=quats,
        scales=torch.full((b, n, 2), 0.025, device=device),
        opacities=torch.full((b, n), 0.3, device=device),
        view_matrices=views,
        intrinsics=intrinsics,
        backgrounds=torch.full((b, c, 3), 0.05, device=device),
    )
    if method == "classic":
        scene["colors"] = torch.rand(b, n, 3, device=device, generator=gen)
        scene["secondary_colors"] = torch.rand(b, n, 3, device=device, generator=gen)
        scene["frequency_weights"] = torch.full((b, n, 4), 0.25, device=device)
        scene["frequency_magnitudes"] = torch.ones(b, n, 4, device=device)
        scene["phases"] = torch.zeros(b, n, 4, device=device)
    else:
        for name, shape, bound in NEURAL_FIELDS:
            value = torch.empty(b, n, *shape, device=device)
            scene[name] = value.uniform_(-bound, bound, generator=gen)
    for name, value in scene.items():
        value.requires_grad_(name not in CAMERA_KEYS)
    return scene


def _maps(result):
    rgb, alpha, meta = result
    return torch.cat(
        (rgb, alpha, meta["accumulated_depth"], meta["normals"], meta["distortion"]), -1
    )


def render_maps(scene: dict, args: argparse.Namespace, method: str, implementation: str):
    """All nine differentiable channels [B, C, H, W, 9] for one implementation."""
    function = rasterize_gabors if method == "classic" else rasterize_neural_gabors
    options = dict(width=args.image_width, height=args.image_height,
                   validate=not args.skip_validation)
    if implementation != "single_view_loop":
        return _maps(function(**scene, packed=implementation == "fused_packed", **options))
    per_scene = []
    for s in range(args.num_scenes):
        per_camera = []
        for c in range(args.num_cameras):
            view = {
                name: (value[s, c:c + 1] if name in CAMERA_KEYS else value[s]).contiguous()
                for name, value in scene.items()
            }
            per_camera.append(_maps(function(**view, **options)))
        per_scene.append(torch.cat(per_camera, 0))
    return torch.stack(per_scene)


def check_parity(scene: dict, args: argparse.Namespace, method: str) -> None:
    """Fused dense and packed calls must reproduce the per-camera loop."""
    parameters = [value for value in scene.values() if value.requires_grad]
    loop = render_maps(scene, args, method, "single_view_loop")
    expected = torch.autograd.grad(loop.square().mean(), parameters)
    for implementation in IMPLEMENTATIONS[1:]:
        maps = render_maps(scene, args, method, implementation)
        torch.testing.assert_close(maps, loop, atol=2e-5, rtol=2e-4)
        actual = torch.autograd.grad(maps.square().mean(), parameters)
        for value, reference in zip(actual, expected):
            torch.testing.assert_close(value, reference, atol=2e-5, rtol=2e-3)


def _clear_gradients(scene: dict) -> None:
    for value in scene.values():
        value.grad = None


def measure(scene: dict, args: argparse.Namespace, method: str, implementation: str) -> dict:
    """Mean forward (with the scalar loss) and backward milliseconds."""
    for _ in range(args.warmup_iterations):
        _clear_gradients(scene)
        render_maps(scene, args, method, implementation).square().mean().backward()
    _clear_gradients(scene)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    forward_ms, backward_ms = [], []
    for _ in range(args.measurement_iterations):
        _clear_gradients(scene)
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        marks[0].record()
        loss = render_maps(scene, args, method, implementation).square().mean()
        marks[1].record()
        loss.backward()
        marks[2].record()
        marks[2].synchronize()
        forward_ms.append(marks[0].elapsed_time(marks[1]))
        backward_ms.append(marks[1].elapsed_time(marks[2]))
    forward = sum(forward_ms) / len(forward_ms)
    backward = sum(backward_ms) / len(backward_ms)
    return {
        "implementation": implementation,
        "forward_ms": forward,
        "backward_ms": backward,
        "forward_backward_ms": forward + backward,
        "images_per_second": args.num_scenes * args.num_cameras * 1000 / (forward + backward),
        "peak_allocated_memory_mb": torch.cuda.max_memory_allocated() / 1_000_000,
    }


def profile_kernels(scene: dict, args: argparse.Namespace, method: str,
                    implementation: str) -> dict:
    """Per-family kernel milliseconds from the library's HIP-event counters,
    measured separately from the uninstrumented timing."""
    _native.profile_enable(True)
    for _ in range(args.profile_iterations):
        _clear_gradients(scene)
        render_maps(scene, args, method, implementation).square().mean().backward()
    torch.cuda.synchronize()
    families = {name: _native.profile_read(name)[0] / args.profile_iterations
                for name in _native.PROFILE_FAMILIES}
    _native.profile_enable(False)
    forward = families["render_forward"]
    backward = families["render_backward"]
    if not forward or not backward:
        raise RuntimeError("profiling did not record the forward/backward compositor kernels")
    return {
        "forward_kernel_ms": forward,
        "backward_kernel_ms": backward,
        "other_cuda_kernel_ms": sum(families.values()) - forward - backward,
        "kernels_ms": families,
    }


def _parse(argv=None) -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--method", choices=["classic", "neural", "both"], default="both")
    parser.add_argument("--num-primitives", type=int, default=10_000)
    parser.add_argument("--num-scenes", type=int, default=1)
    parser.add_argument("--num-cameras", type=int, default=4)
    parser.add_argument("--image-width", type=int, default=256)
    parser.add_argument("--image-height", type=int, default=256)
    parser.add_argument("--warmup-iterations", type=int, default=5)
    parser.add_argument("--measurement-iterations", type=int, default=20)
    parser.add_argument("--seed", type=int, default=42)
    parser.add_argument("--profile-iterations", type=int, default=0,
                        help="separately profile this many steps per implementation; "
                             "0 disables profiling")
    parser.add_argument("--skip-validation", action="store_true")
    parser.add_argument("--output-json", type=Path)
    args = parser.parse_args(argv)
    positive = ("num_primitives", "num_scenes", "num_cameras", "image_width", "image_height",
                "measurement_iterations")
    for name in positive:
        if getattr(args, name) < 1:
            parser.error(f"--{name.replace('_', '-')} must be positive")
    if args.warmup_iterations < 0 or args.profile_iterations < 0:
        parser.error("--warmup-iterations and --profile-iterations must be nonnegative")
    return args


def run(argv=None) -> dict:
    """Parity gate, then timing of the three implementations; returns the report."""
    args = _parse(argv)
    revision = subprocess.run(["git", "rev-parse", "HEAD"], capture_output=True, text=True,
                              cwd=Path(__file__).resolve().parent)
    report = {
        "environment": {
            "gpu": torch.cuda.get_device_name(),
            "torch": torch.__version__,
            "cuda": torch.version.cuda,
            "hip": torch.version.hip,
            "python": platform.python_version(),
            "revision": revision.stdout.strip() if revision.returncode == 0 else None,
        },
        "workload": {k: v for k, v in vars(args).items() if k != "output_json"},
        "timing": "HIP events; forward includes autograd graph construction and scalar loss; "
                  "combined throughput includes backward",
        "profiling": "optional separate pass with the library's HIP-event kernel counters",
        "memory": "peak total PyTorch-allocated device memory in decimal MB, including inputs "
                  "and autograd state",
        "results": [],
    }
    methods = ("classic", "neural") if args.method == "both" else (args.method,)
    for method in methods:
        scene = make_scene(args, method)
        check_parity(scene, args, method)
        loop_ms = None
        for implementation in IMPLEMENTATIONS:
            result = measure(scene, args, method, implementation)
            if args.profile_iterations:
                result.update(profile_kernels(scene, args, method, implementation))
            loop_ms = loop_ms or result["forward_backward_ms"]
            result["method"] = method
            result["speedup_vs_single_view_loop"] = loop_ms / result["forward_backward_ms"]
            report["results"].append(result)
            print(f"{method:7s} {implementation:16s} forward={result['forward_ms']:.3f} ms "
                  f"backward={result['backward_ms']:.3f} ms "
                  f"speedup={result['speedup_vs_single_view_loop']:.2f}x", flush=True)
        del scene
    if args.output_json:
        args.output_json.parent.mkdir(parents=True, exist_ok=True)
        args.output_json.write_text(json.dumps(report, indent=2) + "\n")
    return report


if __name__ == "__main__":
    run()
