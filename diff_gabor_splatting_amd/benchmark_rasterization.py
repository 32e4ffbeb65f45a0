"""Per-camera loop, fused dense and fused packed rendering, timed through the public API.

Counterpart of the reference's benchmark harness
(benchmarks/benchmark_rasterization.py). Its command line, the synthetic
scene it draws and the keys of its JSON report are kept, so that results
of the two can be read side by side; everything else is this library's:

* scenes come from a declarative recipe (``SCENE_RECIPE``), drawn on the
  CPU from one seeded generator and then moved to the GPU, so a seed gives
  the same scene on every machine;
* each implementation is a strategy object that renders all nine map
  channels of every (scene, camera) image;
* before anything is timed, a parity gate holds the fused strategies to
  the per-camera loop at the project's float bars - maps within 1e-5
  absolute + 1e-4 relative, parameter gradients within 1e-3 of their
  tensor's scale and norm - and records the worst errors in the report;
* steps are timed with HIP events on the launch stream
  (``timing.time_phases``): forward (rendering and the scalar loss) and
  backward, with the garbage collector paused over the measured steps (a
  collection of the interpreter's heap, about 40 ms, otherwise lands in a
  step now and then and dominates the per-camera loop's mean);
* the optional kernel split comes from the library's own per-family event
  counters (``gs_profile_enable``), in a separate pass.

    python -m diff_gabor_splatting_amd.benchmark_rasterization --method both \\
        --num-primitives 10000 --num-cameras 4 --output-json results.json
"""

from __future__ import annotations

import argparse
import json
import platform
import subprocess
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Callable

import torch

from . import _native
from .rendering import rasterize_gabors, rasterize_neural_gabors
from .timing import mean, time_phases

IMPLEMENTATIONS = ("single_view_loop", "fused_dense", "fused_packed")
METHODS = ("classic", "neural")
# Inputs that describe the cameras rather than the surfels: not optimised,
# and sliced per camera by the loop strategy.
CAMERA_INPUTS = ("view_matrices", "intrinsics", "backgrounds")
MAP_OUTPUTS = ("accumulated_depth", "normals", "distortion")

# The parity gate's bars: the project's float32 forward tolerance, and
# gradients within 1e-3 of the tensor's scale (elementwise) and norm.
MAP_ATOL, MAP_RTOL = 1e-5, 1e-4
GRADIENT_TOLERANCE = 1e-3


# --------------------------------------------------------------------------
# Workload


@dataclass(frozen=True)
class Workload:
    """The command line, validated: sizes of the synthetic scene and the
    measurement schedule."""

    method: str
    num_primitives: int
    num_scenes: int
    num_cameras: int
    image_width: int
    image_height: int
    warmup_iterations: int
    measurement_iterations: int
    seed: int
    profile_iterations: int
    skip_validation: bool

    @property
    def images(self) -> int:
        return self.num_scenes * self.num_cameras

    @property
    def methods(self) -> tuple[str, ...]:
        return METHODS if self.method == "both" else (self.method,)


_SIZE_OPTIONS = (
    # flag, default, lower bound
    ("--num-primitives", 10_000, 1),
    ("--num-scenes", 1, 1),
    ("--num-cameras", 4, 1),
    ("--image-width", 256, 1),
    ("--image-height", 256, 1),
    ("--warmup-iterations", 5, 0),
    ("--measurement-iterations", 20, 1),
    ("--seed", 42, None),
    ("--profile-iterations", 0, 0),
)


def parse_workload(argv=None) -> tuple[Workload, Path | None]:
    """Workload and report path from the reference harness's flags."""
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--method", choices=[*METHODS, "both"], default="both")
    for flag, default, _ in _SIZE_OPTIONS:
        help_text = ("separately profile this many steps per implementation; 0 disables "
                     "profiling") if flag == "--profile-iterations" else None
        parser.add_argument(flag, type=int, default=default, help=help_text)
    parser.add_argument("--skip-validation", action="store_true")
    parser.add_argument("--output-json", type=Path)
    args = parser.parse_args(argv)
    for flag, _, lower in _SIZE_OPTIONS:
        value = getattr(args, flag[2:].replace("-", "_"))
        if lower is not None and value < lower:
            parser.error(f"{flag} must be {'positive' if lower else 'nonnegative'}")
    output = args.output_json
    fields = {k: v for k, v in vars(args).items() if k != "output_json"}
    return Workload(**fields), output


# --------------------------------------------------------------------------
# Scenes


def _normal(scale: float = 1.0, shift: float = 0.0):
    return lambda gen, shape: torch.randn(shape, generator=gen) * scale + shift


def _uniform(low: float, high: float):
    return lambda gen, shape: torch.rand(shape, generator=gen) * (high - low) + low


def _constant(value: float):
    return lambda gen, shape: torch.full(shape, value)


def _means(gen, shape):
    """Surfel centres N(0, 0.6^2) across the view, depth uniform in [3, 5]."""
    means = torch.randn(shape, generator=gen) * 0.6
    means[..., 2] = torch.rand(shape[:-1], generator=gen) * 2 + 3
    return means


def _near_identity_rotations(gen, shape):
    """Unit wxyz quaternions close to the identity: N(0, 0.1^2) + (1, 0, 0, 0)."""
    q = torch.randn(shape, generator=gen) * 0.1
    q[..., 0] += 1
    return q / q.norm(dim=-1, keepdim=True)


# name -> (trailing shape, sampler); surfel tensors are [B, N, ...].
SCENE_RECIPE = {
    "common": (
        ("means", (3,), _means),
        ("quaternions", (4,), _near_identity_rotations),
        ("scales", (2,), _constant(0.025)),
        ("opacities", (), _constant(0.3)),
    ),
    "classic": (
        ("colors", (3,), _uniform(0.0, 1.0)),
        ("secondary_colors", (3,), _uniform(0.0, 1.0)),
        ("frequency_weights", (4,), _constant(0.25)),
        ("frequency_magnitudes", (4,), _constant(1.0)),
        ("phases", (4,), _constant(0.0)),
    ),
    "neural": (
        ("input_weights", (6, 5), _uniform(-1 / 5, 1 / 5)),
        ("input_biases", (6,), _uniform(-1 / 5, 1 / 5)),
        ("output_weights", (3, 6), _uniform(-1 / 30, 1 / 30)),
        ("output_biases", (3,), _uniform(-0.1, 0.1)),
    ),
}


def cameras(work: Workload) -> dict[str, torch.Tensor]:
    """Identity views shifted along x over [-0.2, 0.2], pinhole intrinsics
    with focal length 0.8 x the image size and the principal point at the
    image centre, and a 0.05 grey background."""
    b, c = work.num_scenes, work.num_cameras
    views = torch.eye(4).repeat(b, c, 1, 1)
    if c > 1:
        views[..., 0, 3] = torch.linspace(-0.2, 0.2, c)
    w, h = work.image_width, work.image_height
    K = torch.tensor([[0.8 * w, 0.0, (w - 1) / 2], [0.0, 0.8 * h, (h - 1) / 2], [0, 0, 1.0]])
    return {"view_matrices": views, "intrinsics": K.repeat(b, c, 1, 1),
            "backgrounds": torch.full((b, c, 3), 0.05)}


def synthesize(work: Workload, method: str, device: torch.device) -> dict[str, torch.Tensor]:
    """The benchmark scene of one method, outside every timed region: surfel
    tensors from SCENE_RECIPE (optimised, requires_grad), then the cameras."""
    gen = torch.Generator().manual_seed(work.seed)
    batch = (work.num_scenes, work.num_primitives)
    scene = {}
    for name, trailing, sample in SCENE_RECIPE["common"] + SCENE_RECIPE[method]:
        scene[name] = sample(gen, batch + trailing)
    scene.update(cameras(work))
    return {name: value.to(device).contiguous().requires_grad_(name not in CAMERA_INPUTS)
            for name, value in scene.items()}


# --------------------------------------------------------------------------
# Strategies: one way each of rendering all images of a scene.


def _all_maps(result) -> torch.Tensor:
    rgb, alpha, meta = result
    return torch.cat((rgb, alpha, *(meta[key] for key in MAP_OUTPUTS)), -1)


class Strategy:
    """Renders every (scene, camera) image of a scene: maps [B, C, H, W, 9]."""

    name = ""

    def __init__(self, work: Workload, method: str) -> None:
        self.render = rasterize_gabors if method == "classic" else rasterize_neural_gabors
        self.options = dict(width=work.image_width, height=work.image_height,
                            validate=not work.skip_validation)

    def maps(self, scene: dict) -> torch.Tensor:
        raise NotImplementedError


class Fused(Strategy):
    """All scenes and cameras in one call, dense or packed."""

    def __init__(self, work: Workload, method: str, packed: bool) -> None:
        super().__init__(work, method)
        self.packed = packed
        self.name = "fused_packed" if packed else "fused_dense"

    def maps(self, scene: dict) -> torch.Tensor:
        return _all_maps(self.render(**scene, packed=self.packed, **self.options))


class PerView(Strategy):
    """One call per (scene, camera) image, stacked afterwards."""

    name = "single_view_loop"

    def __init__(self, work: Workload, method: str) -> None:
        super().__init__(work, method)
        self.shape = (work.num_scenes, work.num_cameras)

    def maps(self, scene: dict) -> torch.Tensor:
        images = []
        for s in range(self.shape[0]):
            for c in range(self.shape[1]):
                view = {name: (value[s, c:c + 1] if name in CAMERA_INPUTS else value[s])
                        for name, value in scene.items()}
                view = {name: value.contiguous() for name, value in view.items()}
                images.append(_all_maps(self.render(**view, **self.options))[0])
        return torch.stack(images).unflatten(0, self.shape)


def strategies(work: Workload, method: str) -> dict[str, Strategy]:
    """Every implementation, keyed by its report name, loop first."""
    made = [PerView(work, method), Fused(work, method, False), Fused(work, method, True)]
    return {strategy.name: strategy for strategy in made}


def objective(maps: torch.Tensor) -> torch.Tensor:
    """The scalar every implementation is timed on: the mean square of all
    nine channels."""
    return maps.square().mean()


# --------------------------------------------------------------------------
# Parity gate


class ParityError(AssertionError):
    """A fused implementation differs from the per-camera loop."""


def _gradient_error(actual: torch.Tensor, expected: torch.Tensor) -> tuple[float, float]:
    """(largest elementwise error, error norm), both relative to the
    expected tensor's largest element and norm."""
    scale = float(expected.abs().max()) if expected.numel() else 0.0
    diff = (actual - expected).abs()
    elementwise = float((diff - GRADIENT_TOLERANCE * expected.abs()).clamp_min(0).max()
                        ) / scale if scale and diff.numel() else 0.0
    norm = float(expected.norm())
    return elementwise, float(diff.norm()) / norm if norm else float(diff.norm())


def parity_gate(scene: dict, candidates: dict[str, Strategy], baseline: str) -> dict:
    """Compare every strategy with ``baseline`` on maps and on the gradients
    of ``objective``; raise ParityError naming the worst differences, or
    return them (one entry per compared strategy)."""
    parameters = {name: value for name, value in scene.items() if value.requires_grad}

    def evaluate(strategy):
        maps = strategy.maps(scene)
        grads = torch.autograd.grad(objective(maps), list(parameters.values()))
        return maps.detach(), dict(zip(parameters, grads))

    reference_maps, reference_grads = evaluate(candidates[baseline])
    record = {}
    for name, strategy in candidates.items():
        if name == baseline:
            continue
        maps, grads = evaluate(strategy)
        excess = ((maps - reference_maps).abs()
                  - (MAP_ATOL + MAP_RTOL * reference_maps.abs())).clamp_min(0)
        worst_grads = {key: _gradient_error(grads[key], reference_grads[key]) for key in grads}
        record[name] = {
            "max_map_error": float((maps - reference_maps).abs().max()),
            "map_excess": float(excess.max()),
            "max_gradient_error": max((e for e, _ in worst_grads.values()), default=0.0),
            "max_gradient_norm_error": max((n for _, n in worst_grads.values()), default=0.0),
        }
        failures = []
        if record[name]["map_excess"] > 0:
            failures.append(f"maps differ by up to {record[name]['max_map_error']:.3e}")
        for key, (element, norm) in worst_grads.items():
            if element > GRADIENT_TOLERANCE or norm > GRADIENT_TOLERANCE:
                failures.append(f"{key} gradient error {element:.3e} (elementwise, of max) / "
                                f"{norm:.3e} (norm)")
        if failures:
            raise ParityError(f"{name} differs from {baseline}: " + "; ".join(failures))
    return record


# --------------------------------------------------------------------------
# Measurement


def _clear_gradients(scene: dict) -> Callable[[], None]:
    def clear():
        for value in scene.values():
            value.grad = None
    return clear


def measure(scene: dict, strategy: Strategy, work: Workload) -> dict:
    """Mean forward (render + loss) and backward milliseconds over the
    measured steps, and the peak memory they allocated."""

    def step(clock):
        clock.mark("start")
        loss = objective(strategy.maps(scene))
        clock.mark("forward")
        loss.backward()
        clock.mark("backward")

    clear = _clear_gradients(scene)
    clear()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    samples = time_phases(step, work.warmup_iterations, work.measurement_iterations, clear)
    forward, backward = mean(samples["forward"]), mean(samples["backward"])
    return {
        "implementation": strategy.name,
        "forward_ms": forward,
        "backward_ms": backward,
        "forward_backward_ms": forward + backward,
        "images_per_second": work.images * 1000.0 / (forward + backward),
        "peak_allocated_memory_mb": torch.cuda.max_memory_allocated() / 1e6,
    }


def kernel_split(scene: dict, strategy: Strategy, work: Workload) -> dict:
    """Per-family kernel milliseconds per step from the library's HIP-event
    counters, in a pass of its own (the events add host work)."""
    clear = _clear_gradients(scene)
    _native.profile_enable(True)
    try:
        for _ in range(work.profile_iterations):
            clear()
            objective(strategy.maps(scene)).backward()
        torch.cuda.synchronize()
        families = {family: _native.profile_read(family)[0] / work.profile_iterations
                    for family in _native.PROFILE_FAMILIES}
    finally:
        _native.profile_enable(False)
    forward, backward = families["render_forward"], families["render_backward"]
    if forward <= 0 or backward <= 0:
        raise RuntimeError("the kernel counters recorded no compositor launches")
    return {"forward_kernel_ms": forward, "backward_kernel_ms": backward,
            "other_cuda_kernel_ms": sum(families.values()) - forward - backward,
            "kernels_ms": families}


# --------------------------------------------------------------------------
# Report


def environment() -> dict:
    revision = subprocess.run(["git", "rev-parse", "HEAD"], capture_output=True, text=True,
                              cwd=Path(__file__).resolve().parent)
    return {
        "gpu": torch.cuda.get_device_name(),
        "torch": torch.__version__,
        "cuda": torch.version.cuda,
        "hip": torch.version.hip,
        "python": platform.python_version(),
        "revision": revision.stdout.strip() if revision.returncode == 0 else None,
    }


def run(argv=None) -> dict:
    """Parity gate, then timing of every implementation; the report is
    returned and, with --output-json, written."""
    work, output = parse_workload(argv)
    device = torch.device("cuda", torch.cuda.current_device())
    report = {
        "environment": environment(),
        "workload": asdict(work),
        "timing": "HIP events on the launch stream; forward covers rendering, autograd graph "
                  "construction and the scalar loss, backward the whole reverse pass",
        "profiling": "optional separate pass over the library's per-family HIP-event kernel "
                     "counters",
        "memory": "peak PyTorch-allocated device memory over the measured steps, decimal MB, "
                  "inputs and autograd state included",
        "parity": {},
        "results": [],
    }
    for method in work.methods:
        scene = synthesize(work, method, device)
        candidates = strategies(work, method)
        report["parity"][method] = parity_gate(scene, candidates, "single_view_loop")
        loop_ms = None
        for strategy in candidates.values():
            row = measure(scene, strategy, work)
            if work.profile_iterations:
                row.update(kernel_split(scene, strategy, work))
            loop_ms = loop_ms if loop_ms is not None else row["forward_backward_ms"]
            row["method"] = method
            row["speedup_vs_single_view_loop"] = loop_ms / row["forward_backward_ms"]
            report["results"].append(row)
            print(f"[{method}/{row['implementation']}] fwd {row['forward_ms']:.3f} ms + bwd "
                  f"{row['backward_ms']:.3f} ms = {row['forward_backward_ms']:.3f} ms, "
                  f"{row['images_per_second']:.0f} img/s, "
                  f"x{row['speedup_vs_single_view_loop']:.2f} vs the per-camera loop",
                  flush=True)
        del scene
    if output is not None:
        output.parent.mkdir(parents=True, exist_ok=True)
        output.write_text(json.dumps(report, indent=2) + "\n")
    return report


if __name__ == "__main__":
    run()
