"""The BASELINE workloads: seeded synthetic scenes of the five benchmark
configurations, the benchmark objective and a closure running one
forward + loss + backward step through the public API.

Scenes are generated on the CPU with a seeded ``torch.Generator`` (seed =
config index unless given), so every device sees the same bits. The
distributions are BASELINE.json's ``configs``; the objective is the
reference benchmark's mean of squares over the listed map channels
(benchmarks/benchmark_rasterization.py:80-82, 133).
"""

from __future__ import annotations

import math

import torch

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


class MeanOfSquares(torch.autograd.Function):
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


def loss(rgb, alpha, meta, channels):
    """Mean of squares of the first `channels` map channels in the reference
    benchmark's order - rgb, alpha, depth, normals, distortion - its objective
    ``torch.cat(maps, -1).square().mean()`` (benchmarks/
    benchmark_rasterization.py:80-82, 133).

    Same value and gradient, less glue: a mean of squares does not depend on
    the order or grouping of the elements, so each group enters as it is
    (`MeanOfSquares`). Groups past `channels` are left out rather than
    sliced off (a slice adds a zero-filled full-size gradient).
    """
    return MeanOfSquares.apply(*loss_groups(rgb, alpha, meta, channels))


def loss_groups(rgb, alpha, meta, channels):
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


def reference_loss(rgb, alpha, meta, channels):
    """The reference benchmark's objective written as it is there: the maps
    concatenated along the channel axis, the first `channels` channels kept,
    then ``.square().mean()`` (benchmarks/benchmark_rasterization.py:80-82,
    133). The concatenation copies every map element and its backward
    slices the gradient back into the five groups."""
    maps = torch.cat((rgb, alpha, meta["accumulated_depth"], meta["normals"],
                      meta["distortion"]), -1)
    return maps[..., :channels].square().mean()


OBJECTIVES = {"fused": loss, "reference": reference_loss}


def prepare(index: int, device, validate: bool, objective: str = "fused"):
    """Seeded inputs of one config on the device and a closure running one
    fwd+bwd step on them through the public API. `objective` picks the loss
    expression (OBJECTIVES): both give the same value and gradient."""
    from .rendering import rasterize_gabors, rasterize_neural_gabors

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
    objective_fn = OBJECTIVES[objective]

    def step():
        for p in params:
            p.grad = None
        rgb, alpha, meta = renderer(**values, **options)
        objective_fn(rgb, alpha, meta, cfg["channels"]).backward()
        return meta

    return cpu_values, values, renderer, options, step
