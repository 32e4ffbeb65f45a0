"""Deterministic scenes shared by the tests (CPU tensors).

`make_inputs` restates the reference test fixture (tests/test_rendering.py:
11-48): overlapping tilted surfels inside one 9x9 tile, cameras shifted along
x, all inputs differentiable. Values are drawn from a CPU generator.
"""

from __future__ import annotations

import math

import numpy as np

import torch

NEURAL_FIELDS = (("input_weights", (6, 5)), ("input_biases", (6,)),
                 ("output_weights", (3, 6)), ("output_biases", (3,)))
CLASSIC_FIELDS = ("colors", "secondary_colors", "frequency_weights", "frequency_magnitudes",
                  "phases")
OUTPUT_KEYS = ("accumulated_depth", "normals", "distortion")


def make_inputs(method, scenes=1, cameras=2, primitives=3, seed=7):
    g = torch.Generator().manual_seed(seed)
    means = torch.randn(scenes, primitives, 3, generator=g) * 0.08
    means[..., 2] = torch.linspace(2.4, 3.5, primitives)
    quats = torch.tensor([1.0, 0.08, -0.05, 0.02])
    quats = (quats / quats.norm()).expand(scenes, primitives, 4).clone()
    views = torch.eye(4).expand(scenes, cameras, 4, 4).clone()
    views[..., 0, 3] = torch.linspace(-0.03, 0.04, cameras)
    K = torch.tensor([[16.0, 0.0, 4.0], [0.0, 17.0, 4.0], [0.0, 0.0, 1.0]])
    values = dict(
        means=means,
        quaternions=quats,
        scales=torch.full((scenes, primitives, 2), 0.37),
        opacities=torch.full((scenes, primitives), 0.32),
        view_matrices=views,
        intrinsics=K.expand(scenes, cameras, 3, 3).clone(),
        backgrounds=torch.full((scenes, cameras, 3), 0.13),
    )
    if method == "classic":
        values.update(
            colors=torch.rand(scenes, primitives, 3, generator=g),
            secondary_colors=torch.rand(scenes, primitives, 3, generator=g),
            frequency_weights=torch.full((scenes, primitives, 4), 0.25),
            frequency_magnitudes=torch.full((scenes, primitives, 4), 0.4),
            phases=torch.rand(scenes, primitives, 4, generator=g),
        )
    else:
        for name, shape in NEURAL_FIELDS:
            values[name] = torch.randn(scenes, primitives, *shape, generator=g) * 0.08
    return values


def random_scene(method, scenes=1, cameras=1, n=64, width=32, height=32, seed=0, sh=None,
                 focal=40.0, magnitudes=2.0):
    """Random surfels in front of identity-ish cameras covering a small image."""
    g = torch.Generator().manual_seed(seed)
    means = torch.cat(
        [torch.rand(scenes, n, 2, generator=g) * 2 - 1, torch.rand(scenes, n, 1, generator=g) * 2 + 2],
        -1,
    )
    quats = torch.randn(scenes, n, 4, generator=g)
    quats = quats / quats.norm(dim=-1, keepdim=True)
    scales = torch.exp(torch.rand(scenes, n, 2, generator=g) * math.log(10) + math.log(0.03))
    views = torch.eye(4).expand(scenes, cameras, 4, 4).clone()
    views[..., 0, 3] = torch.linspace(-0.1, 0.1, cameras) if cameras > 1 else 0.0
    K = torch.tensor([[focal, 0.0, (width - 1) / 2], [0.0, focal, (height - 1) / 2], [0, 0, 1.0]])
    values = dict(
        means=means, quaternions=quats, scales=scales,
        opacities=torch.rand(scenes, n, generator=g) * 0.8 + 0.1,
        view_matrices=views, intrinsics=K.expand(scenes, cameras, 3, 3).clone(),
        backgrounds=torch.rand(scenes, cameras, 3, generator=g),
    )
    if method == "classic":
        shape = (3,) if sh is None else ((sh + 1) ** 2, 3)
        weights = torch.rand(scenes, n, 4, generator=g)
        values.update(
            colors=torch.rand(scenes, n, *shape, generator=g),
            secondary_colors=torch.rand(scenes, n, *shape, generator=g),
            frequency_weights=weights / weights.sum(-1, keepdim=True),
            frequency_magnitudes=torch.rand(scenes, n, 4, generator=g) * magnitudes,
            phases=torch.rand(scenes, n, 4, generator=g) * 2 * math.pi,
        )
    else:
        values.update(
            input_weights=(torch.rand(scenes, n, 6, 5, generator=g) * 2 - 1) / 5,
            input_biases=torch.zeros(scenes, n, 6),
            output_weights=(torch.rand(scenes, n, 3, 6, generator=g) * 2 - 1) / 30,
            output_biases=torch.zeros(scenes, n, 3),
        )
    return values


def maps_from_result(result):
    """Every differentiable output of the public API as one [..., 9] tensor."""
    rgb, alpha, meta = result
    return torch.cat((rgb, alpha, *(meta[k] for k in OUTPUT_KEYS)), -1)


def _rotation_rodrigues(q: torch.Tensor) -> torch.Tensor:
    """R = I + 2 w [v]x + 2 [v]x^2 for a unit quaternion (w, v)."""
    q = q / q.norm()
    w, v = q[0], q[1:]
    zero = torch.zeros((), dtype=q.dtype)
    cross = torch.stack([
        torch.stack([zero, -v[2], v[1]]),
        torch.stack([v[2], zero, -v[0]]),
        torch.stack([-v[1], v[0], zero]),
    ])
    return torch.eye(3, dtype=q.dtype) + 2 * w * cross + 2 * cross @ cross


def _surfel_samples(method, v, scene, camera, i, px, py):
    """Alpha, depth, colour, normal of surfel i at every pixel (float64)."""
    view, K = v["view_matrices"][scene, camera], v["intrinsics"][scene, camera]
    R = _rotation_rodrigues(v["quaternions"][scene, i])
    centre = view[:3, :3] @ v["means"][scene, i] + view[:3, 3]
    axes = view[:3, :3] @ (R[:, :2] * v["scales"][scene, i])
    T = K @ torch.cat((axes, centre[:, None]), -1)
    # Ray through pixel (px, py) meets the plane where x*T2 - T0 and y*T2 - T1
    # both vanish on (u, v, 1): a 2x2 linear system per pixel.
    row_x = px[..., None] * T[2] - T[0]
    row_y = py[..., None] * T[2] - T[1]
    system = torch.stack((row_x[..., :2], row_y[..., :2]), -2)
    uv = torch.linalg.solve(system, -torch.stack((row_x[..., 2], row_y[..., 2]), -1))
    bound = T.new_tensor([9.0, 9.0, -1.0])
    f = bound / (bound * T[2] ** 2).sum()
    centre_px = (f * T[:2] * T[2]).sum(-1)
    rho_surface = (uv**2).sum(-1)
    rho_screen = 2 * ((centre_px - torch.stack((px, py), -1)) ** 2).sum(-1)
    depth = (uv * T[2, :2]).sum(-1) + T[2, 2]
    if method == "classic":
        depth = torch.where(rho_surface <= rho_screen, depth, T[2, 2])
    alpha = v["opacities"][scene, i] * torch.exp(-0.5 * torch.minimum(rho_surface, rho_screen))
    alpha = alpha.clamp_max(0.99)
    if method == "classic":
        phi = torch.arange(4, dtype=torch.float64) * (math.pi / 4)
        projection = uv[..., 0:1] * phi.cos() + uv[..., 1:2] * phi.sin()
        wave = torch.cos(2 * math.pi * v["frequency_magnitudes"][scene, i] * projection
                         + v["phases"][scene, i])
        mix = v["frequency_weights"][scene, i]
        first = (mix * (1 + wave)).sum(-1, keepdim=True) / 2
        second = (mix * (1 - wave)).sum(-1, keepdim=True) / 2
        color = first * v["colors"][scene, i] + second * v["secondary_colors"][scene, i]
    else:
        eye = -view[:3, :3].T @ view[:3, 3]
        toward = v["means"][scene, i] - eye
        toward = toward / toward.norm()
        features = torch.cat((uv / 3, toward.expand(*uv.shape[:-1], 3)), -1)
        hidden = torch.sin(30 * (features @ v["input_weights"][scene, i].T + v["input_biases"][scene, i]))
        color = torch.sigmoid(hidden @ v["output_weights"][scene, i].T + v["output_biases"][scene, i])
    normal = view[:3, :3] @ R[:, 2]
    if -(normal * centre).sum() <= 0:
        normal = -normal
    return alpha, depth, color, normal


def pixel_reference(method, values, width=9, height=9, near=0.2, far=100.0):
    """Per-pixel float64 compositor that solves the ray/plane system directly.

    Independent of the kernels' cross-product form (the local coordinates
    solve a 2x2 system with torch.linalg.solve, as the reference's own test
    oracle does, tests/test_rendering.py:64-171) and of both rotation forms
    used elsewhere (Rodrigues form here). Surfels are composited in list
    order, so it matches the rasterizer only for single-tile scenes whose
    surfels are sorted by depth and stay inside their tile bounds.
    """
    v = {k: t.double() for k, t in values.items()}
    py, px = torch.meshgrid(torch.arange(height, dtype=torch.float64),
                            torch.arange(width, dtype=torch.float64), indexing="ij")
    S, N = v["means"].shape[:2]
    C = v["view_matrices"].shape[1]
    mscale = far / (far - near)
    images = []
    for scene in range(S):
        for camera in range(C):
            transmittance = torch.ones_like(px)
            rgb = torch.zeros(height, width, 3, dtype=torch.float64)
            normals = torch.zeros(height, width, 3, dtype=torch.float64)
            depth_sum, distortion = torch.zeros_like(px), torch.zeros_like(px)
            first_moment, second_moment = torch.zeros_like(px), torch.zeros_like(px)
            finished = torch.zeros_like(px, dtype=torch.bool)
            for i in range(N):
                alpha, depth, color, normal = _surfel_samples(method, v, scene, camera, i, px, py)
                visible = alpha >= 1 / 255
                finished = finished | (visible & (transmittance * (1 - alpha) < 1e-4))
                alpha = torch.where(visible & (depth >= near) & ~finished, alpha, 0)
                weight = transmittance * alpha
                m = mscale * (1 - near / depth)
                rgb = rgb + weight[..., None] * color
                depth_sum = depth_sum + weight * depth
                normals = normals + weight[..., None] * normal
                distortion = distortion + weight * (
                    m * m * (1 - transmittance) + second_moment - 2 * m * first_moment
                )
                first_moment = first_moment + weight * m
                second_moment = second_moment + weight * m * m
                transmittance = transmittance * (1 - alpha)
            rgb = rgb + transmittance[..., None] * v["backgrounds"][scene, camera]
            images.append(torch.cat((rgb, (1 - transmittance)[..., None], depth_sum[..., None],
                                     normals, distortion[..., None]), -1))
    return torch.stack(images).reshape(S, C, height, width, 9)


def fp32_conditioned(render, values, eps=3e-7, trials=3, atol=1e-5, rtol=1e-4,
                     return_worst=False, **options):
    """float64 oracle maps and a mask of the pixels that are well conditioned at
    float32 precision.

    A pixel is flagged when some of the `trials` random relative perturbations
    of size `eps` (about five float32 ulps) applied to every float input move
    its float64 output by more than atol + rtol*|value| in any channel:
    near-grazing ray/plane intersections (the reference's contract calls
    them ill-conditioned) and samples sitting on a discrete threshold
    (alpha = 1/255, the stop test, the surface/screen switch). No float32
    implementation, the reference's included, can match float64 there.
    `render(**values, **options)` must return the maps first. With
    `return_worst` the largest change of every output element under the
    perturbations is returned as well (the pixel's float64 sensitivity).
    """
    base = {k: v.detach().cpu().double() for k, v in values.items()}
    with torch.no_grad():
        maps = render(**base, **options)[0]
        worst = torch.zeros_like(maps)
        for trial in range(trials):
            g = torch.Generator().manual_seed(1000 + trial)
            noisy = {k: v * (1 + eps * torch.randn(v.shape, generator=g, dtype=torch.float64))
                     for k, v in base.items()}
            worst = torch.maximum(worst, (render(**noisy, **options)[0] - maps).abs())
    mask = ~(worst > atol + rtol * maps.abs()).any(-1)
    if return_worst:
        return maps, mask, worst
    return maps, mask


def plain_bar_pixels(maps, expected, atol=1e-5, rtol=1e-4):
    """Pixels whose every channel lies within atol + rtol * |expected| of the
    float64 `expected` maps (the north star's forward bar, no allowance)."""
    a = maps.detach().cpu().double()
    return ((a - expected).abs() <= atol + rtol * expected.abs()).all(-1)


def describe_mismatch(actual, expected):
    """Worst elements and norms of a comparison, for assertion messages."""
    a = actual.detach().cpu().double()
    e = expected.detach().cpu().double()
    diff = (a - e).abs()
    flat = int(diff.argmax()) if diff.numel() else 0
    index = tuple(int(i) for i in np.unravel_index(flat, diff.shape)) if diff.numel() else ()
    norm = float(e.norm()) or 1.0
    return (f"max |diff| {float(diff.max()) if diff.numel() else 0:.3e} at {index} "
            f"(actual {float(a.reshape(-1)[flat]) if diff.numel() else 0:.6e}, "
            f"expected {float(e.reshape(-1)[flat]) if diff.numel() else 0:.6e}); "
            f"max |expected| {float(e.abs().max()) if e.numel() else 0:.3e}; "
            f"relative norm error {float((a - e).norm()) / norm:.3e}")


def assert_gradients_close(actual, expected, name, sensitivity=None, rel_norm=1e-3, elem=1e-3,
                           rtol=1e-3, factor=4.0):
    """Gradient parity as the north star states it - within 1e-3 relative.

    Per element: |a - e| <= elem * max|e| + rtol * |e| + factor * sensitivity
    (float32 atomic sums of terms that cancel carry absolute rounding error;
    `sensitivity` is the float64 gradient's own change under float32-sized
    input perturbations, see oracle_reference). Per tensor: the norm of the
    error over the well-conditioned elements (sensitivity <= 1e-4 max|e|) is
    at most `rel_norm` times the tensor's norm.
    """
    a = actual.detach().cpu().double()
    e = expected.detach().cpu().double()
    scale = float(e.abs().max()) if e.numel() else 0.0
    sens = torch.zeros_like(e) if sensitivity is None else sensitivity.detach().cpu().double()
    well = sens <= 1e-4 * scale
    diff = a - e
    norm_ok = float(diff[well].norm()) <= rel_norm * float(e.norm()) + 1e-12
    elem_ok = bool((diff.abs() <= elem * scale + rtol * e.abs() + factor * sens + 1e-12).all())
    ill = 1.0 - float(well.double().mean()) if e.numel() else 0.0
    assert norm_ok and elem_ok, (
        f"{name}: {describe_mismatch(a, e)}; well-conditioned error norm / tensor norm "
        f"{float(diff[well].norm()) / (float(e.norm()) or 1.0):.3e}; "
        f"ill-conditioned share {ill:.3f}"
    )
    return 1.0 - ill


def oracle_reference(render, values, weights, eps=3e-7, trials=3, **options):
    """float64 oracle maps and gradients of sum(maps * weights), with the
    largest change of every gradient element under `trials` random relative
    input perturbations of size `eps` (about five float32 ulps)."""
    names = list(values)

    def run(tensors):
        leaves = {k: t.detach().cpu().double().requires_grad_() for k, t in tensors.items()}
        maps = render(**leaves, **options)[0]
        out = torch.autograd.grad((maps * weights.double()).sum(), list(leaves.values()),
                                  allow_unused=True)
        return maps.detach(), [torch.zeros_like(l) if g is None else g for g, l in zip(out, leaves.values())]

    maps, grads = run(values)
    sensitivity = [torch.zeros_like(g) for g in grads]
    base = {k: v.detach().cpu().double() for k, v in values.items()}
    for trial in range(trials):
        gen = torch.Generator().manual_seed(3000 + trial)
        noisy = {k: v * (1 + eps * torch.randn(v.shape, generator=gen, dtype=torch.float64))
                 for k, v in base.items()}
        _, other = run(noisy)
        sensitivity = [torch.maximum(s, (o - g).abs()) for s, o, g in zip(sensitivity, other, grads)]
    return maps, dict(zip(names, grads)), dict(zip(names, sensitivity))


def perturbation_sensitivity(function, inputs, eps=3e-7, trials=3, seed=2000):
    """Largest change of each float64 output of `function(*inputs)` under
    `trials` random relative input perturbations of size `eps` (about five
    float32 ulps): the error any float32 evaluation can be expected to carry."""
    base = [t.detach().cpu().double() for t in inputs]
    with torch.no_grad():
        reference = function(*base)
        reference = reference if isinstance(reference, (tuple, list)) else [reference]
        worst = [torch.zeros_like(r, dtype=torch.float64) for r in reference]
        for trial in range(trials):
            g = torch.Generator().manual_seed(seed + trial)
            noisy = [t * (1 + eps * torch.randn(t.shape, generator=g, dtype=torch.float64)) for t in base]
            out = function(*noisy)
            out = out if isinstance(out, (tuple, list)) else [out]
            worst = [torch.maximum(w, (o.double() - r.double()).abs()) for w, o, r in zip(worst, out, reference)]
    return worst
