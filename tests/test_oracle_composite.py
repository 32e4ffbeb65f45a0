"""Pins oracle/composite.py and oracle/render.py on the CPU (float64)."""

import math

import numpy as np
import pytest
import torch

from oracle import render as oracle_render
from scenes import _surfel_samples, make_inputs, pixel_reference

RENDER = {"classic": oracle_render.rasterize_gabors, "neural": oracle_render.rasterize_neural_gabors}


def oracle_maps(method, values, width=9, height=9, **options):
    values = dict(values)
    backgrounds = values.pop("backgrounds")
    maps, meta, aux = RENDER[method](**values, width=width, height=height,
                                     backgrounds=backgrounds, **options)
    return maps, meta, aux


def as64(values):
    return {k: v.double().requires_grad_() for k, v in values.items()}


# The oracle keeps the reference's float32 pi and frequency directions
# (cos(pi f / 4) with f = 2 is -4.4e-8, not 0); the pixel reference uses
# exact ones, so maps agree to ~1e-7 rather than to double rounding.
TOLERANCE = dict(atol=2e-7, rtol=1e-6)


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("scenes, cameras", [(1, 2), (2, 3)])
def test_oracle_matches_pixel_reference(method, packed, scenes, cameras):
    values = as64(make_inputs(method, scenes=scenes, cameras=cameras))
    actual, _, _ = oracle_maps(method, values, packed=packed)
    expected = pixel_reference(method, values)
    torch.testing.assert_close(actual, expected, **TOLERANCE)
    weights = torch.linspace(-0.4, 0.7, actual.numel(), dtype=torch.float64).reshape(actual.shape)
    grads = torch.autograd.grad((actual * weights).sum(), list(values.values()), retain_graph=True)
    expected_grads = torch.autograd.grad((expected * weights).sum(), list(values.values()))
    for name, a, e in zip(values, grads, expected_grads):
        torch.testing.assert_close(a, e, atol=2e-6, rtol=1e-5, msg=name)


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("opacity", [0.0, 1.0])
def test_opacity_cutoff_and_saturation(method, opacity):
    values = make_inputs(method, cameras=1, primitives=7)
    values["opacities"].fill_(0.85 if opacity == 1.0 else opacity)
    values["opacities"][..., 0] = opacity
    values["quaternions"].zero_()
    values["quaternions"][..., 0] = 1
    values["means"][..., :2] = 0
    values = as64(values)
    stopped = {}
    actual, _, aux = oracle_maps(method, values, stopped=stopped)
    torch.testing.assert_close(actual, pixel_reference(method, values), **TOLERANCE)
    if opacity == 1.0:
        # Alpha 0.99 then 0.85s: T goes 1 -> 1e-2 -> 1.5e-3 -> 2.25e-4; the
        # fourth would take it to 3.4e-5 < 1e-4, so exactly three contribute
        # at the centre pixel and the next stops it.
        assert int(aux["contributors"][0, 4, 4]) == 3
        assert bool(stopped["pixels"][0, 0, 4, 4])
        # The same three alone leave T = 2.25e-4 at the centre: the walk ends
        # with the list, not on the transmittance rule.
        first = {k: (v if k in ("view_matrices", "intrinsics", "backgrounds")
                     else v[:, :3].detach().clone().requires_grad_()) for k, v in values.items()}
        three = {}
        _, _, aux3 = oracle_maps(method, first, stopped=three)
        assert int(aux3["contributors"][0, 4, 4]) == 3
        assert not bool(three["pixels"].any())
    else:
        assert not bool(stopped["pixels"].any())


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_lowpass_and_batch_boundary(method):
    tiny = make_inputs(method, cameras=1, primitives=1)
    tiny["scales"].fill_(0.02)
    tiny["quaternions"].zero_()
    tiny["quaternions"][..., 0] = 1
    many = make_inputs(method, cameras=1, primitives=65)
    many["opacities"].fill_(0.03)
    for values in (tiny, many):
        values = as64(values)
        actual, _, _ = oracle_maps(method, values)
        torch.testing.assert_close(actual, pixel_reference(method, values), **TOLERANCE)


def test_single_surfel_closed_form():
    # Fronto-parallel surfel whose mean projects exactly on pixel (4, 4):
    # rho = 0 there, so alpha = min(0.99, o); magnitudes 0 make every wave
    # cos(phase), i.e. h1 = sum w (1 + cos phase) / 2.
    values = make_inputs("classic", cameras=1, primitives=1)
    values["means"][:] = torch.tensor([0.0, 0.0, 3.0])
    values["quaternions"][:] = torch.tensor([1.0, 0, 0, 0])
    values["view_matrices"][..., :3, 3] = 0.0
    values["frequency_magnitudes"].zero_()
    values["opacities"].fill_(0.6)
    values = as64(values)
    maps, meta, aux = oracle_maps("classic", values)
    px = maps[0, 0, 4, 4]
    phases, weights = values["phases"][0, 0], values["frequency_weights"][0, 0]
    h1 = (weights * (1 + phases.cos()) / 2).sum()
    h2 = (weights * (1 - phases.cos()) / 2).sum()
    color = h1 * values["colors"][0, 0] + h2 * values["secondary_colors"][0, 0]
    expected_rgb = 0.6 * color + 0.4 * values["backgrounds"][0, 0]
    torch.testing.assert_close(px[:3], expected_rgb.detach())
    torch.testing.assert_close(px[3], torch.tensor(0.6, dtype=torch.float64))
    torch.testing.assert_close(px[4], torch.tensor(0.6 * 3.0, dtype=torch.float64))
    torch.testing.assert_close(px[5:8], torch.tensor([0.0, 0.0, -0.6], dtype=torch.float64))
    assert float(px[8]) == 0.0  # one surfel: no distortion
    assert int(aux["contributors"][0, 4, 4]) == 1
    assert int(meta["radii"][0, 0, 0]) > 0


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_distortion_is_pairwise_sum(method):
    values = as64(make_inputs(method, cameras=1, primitives=5))
    maps, _, _ = oracle_maps(method, values)
    near, far = 0.2, 100.0
    py, px = torch.meshgrid(torch.arange(9.0, dtype=torch.float64), torch.arange(9.0, dtype=torch.float64), indexing="ij")
    transmittance = torch.ones_like(px)
    weights, ms = [], []
    for i in range(5):
        alpha, depth, _, _ = _surfel_samples(method, {k: v.detach() for k, v in values.items()}, 0, 0, i, px, py)
        alpha = torch.where((alpha >= 1 / 255) & (depth >= near), alpha, 0)
        weights.append(transmittance * alpha)
        ms.append(far / (far - near) * (1 - near / depth))
        transmittance = transmittance * (1 - alpha)
    pairwise = sum(weights[i] * weights[j] * (ms[i] - ms[j]) ** 2 for i in range(5) for j in range(i))
    torch.testing.assert_close(maps[0, 0, ..., 8].detach(), pairwise, atol=1e-12, rtol=1e-9)


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_oracle_gradients_match_finite_differences(method):
    values = as64(make_inputs(method, cameras=2, primitives=3))
    names = ["means", "scales", "opacities", "quaternions", "view_matrices", "intrinsics",
             "phases" if method == "classic" else "input_biases"]
    weights = torch.linspace(-0.2, 0.4, 2 * 81 * 9, dtype=torch.float64).reshape(1, 2, 9, 9, 9)

    def objective():
        return (oracle_maps(method, values)[0] * weights).sum()

    grads = torch.autograd.grad(objective(), [values[n] for n in names])
    step = 1e-6
    for name, grad in zip(names, grads):
        value = values[name]
        flat = value.detach().view(-1)
        for index in range(0, flat.numel(), max(1, flat.numel() // 4)):
            original = float(flat[index])
            with torch.no_grad():
                flat[index] = original + step
                plus = float(objective())
                flat[index] = original - step
                minus = float(objective())
                flat[index] = original
            numeric = (plus - minus) / (2 * step)
            analytic = float(grad.reshape(-1)[index])
            assert abs(analytic - numeric) <= 1e-5 + 1e-5 * abs(numeric), (name, index, analytic, numeric)


def test_empty_and_invisible_scenes_are_background():
    for n, z in ((0, 3.0), (3, -2.0)):
        values = make_inputs("classic", primitives=n)
        if n:
            values["means"][..., 2] = z
        values = as64(values)
        maps, meta, aux = oracle_maps("classic", values)
        torch.testing.assert_close(maps[..., :3], values["backgrounds"][:, :, None, None, :].expand(1, 2, 9, 9, 3))
        assert maps[..., 3].count_nonzero() == 0
        assert len(aux["point_list"]) == 0


def _tile_quadrant_last(contributors, width, height):
    """Largest contributor count of every (tile, 8x8 quadrant): [tiles, 4]."""
    images = contributors.shape[0]
    tw, th = (width + 15) // 16, (height + 15) // 16
    out = np.zeros((images * tw * th, 4), dtype=np.int64)
    for image in range(images):
        for py in range(height):
            for px in range(width):
                tile = (image * th + py // 16) * tw + px // 16
                q = 2 * ((py % 16) >= 8) + ((px % 16) >= 8)
                out[tile, q] = max(out[tile, q], int(contributors[image, py, px]))
    return out


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_taken_quadrants_agree_with_contributors(method):
    from scenes import random_scene

    values = random_scene(method, cameras=2, n=48, width=40, height=24, seed=3)
    backgrounds = values.pop("backgrounds")
    taken = {}
    _, _, aux = RENDER[method](**values, width=40, height=24, backgrounds=backgrounds,
                               taken=taken)
    quadrants = taken["quadrants"]
    contributors = aux["contributors"].reshape(-1, 24, 40)
    lengths = aux["ranges"][:, 1] - aux["ranges"][:, 0]
    # Each pixel's last contributor was taken in its quadrant.
    tw = 3
    for image in range(contributors.shape[0]):
        for py in range(24):
            for px in range(40):
                c = int(contributors[image, py, px])
                if c:
                    tile = (image * 2 + py // 16) * tw + px // 16
                    q = 2 * ((py % 16) >= 8) + ((px % 16) >= 8)
                    assert quadrants[tile, c - 1] >> q & 1
    # A record taken in quadrant q lies within some pixel's contributors there,
    # and records beyond a tile's list are never taken.
    last = _tile_quadrant_last(contributors, 40, 24)
    tiles, longest = quadrants.shape
    position = np.arange(longest)
    for q in range(4):
        bit = (quadrants >> q) & 1
        assert not np.any(bit & (position[None, :] >= last[:, q:q + 1]))
    assert not np.any(quadrants & (position[None, :] >= lengths[:, None]))
    assert np.count_nonzero(quadrants) > 20


def test_taken_quadrants_closed_form():
    """One fronto-parallel surfel in a 16x16 image: a small one near pixel
    (3, 12) is taken only in quadrant 2 (x < 8, y >= 8); a large centred one
    in all four."""
    base = make_inputs("classic", scenes=1, cameras=1, primitives=1)
    base["quaternions"].zero_()
    base["quaternions"][..., 0] = 1
    base["intrinsics"][..., 0, 0] = 20.0
    base["intrinsics"][..., 1, 1] = 20.0
    base["intrinsics"][..., 0, 2] = 7.5
    base["intrinsics"][..., 1, 2] = 7.5
    base["opacities"].fill_(0.8)
    for (px, py, scale), expected in (((3.0, 12.0, 0.01), 0b0100), ((7.5, 7.5, 0.3), 0b1111)):
        values = dict(base)
        z = 3.0
        values["means"] = torch.tensor([[[(px - 7.5) * z / 20.0, (py - 7.5) * z / 20.0, z]]])
        values["scales"] = torch.full((1, 1, 2), scale)
        backgrounds = values.pop("backgrounds")
        taken = {}
        RENDER["classic"](**values, width=16, height=16, backgrounds=backgrounds, taken=taken)
        assert taken["quadrants"].tolist() == [[expected]]
