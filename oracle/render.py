"""End-to-end oracle render (reference: rendering.py:241-400, minus validation).

Projection, SH, record layout, packing, binning and compositing as in the
reference, all differentiable through torch autograd on the CPU.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import binning
from .composite import composite
from .projection import project
from .sh import sh_colors

_NEURAL_SHAPES = ((6, 5), (6,), (3, 6), (3,))


def records(means, quaternions, scales, opacities, appearance, view_matrices, intrinsics,
            width, height, packed=False, near_plane=0.2, far_plane=100.0, neural=False,
            sh_degree=None, radii=None):
    """Compositor inputs of one call: a dict with geometry [Q,17], appearance
    rows, opacity rows, primitive/image ids, radii [Q], selected pair indices,
    projected means and dense radii. ``radii`` overrides the projected radii."""
    batch = tuple(means.shape[:-2])
    n = means.shape[-2]
    cameras = view_matrices.shape[-3]
    scenes = math.prod(batch)
    T, xy, normals, directions, projected_radii = project(
        means.reshape(scenes, n, 3),
        quaternions.reshape(scenes, n, 4),
        scales.reshape(scenes, n, 2),
        view_matrices.reshape(scenes, cameras, 4, 4),
        intrinsics.reshape(scenes, cameras, 3, 3),
        width, height, near_plane, far_plane,
    )
    if radii is not None:
        projected_radii = radii.reshape(scenes, cameras, n).to(torch.int32).cpu()
    pairs = scenes * cameras * n
    if sh_degree is not None:
        k = (sh_degree + 1) ** 2
        colors = sh_colors(
            appearance[0].reshape(scenes, n, k, 3), appearance[1].reshape(scenes, n, k, 3),
            directions, sh_degree,
        )
        rest = [t.reshape(scenes, 1, n, 4).expand(scenes, cameras, n, 4) for t in appearance[2:]]
        rows = torch.cat([colors, *rest], -1).reshape(pairs, 18)
        opacity_rows = opacities.reshape(scenes, 1, n).expand(scenes, cameras, n).reshape(pairs)
        primitive_ids = torch.arange(pairs)
    else:
        shapes = _NEURAL_SHAPES if neural else ((3,), (3,), (4,), (4,), (4,))
        rows = torch.cat(
            [t.reshape(scenes, n, math.prod(s)) for t, s in zip(appearance, shapes)], -1
        ).reshape(scenes * n, 57 if neural else 18)
        opacity_rows = opacities.reshape(scenes * n)
        primitive_ids = torch.arange(scenes * n).reshape(scenes, 1, n).expand(scenes, cameras, n)
        primitive_ids = primitive_ids.reshape(pairs)
    image_ids = torch.arange(scenes * cameras).reshape(scenes, cameras, 1)
    image_ids = image_ids.expand(scenes, cameras, n).reshape(pairs)
    flat_radii = projected_radii.reshape(pairs)
    if packed:
        selected = torch.from_numpy(binning.pack_visible(flat_radii.numpy()))
    else:
        selected = torch.arange(pairs)
    projected_means = xy.reshape(pairs, 2)[selected]
    geometry = torch.cat(
        [
            T.reshape(pairs, 9)[selected],
            projected_means,
            normals.reshape(pairs, 3)[selected],
            directions.reshape(pairs, 3)[selected],
        ],
        -1,
    )
    return {
        "geometry": geometry,
        "appearance": rows,
        "opacities": opacity_rows,
        "primitive_ids": primitive_ids[selected],
        "image_ids": image_ids[selected],
        "radii": flat_radii[selected],
        "selected": selected,
        "projected_means": projected_means,
        "dense_radii": projected_radii,
        "batch": batch,
        "cameras": cameras,
        "n": n,
    }


def render(means, quaternions, scales, opacities, appearance, view_matrices, intrinsics,
           width, height, backgrounds=None, packed=False, near_plane=0.2, far_plane=100.0,
           neural=False, sh_degree=None, radii=None, lists=None, margins=None, taken=None,
           stopped=None):
    """Returns maps [..., C, H, W, 9], meta (as the reference) and the
    compositor's auxiliary outputs (point_list, ranges, state, contributors)."""
    rec = records(
        means, quaternions, scales, opacities, appearance, view_matrices, intrinsics, width,
        height, packed, near_plane, far_plane, neural, sh_degree, radii,
    )
    batch, cameras, n = rec["batch"], rec["cameras"], rec["n"]
    scenes = math.prod(batch)
    if backgrounds is None:
        backgrounds = means.new_zeros(batch + (cameras, 3))
    maps, point_list, ranges, state, contributors = composite(
        rec["geometry"], rec["appearance"], rec["opacities"], rec["primitive_ids"],
        rec["image_ids"], rec["radii"], backgrounds.reshape(scenes * cameras, 3), width, height,
        neural, near_plane, far_plane, lists=lists, margins=margins, taken=taken,
        stopped=stopped,
    )
    if margins is not None:
        margins["pixels"] = margins["pixels"].reshape(batch + (cameras, height, width))
    if stopped is not None:
        stopped["pixels"] = stopped["pixels"].reshape(batch + (cameras, height, width))
    maps = maps.reshape(batch + (cameras, height, width, 9))
    selected = rec["selected"]
    stride = max(n, 1)
    meta = {
        "radii": rec["radii"] if packed else rec["dense_radii"].reshape(batch + (cameras, n)),
        "projected_means": rec["projected_means"],
        "scene_ids": selected // (cameras * stride),
        "camera_ids": selected // stride % cameras,
        "primitive_ids": selected % stride,
        "packed": packed,
        "accumulated_depth": maps[..., 4:5],
        "normals": maps[..., 5:8],
        "distortion": maps[..., 8:9],
    }
    aux = {
        "point_list": point_list,
        "ranges": ranges,
        "state": state,
        "contributors": contributors,
        "records": rec,
    }
    return maps, meta, aux


def rasterize_gabors(means, quaternions, scales, opacities, colors, secondary_colors,
                     frequency_weights, frequency_magnitudes, phases, view_matrices, intrinsics,
                     width, height, **options):
    """Oracle counterpart of the public classic renderer: (maps, meta, aux)."""
    return render(
        means, quaternions, scales, opacities,
        (colors, secondary_colors, frequency_weights, frequency_magnitudes, phases),
        view_matrices, intrinsics, width, height, neural=False, **options,
    )


def rasterize_neural_gabors(means, quaternions, scales, opacities, input_weights, input_biases,
                            output_weights, output_biases, view_matrices, intrinsics, width,
                            height, **options):
    """Oracle counterpart of the public neural renderer: (maps, meta, aux)."""
    options.pop("sh_degree", None)
    return render(
        means, quaternions, scales, opacities,
        (input_weights, input_biases, output_weights, output_biases),
        view_matrices, intrinsics, width, height, neural=True, **options,
    )


def as_numpy(value):
    return value.detach().cpu().numpy() if isinstance(value, torch.Tensor) else np.asarray(value)
