"""PyTorch custom operators over the HIP library: ``torch.ops.gabor_splatting.*``.

Importing this module registers, in the ``gabor_splatting`` namespace:

* ``rasterize_forward`` / ``rasterize_backward`` and ``evaluate_sh_forward`` /
  ``evaluate_sh_backward``: the four functions the reference binds into its
  ``_C`` module (src/gabor_splatting/csrc/bindings.cpp:5-10, signatures at
  csrc/rasterize.h:6-21), with the same arguments and outputs;
* ``rasterize_forward_bounded``: rasterize_forward into a point list of a
  fixed capacity, so every output shape follows from the inputs (no host
  read of the intersection count);
* ``project_forward`` / ``project_backward``, ``records_forward`` /
  ``records_backward``: the renderer's fused front end (projection, SH colours
  and compositor rows; rendering.py:176-238, 323-374 of the reference);
* ``pack_visible``, ``bin_tiles`` and ``sort_pairs``: compaction, binning
  (count, emit, sort, ranges; rasterize.cu:24-69, 459-501) and the radix
  sort, exposed separately as the reference's stages are.

Each operator has a schema, a fake (meta) kernel for FakeTensor tracing and
``torch.compile``, and, where it is differentiable, an autograd formula that
calls its backward operator. Sizes that depend on the data (the intersection
count M, the visible row count) are new dynamic sizes in the fake kernels.
The operators run on CUDA (HIP) tensors only: there is no CPU kernel, and a
CPU call raises. The C ABI (include/gabor_hip.h) stays underneath; the
operators are thin allocation-and-launch wrappers over it.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor
from torch.library import custom_op, get_ctx

from . import _native

NAMESPACE = "gabor_splatting"
_MAPS = 9


def _op(name: str):
    return custom_op(f"{NAMESPACE}::{name}", mutates_args=(), device_types="cuda")


def _tiles(images: int, width: int, height: int) -> int:
    tw, th = _native.tile_grid(width, height)
    return images * tw * th


def _empty(like: Tensor, shape, dtype=None) -> Tensor:
    return like.new_empty(shape, dtype=dtype or like.dtype)


# --------------------------------------------------------------------------
# Compositor (the reference's _C.rasterize_forward / rasterize_backward)


@_op("rasterize_forward")
def rasterize_forward(geometry: Tensor, appearance: Tensor, opacities: Tensor,
                      primitive_ids: Tensor, image_ids: Tensor, radii: Tensor,
                      backgrounds: Tensor, width: int, height: int, neural: bool,
                      near_plane: float, far_plane: float
                      ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """maps [I,H,W,9], point_list int32 [M], ranges int32 [I*tw*th, 2],
    state [I,H,W,3], contributors int32 [I,H,W] (rasterize.cu:426-503)."""
    maps, point_list, ranges, state, contributors = _native.rasterize_forward(
        geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds, width,
        height, neural, near_plane, far_plane)
    return maps, point_list, ranges, state, contributors


def _forward_outputs(geometry, backgrounds, width, height, points):
    images = backgrounds.size(0)
    return (_empty(geometry, (images, height, width, _MAPS)),
            _empty(geometry, (points,), torch.int32),
            _empty(geometry, (_tiles(images, width, height), 2), torch.int32),
            _empty(geometry, (images, height, width, 3)),
            _empty(geometry, (images, height, width), torch.int32))


@rasterize_forward.register_fake
def _(geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds, width,
      height, neural, near_plane, far_plane):
    return _forward_outputs(geometry, backgrounds, width, height, get_ctx().new_dynamic_size())


@_op("rasterize_forward_bounded")
def rasterize_forward_bounded(geometry: Tensor, appearance: Tensor, opacities: Tensor,
                              primitive_ids: Tensor, image_ids: Tensor, radii: Tensor,
                              backgrounds: Tensor, width: int, height: int, neural: bool,
                              near_plane: float, far_plane: float, capacity: int
                              ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """rasterize_forward into a point list of ``capacity`` entries, without a
    host synchronisation. The sixth output, int64 [2] on the device, holds
    the binning status bits (1: M exceeded the capacity, the maps are then
    incomplete; 2: a sort output failed its range check) and M."""
    _native._require(0 < capacity <= _native.INT_MAX, "invalid point-list capacity")
    found = {}

    def flags(overflow, total):
        found["status"] = torch.cat((overflow.long(), total.long()))

    maps, point_list, ranges, state, contributors = _native.rasterize_forward(
        geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds, width,
        height, neural, near_plane, far_plane, capacity=capacity, flags=flags)
    return maps, point_list, ranges, state, contributors, found["status"]


@rasterize_forward_bounded.register_fake
def _(geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds, width,
      height, neural, near_plane, far_plane, capacity):
    return (*_forward_outputs(geometry, backgrounds, width, height, capacity),
            _empty(geometry, (2,), torch.int64))


@_op("rasterize_backward")
def rasterize_backward(geometry: Tensor, appearance: Tensor, opacities: Tensor,
                       primitive_ids: Tensor, backgrounds: Tensor, point_list: Tensor,
                       ranges: Tensor, state: Tensor, contributors: Tensor, grad_maps: Tensor,
                       width: int, height: int, neural: bool, near_plane: float,
                       far_plane: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients of geometry, appearance, opacities and backgrounds
    (rasterize.cu:506-529)."""
    gg, ga, go, gb = _native.rasterize_backward(
        geometry, appearance, opacities, primitive_ids, backgrounds, point_list, ranges, state,
        contributors, grad_maps, width, height, neural, near_plane, far_plane)
    return gg, ga, go, gb


@rasterize_backward.register_fake
def _(geometry, appearance, opacities, primitive_ids, backgrounds, point_list, ranges, state,
      contributors, grad_maps, width, height, neural, near_plane, far_plane):
    return (torch.empty_like(geometry), torch.empty_like(appearance),
            torch.empty_like(opacities), torch.empty_like(backgrounds))


def _save_rasterize(ctx, inputs, output):
    geometry, appearance, opacities, primitive_ids, _, _, backgrounds = inputs[:7]
    width, height, neural, near_plane, far_plane = inputs[7:12]
    _, point_list, ranges, state, contributors = output[:5]
    ctx.save_for_backward(geometry, appearance, opacities, primitive_ids, backgrounds,
                          point_list, ranges, state, contributors)
    ctx.settings = (width, height, neural, near_plane, far_plane)
    ctx.extra_inputs = len(inputs) - 12


def _rasterize_grad(ctx, grad_maps, *_):
    saved = ctx.saved_tensors
    gg, ga, go, gb = torch.ops.gabor_splatting.rasterize_backward(
        *saved, grad_maps.contiguous(), *ctx.settings)
    return (gg, ga, go, None, None, None, gb) + (None,) * (5 + ctx.extra_inputs)


rasterize_forward.register_autograd(_rasterize_grad, setup_context=_save_rasterize)
rasterize_forward_bounded.register_autograd(_rasterize_grad, setup_context=_save_rasterize)


# --------------------------------------------------------------------------
# Spherical harmonics (the reference's _C.evaluate_sh_forward / backward)


@_op("evaluate_sh_forward")
def evaluate_sh_forward(first: Tensor, second: Tensor, directions: Tensor, degree: int) -> Tensor:
    """Both SH colours per (scene, camera, surfel): [S, C, N, 6]
    (spherical_harmonics.cu:106-122)."""
    return _native.evaluate_sh_forward(first, second, directions, degree)


@evaluate_sh_forward.register_fake
def _(first, second, directions, degree):
    return _empty(first, (*directions.shape[:3], 6))


@_op("evaluate_sh_backward")
def evaluate_sh_backward(first: Tensor, second: Tensor, directions: Tensor, grad_colors: Tensor,
                         degree: int) -> tuple[Tensor, Tensor, Tensor]:
    """Coefficient gradients summed over cameras and per-pair direction
    gradients (spherical_harmonics.cu:125-150)."""
    gf, gs, gd = _native.evaluate_sh_backward(first, second, directions, grad_colors, degree)
    return gf, gs, gd


@evaluate_sh_backward.register_fake
def _(first, second, directions, grad_colors, degree):
    return torch.empty_like(first), torch.empty_like(second), torch.empty_like(directions)


def _save_sh(ctx, inputs, output):
    first, second, directions, degree = inputs
    ctx.save_for_backward(first, second, directions)
    ctx.degree = degree


def _sh_grad(ctx, grad_colors):
    first, second, directions = ctx.saved_tensors
    gf, gs, gd = torch.ops.gabor_splatting.evaluate_sh_backward(
        first, second, directions, grad_colors.contiguous(), ctx.degree)
    return gf, gs, gd, None


evaluate_sh_forward.register_autograd(_sh_grad, setup_context=_save_sh)


# --------------------------------------------------------------------------
# Projection (project_surfaces, rendering.py:176-218 of the reference)


@_op("project_forward")
def project_forward(means: Tensor, quaternions: Tensor, scales: Tensor, view_matrices: Tensor,
                    intrinsics: Tensor, width: int, height: int, near_plane: float,
                    far_plane: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """transform [S,C,N,3,3], xy [S,C,N,2], normals [S,C,N,3], directions
    [S,C,N,3], radii int32 [S,C,N]."""
    return tuple(_native.project_forward(means, quaternions, scales, view_matrices, intrinsics,
                                         width, height, near_plane, far_plane))


@project_forward.register_fake
def _(means, quaternions, scales, view_matrices, intrinsics, width, height, near_plane,
      far_plane):
    pairs = (means.size(0), view_matrices.size(1), means.size(1))
    return (_empty(means, (*pairs, 3, 3)), _empty(means, (*pairs, 2)), _empty(means, (*pairs, 3)),
            _empty(means, (*pairs, 3)), _empty(means, pairs, torch.int32))


@_op("project_backward")
def project_backward(means: Tensor, quaternions: Tensor, scales: Tensor, view_matrices: Tensor,
                     intrinsics: Tensor, grad_transform: Optional[Tensor],
                     grad_xy: Optional[Tensor], grad_normals: Optional[Tensor],
                     grad_directions: Optional[Tensor]
                     ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of means, quaternions, scales, view matrices and intrinsics;
    a missing output gradient counts as zero."""
    return tuple(_native.project_backward(means, quaternions, scales, view_matrices, intrinsics,
                                          grad_transform, grad_xy, grad_normals,
                                          grad_directions))


@project_backward.register_fake
def _(means, quaternions, scales, view_matrices, intrinsics, grad_transform, grad_xy,
      grad_normals, grad_directions):
    return tuple(torch.empty_like(t) for t in (means, quaternions, scales, view_matrices,
                                                intrinsics))


def _save_project(ctx, inputs, output):
    ctx.save_for_backward(*inputs[:5])


def _project_grad(ctx, g_transform, g_xy, g_normals, g_directions, _g_radii):
    grads = torch.ops.gabor_splatting.project_backward(
        *ctx.saved_tensors, g_transform, g_xy, g_normals, g_directions)
    return (*grads, None, None, None, None)


project_forward.register_autograd(_project_grad, setup_context=_save_project)


# --------------------------------------------------------------------------
# Fused front end: projection + SH + compositor rows


@_op("records_forward")
def records_forward(means: Tensor, quaternions: Tensor, scales: Tensor,
                    opacities: Optional[Tensor],
                    view_matrices: Tensor, intrinsics: Tensor, first: Optional[Tensor],
                    second: Optional[Tensor], weights: Optional[Tensor],
                    magnitudes: Optional[Tensor], phases: Optional[Tensor], sh_degree: int,
                    width: int, height: int, near_plane: float, far_plane: float, packed: bool
                    ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                               Tensor, Tensor]:
    """Compositor rows for every visible (packed) or every (dense) pair.

    Outputs: geometry [Q,17], projected_means [Q,2], appearance [Q,18] and
    opacity_rows [Q] (with SH, sh_degree 0-3; [Q,0] and [0] with sh_degree
    -1), row_radii int32 [Q], primitive_ids int64 [Q], image_ids int64 [Q],
    meta_ids int64 [3,Q] (scene, camera, surfel of each row), dense_radii
    int32 [S,C,N], row_of_pair int32 [S*C*N] (each pair's row or -1; [0]
    when dense). Q = S*C*N dense, the visible count packed."""
    with_sh = sh_degree >= 0
    out = _native.records_forward(
        means, quaternions, scales, opacities, view_matrices, intrinsics,
        (first, second) if with_sh else None,
        (weights, magnitudes, phases) if with_sh else None,
        sh_degree if with_sh else None, width, height, near_plane, far_plane, packed)
    geometry = out["geometry"]
    rows = geometry.size(0)
    appearance = out["appearance"] if with_sh else geometry.new_empty((rows, 0))
    opacity_rows = out["opacity_rows"] if with_sh else geometry.new_empty((0,))
    meta_ids = torch.stack((out["scene_ids"], out["camera_ids"], out["surfel_ids"]))
    row_of_pair = out["row_of_pair"]
    if row_of_pair is None:
        row_of_pair = geometry.new_empty((0,), dtype=torch.int32)
    return (geometry, out["projected_means"], appearance, opacity_rows, out["row_radii"],
            out["primitive_ids"], out["image_ids"], meta_ids, out["dense_radii"], row_of_pair)


@records_forward.register_fake
def _(means, quaternions, scales, opacities, view_matrices, intrinsics, first, second, weights,
      magnitudes, phases, sh_degree, width, height, near_plane, far_plane, packed):
    pairs = means.size(0) * view_matrices.size(1) * means.size(1)
    rows = get_ctx().new_dynamic_size() if packed else pairs
    with_sh = sh_degree >= 0
    return (_empty(means, (rows, _native.GEOMETRY_SIZE)), _empty(means, (rows, 2)),
            _empty(means, (rows, 18 if with_sh else 0)), _empty(means, (rows if with_sh else 0,)),
            _empty(means, (rows,), torch.int32), _empty(means, (rows,), torch.int64),
            _empty(means, (rows,), torch.int64), _empty(means, (3, rows), torch.int64),
            _empty(means, (means.size(0), view_matrices.size(1), means.size(1)), torch.int32),
            _empty(means, (pairs if packed else 0,), torch.int32))


@_op("records_backward")
def records_backward(means: Tensor, quaternions: Tensor, scales: Tensor, view_matrices: Tensor,
                     intrinsics: Tensor, first: Optional[Tensor], second: Optional[Tensor],
                     sh_degree: int, row_of_pair: Optional[Tensor], geometry: Tensor,
                     grad_geometry: Optional[Tensor], grad_projected_means: Optional[Tensor],
                     grad_appearance: Optional[Tensor], grad_opacity_rows: Optional[Tensor]
                     ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                Tensor, Tensor, Tensor]:
    """Gradients of means, quaternions, scales, view matrices, intrinsics and
    (with SH; empty [0] tensors without) first, second, weights, magnitudes,
    phases and opacities. ``row_of_pair`` is records_forward's for packed
    rows, None for dense ones."""
    with_sh = sh_degree >= 0
    grads = _native.records_backward(
        means, quaternions, scales, view_matrices, intrinsics,
        (first, second) if with_sh else None, sh_degree if with_sh else None, row_of_pair,
        geometry, grad_geometry, grad_projected_means, grad_appearance if with_sh else None,
        grad_opacity_rows if with_sh else None)
    return tuple(g if g is not None else means.new_empty((0,)) for g in grads)


@records_backward.register_fake
def _(means, quaternions, scales, view_matrices, intrinsics, first, second, sh_degree,
      row_of_pair, geometry, grad_geometry, grad_projected_means, grad_appearance,
      grad_opacity_rows):
    base = tuple(torch.empty_like(t) for t in (means, quaternions, scales, view_matrices,
                                                intrinsics))
    if sh_degree < 0:
        return base + tuple(means.new_empty((0,)) for _ in range(6))
    shared = (means.size(0), means.size(1), 4)
    return base + (torch.empty_like(first), torch.empty_like(second), _empty(means, shared),
                   _empty(means, shared), _empty(means, shared),
                   _empty(means, (means.size(0), means.size(1))))


def _save_records(ctx, inputs, output):
    means, quaternions, scales, _, view_matrices, intrinsics, first, second = inputs[:8]
    ctx.sh_degree, ctx.packed = inputs[11], inputs[16]
    ctx.save_for_backward(means, quaternions, scales, view_matrices, intrinsics, first, second,
                          output[0], output[9])


def _records_grad(ctx, g_geometry, g_projected, g_appearance, g_opacity_rows, *_):
    means, quats, scales, views, intrinsics, first, second, geometry, rows = ctx.saved_tensors
    with_sh = ctx.sh_degree >= 0
    grads = torch.ops.gabor_splatting.records_backward(
        means, quats, scales, views, intrinsics, first, second, ctx.sh_degree,
        rows if ctx.packed else None, geometry, g_geometry, g_projected,
        g_appearance if with_sh else None, g_opacity_rows if with_sh else None)
    g_means, g_quats, g_scales, g_views, g_intrinsics = grads[:5]
    sh = grads[5:] if with_sh else (None,) * 6
    g_first, g_second, g_weights, g_magnitudes, g_phases, g_opacities = sh
    return (g_means, g_quats, g_scales, g_opacities, g_views, g_intrinsics, g_first, g_second,
            g_weights, g_magnitudes, g_phases) + (None,) * 6


records_forward.register_autograd(_records_grad, setup_context=_save_records)


# --------------------------------------------------------------------------
# Compaction, binning and sorting


@_op("pack_visible")
def pack_visible(radii: Tensor) -> tuple[Tensor, Tensor]:
    """Ascending indices (int64 [V]) of the pairs with radius > 0, and each
    pair's packed row (int32, same shape as radii; -1 when culled)."""
    selected, rows = _native.pack_visible(radii, with_rows=True)
    return selected, rows.view(radii.shape)


@pack_visible.register_fake
def _(radii):
    return _empty(radii, (get_ctx().new_dynamic_size(),), torch.int64), torch.empty_like(radii)


@_op("bin_tiles")
def bin_tiles(geometry: Tensor, radii: Tensor, image_ids: Tensor, images: int, width: int,
              height: int) -> tuple[Tensor, Tensor]:
    """Depth-first binning of compositor rows into tiles: (point_list int32
    [M], ranges int32 [images*tw*th, 2]), the point list and ranges
    rasterize_forward composites (count, emit, sort and ranges;
    rasterize.cu:24-69, 459-501)."""
    _native._require(images > 0 and width > 0 and height > 0, "invalid image dimensions")
    _native.check_image_tiles(images, width, height)
    point_list, ranges = _native.bin_depth_first(geometry, radii, image_ids, images, width,
                                                 height)
    return point_list, ranges


@bin_tiles.register_fake
def _(geometry, radii, image_ids, images, width, height):
    return (_empty(geometry, (get_ctx().new_dynamic_size(),), torch.int32),
            _empty(geometry, (_tiles(images, width, height), 2), torch.int32))


@_op("sort_pairs")
def sort_pairs(keys: Tensor, values: Tensor, begin_bit: int, end_bit: int
               ) -> tuple[Tensor, Tensor]:
    """Stable LSD radix sort of 64-bit keys (int64 holding uint64) with int32
    values over bits [begin_bit, end_bit) (rasterize.cu:478-487)."""
    _native._require(keys.dtype == torch.int64 and values.dtype == torch.int32
                     and keys.shape == values.shape and keys.dim() == 1
                     and keys.is_contiguous() and values.is_contiguous(),
                     "sort_pairs takes contiguous int64 keys and int32 values of one length")
    return _native.sort_pairs(keys, values, begin_bit, end_bit)


@sort_pairs.register_fake
def _(keys, values, begin_bit, end_bit):
    return torch.empty_like(keys), torch.empty_like(values)


OPERATORS = ("rasterize_forward", "rasterize_forward_bounded", "rasterize_backward",
             "evaluate_sh_forward", "evaluate_sh_backward", "project_forward",
             "project_backward", "records_forward", "records_backward", "pack_visible",
             "bin_tiles", "sort_pairs")
