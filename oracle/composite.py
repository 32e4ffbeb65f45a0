"""Tile compositor restated in torch (reference: rasterize.cu:71-281).

Every tile's sorted list is walked front to back; step k of the loop treats
the k-th record of every tile at once for all 256 pixels of each tile, which
keeps the autograd graph O(longest list) deep. Gradients of all inputs come
from torch autograd over this forward - an independent route to the
reference's hand-derived backward (rasterize.cu:284-399).

Masked lanes are evaluated on safe stand-in values so that no inf/NaN from a
rejected sample leaks into autograd.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import binning

TILE = 16
# The reference evaluates pi and the frequency directions in float32
# (rasterize.cu:21, 130): Pi = 3.14159265f, d_f = (cosf(Pi*f/4), sinf(Pi*f/4)).
PI32 = float(np.float32(math.pi))
DIR_X = [float(np.float32(math.cos(np.float32(np.float32(PI32) * f) / np.float32(4)))) for f in range(4)]
DIR_Y = [float(np.float32(math.sin(np.float32(np.float32(PI32) * f) / np.float32(4)))) for f in range(4)]


def appearance_color(a: torch.Tensor, s: torch.Tensor, dirs: torch.Tensor, neural: bool):
    """RGB of records a [..., A] at local coordinates s [..., 2]."""
    if neural:
        inputs = torch.cat([s / 3, dirs], -1)                       # [..., 5]
        W1 = a[..., :30].unflatten(-1, (6, 5))
        b1 = a[..., 30:36]
        W2 = a[..., 36:54].unflatten(-1, (3, 6))
        b2 = a[..., 54:57]
        hidden = torch.sin(30 * ((W1 * inputs[..., None, :]).sum(-1) + b1))
        return torch.sigmoid((W2 * hidden[..., None, :]).sum(-1) + b2)
    dx = s.new_tensor(DIR_X)
    dy = s.new_tensor(DIR_Y)
    dot = s[..., 0:1] * dx + s[..., 1:2] * dy                          # [..., 4]
    wave = torch.cos(2 * PI32 * a[..., 10:14] * dot + a[..., 14:18])
    weights = a[..., 6:10]
    h1 = (weights * (1 + wave) / 2).sum(-1, keepdim=True)
    h2 = (weights * (1 - wave) / 2).sum(-1, keepdim=True)
    return h1 * a[..., 0:3] + h2 * a[..., 3:6]


def composite(geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds,
              width, height, neural, near_plane, far_plane, lists=None, margins=None,
              taken=None, stopped=None):
    """Differentiable forward compositor.

    Returns maps [I,H,W,9], point_list (np.int32), ranges (np.int32 [tiles,2]),
    state [I,H,W,3] (T, m1, m2) and contributors (np.int32 [I,H,W]).
    ``lists`` = (point_list, ranges) replaces the oracle's own binning.
    If ``margins`` is a dict, margins["pixels"] receives [I,H,W] the smallest
    relative distance, over the samples a pixel evaluated, of any discrete
    decision from its threshold (alpha vs 1/255, T(1-alpha) vs 1e-4, the
    surface/screen branch rho3 vs rho2, depth vs near, p.z vs 0).
    If ``taken`` is a dict, taken["quadrants"] receives np.int64 [tiles,
    longest]: for the k-th record of each tile's list, bit q is set when a
    pixel of the tile's 8x8 quadrant q = 2 * (y >= 8) + (x >= 8) took it
    (contributed to its maps, rasterize.cu:254-271).
    If ``stopped`` is a dict, stopped["pixels"] receives bool [I,H,W]: the
    pixels whose walk ended on the transmittance rule - an accepted record
    that would have taken T below 1e-4 (rasterize.cu:254-255) - rather than
    at the end of their tile's list.
    """
    dtype = geometry.dtype
    images = backgrounds.shape[0]
    tw, th = binning.tile_grid(width, height)
    if lists is None:
        g32 = geometry.detach().cpu().to(torch.float32).numpy()
        _, point_list, ranges = binning.bin_pairs(
            g32, radii.cpu().numpy(), image_ids.cpu().numpy(), images, width, height
        )
    else:
        point_list, ranges = (np.asarray(v) for v in lists)
    lengths = ranges[:, 1] - ranges[:, 0]
    tiles = images * tw * th
    # Per-tile record matrix, padded with -1.
    longest = int(lengths.max()) if tiles else 0
    table = np.full((tiles, max(longest, 1)), -1, dtype=np.int64)
    for t in np.flatnonzero(lengths):
        table[t, : lengths[t]] = point_list[ranges[t, 0] : ranges[t, 1]]
    table = torch.from_numpy(table)

    # Pixel coordinates of every tile, row-major 16x16.
    tile_ids = torch.arange(tiles)
    image = tile_ids // (tw * th)
    local = tile_ids % (tw * th)
    offs = torch.arange(TILE * TILE)
    px = (local % tw)[:, None] * TILE + offs % TILE
    py = (local // tw)[:, None] * TILE + offs // TILE
    inside = (px < width) & (py < height)
    x = px.to(dtype)
    y = py.to(dtype)

    T = torch.ones(tiles, TILE * TILE, dtype=dtype)
    out = torch.zeros(tiles, TILE * TILE, 9, dtype=dtype)
    m1 = torch.zeros(tiles, TILE * TILE, dtype=dtype)
    m2 = torch.zeros(tiles, TILE * TILE, dtype=dtype)
    done = ~inside
    ended = torch.zeros(tiles, TILE * TILE, dtype=torch.bool)
    last = torch.zeros(tiles, TILE * TILE, dtype=torch.int64)
    margin = torch.full((tiles, TILE * TILE), math.inf, dtype=torch.float64)
    quadrant_bit = 1 << (2 * ((offs // TILE) >= 8).long() + ((offs % TILE) >= 8).long())
    quadrants = np.zeros((tiles, max(longest, 1)), dtype=np.int64)
    mscale = far_plane / (far_plane - near_plane)
    for k in range(longest):
        rec = table[:, k]
        has = rec >= 0
        if not bool((has[:, None] & ~done).any()):
            break
        r = rec.clamp_min(0)
        g = geometry[r][:, None, :]                                  # [tiles,1,17]
        prim = primitive_ids[r]
        a = appearance[prim][:, None, :]
        o = opacities[prim][:, None]
        kx = x[..., None] * g[..., 6:9] - g[..., 0:3]
        ly = y[..., None] * g[..., 6:9] - g[..., 3:6]
        p = torch.cross(kx, ly, dim=-1)
        degenerate = p[..., 2] == 0
        pz = torch.where(degenerate, torch.ones_like(p[..., 2]), p[..., 2])
        s = p[..., :2] / pz[..., None]
        rho3 = (s**2).sum(-1)
        rho2 = 2 * ((g[..., 9] - x) ** 2 + (g[..., 10] - y) ** 2)
        surface = rho3 <= rho2
        plane_depth = s[..., 0] * g[..., 6] + s[..., 1] * g[..., 7] + g[..., 8]
        depth = plane_depth if neural else torch.where(surface, plane_depth, g[..., 8])
        ok = ~degenerate & torch.isfinite(depth) & (depth >= near_plane)
        e = torch.exp(-0.5 * torch.minimum(rho3, rho2))
        alpha = (o * e).clamp_max(0.99)
        accept = ok & (alpha >= 1.0 / 255.0) & has[:, None] & ~done
        if margins is not None:
            with torch.no_grad():
                walked = has[:, None] & ~done & inside
                tiny = 1e-300
                candidates = [
                    (p[..., 2].abs() / (p.norm(dim=-1) + tiny)).double(),
                    ((o * e - 1 / 255).abs() * 255).double(),
                    ((depth - near_plane).abs() / near_plane).double(),
                    torch.where(accept, ((T * (1 - alpha) - 1e-4).abs() / 1e-4), torch.inf).double(),
                ]
                if not neural:
                    candidates.append(((rho3 - rho2).abs() / (rho3 + rho2 + tiny)).double())
                local = torch.stack(candidates).amin(0)
                margin = torch.where(walked, torch.minimum(margin, local), margin)
        stop = accept & (T * (1 - alpha) < 1e-4)
        done = done | stop
        ended = ended | stop
        take = accept & ~stop
        if taken is not None:
            bits = torch.where(take & inside, quadrant_bit, torch.zeros_like(quadrant_bit))
            for q in range(4):
                quadrants[:, k] |= ((bits & (1 << q)).amax(1) > 0).numpy().astype(np.int64) << q
        a_take = torch.where(take, alpha, torch.zeros_like(alpha))
        s_take = torch.where(take[..., None], s, torch.zeros_like(s))
        z_take = torch.where(take, depth, torch.ones_like(depth))
        color = appearance_color(a, s_take, g[..., 14:17].expand(*s.shape[:-1], 3), neural)
        w = T * a_take
        m = mscale * (1 - near_plane / z_take)
        contribution = torch.cat(
            [
                w[..., None] * color,
                torch.zeros_like(w)[..., None],
                (w * z_take)[..., None],
                w[..., None] * g[..., 11:14],
                (w * (m * m * (1 - T) + m2 - 2 * m * m1))[..., None],
            ],
            -1,
        )
        out = out + contribution
        m1 = m1 + w * m
        m2 = m2 + w * m * m
        T = T * (1 - a_take)
        last = torch.where(take, torch.full_like(last, k + 1), last)

    bg = backgrounds[image][:, None, :]                                # [tiles,1,3]
    out = torch.cat([out[..., :3] + T[..., None] * bg, (1 - T)[..., None], out[..., 4:]], -1)
    # Scatter tile pixels back into images.
    keep = inside.reshape(-1)
    flat_index = ((image[:, None] * height + py) * width + px).reshape(-1)[keep]
    order = torch.argsort(flat_index)
    maps = out.reshape(-1, 9)[keep][order].reshape(images, height, width, 9)
    state = torch.stack([T, m1, m2], -1).reshape(-1, 3)[keep][order].reshape(images, height, width, 3)
    contributors = last.reshape(-1)[keep][order].reshape(images, height, width)
    if margins is not None:
        margins["pixels"] = margin.reshape(-1)[keep][order].reshape(images, height, width)
    if taken is not None:
        taken["quadrants"] = quadrants
    if stopped is not None:
        stopped["pixels"] = ended.reshape(-1)[keep][order].reshape(images, height, width)
    return maps, point_list, ranges, state, contributors.numpy().astype(np.int32)
