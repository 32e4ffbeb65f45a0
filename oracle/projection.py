"""Projection of surfels into every camera (reference: rendering.py:156-218).

Differentiable torch code, any float dtype, any device (used on the CPU).
"""

from __future__ import annotations

import torch

# float32(3 * 0.707106): the minimum screen radius (rendering.py:208).
MIN_RADIUS = 3 * 0.707106


def rotation_from_quaternion(q: torch.Tensor) -> torch.Tensor:
    """Rotation matrices [..., 3, 3] from wxyz quaternions, normalised first.

    Columns 0 and 1 are the tangent axes, column 2 the normal
    (rendering.py:156-173).
    """
    q = q / q.norm(dim=-1, keepdim=True)
    w, x, y, z = q.unbind(-1)
    xx, yy, zz = x * x, y * y, z * z
    xy, xz, yz = x * y, x * z, y * z
    wx, wy, wz = w * x, w * y, w * z
    return torch.stack(
        [
            torch.stack([1 - 2 * (yy + zz), 2 * (xy - wz), 2 * (xz + wy)], -1),
            torch.stack([2 * (xy + wz), 1 - 2 * (xx + zz), 2 * (yz - wx)], -1),
            torch.stack([2 * (xz - wy), 2 * (yz + wx), 1 - 2 * (xx + yy)], -1),
        ],
        -2,
    )


def project(means, quaternions, scales, view_matrices, intrinsics, width, height,
            near_plane, far_plane):
    """Project [S,N] surfels into [S,C] cameras.

    Returns transform [S,C,N,3,3], xy [S,C,N,2], normals [S,C,N,3],
    directions [S,C,N,3] (all differentiable) and radii int32 [S,C,N].
    """
    R = rotation_from_quaternion(quaternions)                      # [S,N,3,3]
    Rc = view_matrices[..., :3, :3]                                 # [S,C,3,3]
    t = view_matrices[..., :3, 3]                                   # [S,C,3]
    # Local plane columns (scaled tangents, mean) mapped into camera space.
    tangents = R[..., :2] * scales[..., None, :]                    # [S,N,3,2]
    cols = torch.cat([tangents, means[..., :, None]], -1)           # [S,N,3,3]
    plane = Rc[:, :, None] @ cols[:, None]                           # [S,C,N,3,3]
    plane = plane + torch.cat(
        [torch.zeros_like(t)[..., None].expand(*t.shape, 2), t[..., None]], -1
    )[:, :, None]
    T = intrinsics[:, :, None] @ plane                               # [S,C,N,3,3]

    # Upstream three-sigma conic bound: f = [9, 9, -1] / sum(f0 * T2^2).
    f0 = T.new_tensor([9.0, 9.0, -1.0])
    denominator = (f0 * T[..., 2, :] ** 2).sum(-1)
    valid = denominator != 0
    f = f0 / torch.where(valid, denominator, torch.ones_like(denominator))[..., None]
    xy = (f[..., None, :] * T[..., :2, :] * T[..., 2:3, :]).sum(-1)  # [S,C,N,2]
    extent_sq = xy**2 - (f[..., None, :] * T[..., :2, :] ** 2).sum(-1)

    camera_means = plane[..., :, 2]                                   # [S,C,N,3]
    normals = (Rc[:, :, None] @ R[:, None, :, :, 2:3]).squeeze(-1)     # [S,C,N,3]
    facing = -(camera_means * normals).sum(-1)
    sign = torch.where(facing > 0, 1.0, -1.0).to(normals.dtype)
    normals = normals * sign[..., None]
    centres = -(Rc.transpose(-1, -2) @ t[..., None]).squeeze(-1)      # [S,C,3]
    offset = means[:, None] - centres[:, :, None]                    # [S,C,N,3]
    directions = offset / offset.norm(dim=-1, keepdim=True).clamp_min(1e-12)

    with torch.no_grad():
        extent = extent_sq.clamp_min(1e-4).sqrt()
        radius = torch.maximum(extent.amax(-1), extent.new_tensor(MIN_RADIUS)).ceil()
        tw, th = (width + 15) // 16, (height + 15) // 16
        lower = torch.trunc((xy - radius[..., None]) / 16).clamp_min(0)
        upper = torch.trunc((xy + radius[..., None] + 15) / 16).clamp_min(0)
        z = camera_means[..., 2]
        visible = valid & (facing != 0) & (z > near_plane) & (z < far_plane)
        visible &= torch.isfinite(radius) & (radius < 2**30) & torch.isfinite(xy).all(-1)
        visible &= upper[..., 0].clamp_max(tw) > lower[..., 0].clamp_max(tw)
        visible &= upper[..., 1].clamp_max(th) > lower[..., 1].clamp_max(th)
        radii = torch.where(visible, radius, torch.zeros_like(radius)).to(torch.int32)
    return T, xy, normals, directions, radii


def radius_before_ceil(means, quaternions, scales, view_matrices, intrinsics) -> torch.Tensor:
    """max(extent, min radius) before the ceiling, for the radius margin rule."""
    T, xy, *_ = project(means, quaternions, scales, view_matrices, intrinsics, 16, 16, 1e-9, 1e30)
    f0 = T.new_tensor([9.0, 9.0, -1.0])
    denominator = (f0 * T[..., 2, :] ** 2).sum(-1)
    denominator = torch.where(denominator != 0, denominator, torch.ones_like(denominator))
    f = f0 / denominator[..., None]
    extent = (xy**2 - (f[..., None, :] * T[..., :2, :] ** 2).sum(-1)).clamp_min(1e-4).sqrt()
    return torch.maximum(extent.amax(-1), extent.new_tensor(MIN_RADIUS)).detach()
