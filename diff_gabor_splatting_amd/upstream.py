"""The upstream rasterizers' calling convention on top of this renderer.

Training code written for the pinned upstream CUDA rasterizers
(diff-gabor-rasterization and diff-neural-gabor-rasterization, which follow
the 2DGS / Inria Gaussian-splatting interface) builds a settings tuple with
transposed view and full projection matrices and FoV tangents, and calls a
rasterizer module per camera. The reference compares itself with those
packages in its optional test (tests/test_upstream.py:13-96), which fixes the
conversion used here:

* view = viewmatrix^T; the full projection P V = projmatrix^T, so
  P = projmatrix^T V^-1 (V rigid);
* fx = W / (2 tanfovx), fy = H / (2 tanfovy), cx = (P[0,2] W + W - 1) / 2,
  cy = (P[1,2] H + H - 1) / 2;
* near and far from P[2,2] = f / (f - n) and P[2,3] = -f n / (f - n);
* bg is the background colour, opacities arrive as [N, 1], scale_modifier
  multiplies the scales.

The rasterizer returns (rgb [3, H, W], radii [N], maps [7, H, W]) with maps =
accumulated depth, alpha, normal (3), median depth, distortion. Median depth
is not produced by this renderer (the reference leaves it out of its release
too, README.md:268-270); that channel is zero. ``means2D`` receives the
screen-space gradient of the projected centres, as upstream. The upstream
packages themselves are not available here, so agreement with their outputs
is unpinned; the conversion is pinned by round trip against the direct API.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import rendering


class GaborRasterizationSettings(NamedTuple):
    """Camera and options of one upstream rasterizer call."""

    image_height: int
    image_width: int
    tanfovx: float
    tanfovy: float
    bg: torch.Tensor
    scale_modifier: float
    viewmatrix: torch.Tensor
    projmatrix: torch.Tensor
    sh_degree: int
    campos: torch.Tensor
    prefiltered: bool
    debug: bool


# The neural upstream package keeps the Gaussian-splatting class names.
GaussianRasterizationSettings = GaborRasterizationSettings


def camera_from_settings(settings: GaborRasterizationSettings):
    """(view [4,4], intrinsics [3,3], near, far) recovered from upstream settings."""
    width, height = settings.image_width, settings.image_height
    view = settings.viewmatrix.t().contiguous()
    rotation, translation = view[:3, :3], view[:3, 3]
    inverse = torch.eye(4, dtype=view.dtype, device=view.device)
    inverse[:3, :3] = rotation.t()
    inverse[:3, 3] = -rotation.t() @ translation
    projection = settings.projmatrix.t() @ inverse
    intrinsics = torch.zeros(3, 3, dtype=view.dtype, device=view.device)
    intrinsics[0, 0] = width / (2 * float(settings.tanfovx))
    intrinsics[1, 1] = height / (2 * float(settings.tanfovy))
    intrinsics[0, 2] = (projection[0, 2] * width + (width - 1)) / 2
    intrinsics[1, 2] = (projection[1, 2] * height + (height - 1)) / 2
    intrinsics[2, 2] = 1.0
    a, b = float(projection[2, 2]), float(projection[2, 3])
    near = -b / a
    far = a * near / (a - 1)
    return view, intrinsics, near, far


class _Rasterizer(torch.nn.Module):
    neural = False

    def __init__(self, raster_settings: GaborRasterizationSettings):
        super().__init__()
        self.raster_settings = raster_settings

    def _render(self, means3D, means2D, opacities, scales, rotations, appearance, sh_degree):
        settings = self.raster_settings
        view, intrinsics, near, far = camera_from_settings(settings)
        n = means3D.shape[0]
        if means2D is not None and tuple(means2D.shape) != (n, 3) and tuple(means2D.shape) != (n, 2):
            raise ValueError("means2D must have shape [N, 3] or [N, 2]")
        rgb, alpha, meta = rendering.render(
            means3D, rotations, scales * settings.scale_modifier, opacities.reshape(n),
            appearance, view[None], intrinsics[None], settings.image_width,
            settings.image_height, settings.bg.reshape(1, 3), False, near, far, self.neural,
            sh_degree, True, None if means2D is None else means2D[:, :2],
        )
        maps = torch.cat((
            meta["accumulated_depth"][0], alpha[0], meta["normals"][0],
            torch.zeros_like(alpha[0]), meta["distortion"][0],
        ), -1)
        return rgb[0].permute(2, 0, 1), meta["radii"][0], maps.permute(2, 0, 1)


class GaborRasterizer(_Rasterizer):
    """Classic Gabor rasterizer with the upstream forward signature."""

    def forward(self, means3D, means2D, opacities, colors_precomp=None, colors_precomp2=None,
                weights_for_frequency_angle=None, frequency_lengths=None, phases=None,
                scales=None, rotations=None, shs=None, cov3D_precomp=None):
        if shs is not None or cov3D_precomp is not None:
            raise ValueError("pass colors_precomp / colors_precomp2 and scales / rotations; "
                             "shs and cov3D_precomp are not supported")
        appearance = (colors_precomp, colors_precomp2, weights_for_frequency_angle,
                      frequency_lengths, phases)
        return self._render(means3D, means2D, opacities, scales, rotations, appearance, None)


class GaussianRasterizer(_Rasterizer):
    """Neural Gabor rasterizer (5->6->3 SIREN per surfel) with the upstream signature."""

    neural = True

    def forward(self, means3D, means2D, opacities, W1, b1, W2, b2, scales=None,
                rotations=None):
        return self._render(means3D, means2D, opacities, scales, rotations, (W1, b1, W2, b2),
                            None)
