"""Pins oracle/projection.py: rotation, projected plane, conic bound, radii."""

import math

import pytest
import torch

from oracle.projection import MIN_RADIUS, project, rotation_from_quaternion
from scenes import _rotation_rodrigues


def test_rotation_matches_rodrigues_and_is_proper():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(64, 4, generator=g, dtype=torch.float64) * 3
    R = rotation_from_quaternion(q)
    for i in range(len(q)):
        torch.testing.assert_close(R[i], _rotation_rodrigues(q[i]), atol=1e-12, rtol=0)
    eye = torch.eye(3, dtype=torch.float64).expand(64, 3, 3)
    torch.testing.assert_close(R.transpose(-1, -2) @ R, eye, atol=1e-12, rtol=0)
    torch.testing.assert_close(torch.linalg.det(R), torch.ones(64, dtype=torch.float64))


def test_rotation_axis_angle_closed_form():
    # 90 degrees about z maps x to y: q = (cos 45, 0, 0, sin 45).
    q = torch.tensor([math.cos(math.pi / 4), 0.0, 0.0, math.sin(math.pi / 4)], dtype=torch.float64)
    R = rotation_from_quaternion(q)
    expected = torch.tensor([[0.0, -1.0, 0.0], [1.0, 0.0, 0.0], [0.0, 0.0, 1.0]], dtype=torch.float64)
    torch.testing.assert_close(R, expected, atol=1e-15, rtol=0)


def _fronto_parallel(mx, my, z, su, sv, f=80.0, cx=32.0, cy=30.0, width=64, height=64):
    means = torch.tensor([[[mx, my, z]]], dtype=torch.float64)
    quats = torch.tensor([[[1.0, 0.0, 0.0, 0.0]]], dtype=torch.float64)
    scales = torch.tensor([[[su, sv]]], dtype=torch.float64)
    views = torch.eye(4, dtype=torch.float64)[None, None]
    K = torch.tensor([[f, 0, cx], [0, f, cy], [0, 0, 1.0]], dtype=torch.float64)[None, None]
    return project(means, quats, scales, views, K, width, height, 0.2, 100.0)


def test_fronto_parallel_closed_form():
    f, cx, cy = 80.0, 32.0, 30.0
    mx, my, z, su, sv = 0.1, -0.2, 3.0, 0.3, 0.15
    T, xy, normals, directions, radii = _fronto_parallel(mx, my, z, su, sv, f, cx, cy)
    expected_T = torch.tensor(
        [[f * su, 0, f * mx + cx * z], [0, f * sv, f * my + cy * z], [0, 0, z]], dtype=torch.float64
    )
    torch.testing.assert_close(T[0, 0, 0], expected_T, atol=1e-12, rtol=0)
    # The conic centre is the pinhole projection of the mean.
    torch.testing.assert_close(
        xy[0, 0, 0], torch.tensor([f * mx / z + cx, f * my / z + cy], dtype=torch.float64)
    )
    # Fronto-parallel: normal (0,0,1) flipped toward the camera.
    torch.testing.assert_close(normals[0, 0, 0], torch.tensor([0.0, 0.0, -1.0], dtype=torch.float64))
    d = torch.tensor([mx, my, z], dtype=torch.float64)
    torch.testing.assert_close(directions[0, 0, 0], d / d.norm())
    # Three-sigma extent along the larger axis: 3 f su / z = 24 px.
    assert int(radii) == math.ceil(max(3 * f * su / z, 3 * f * sv / z, MIN_RADIUS))


@pytest.mark.parametrize(
    "case, expected",
    [
        (dict(mx=0.0, my=0.0, z=3.0, su=0.01, sv=0.01), 3),      # minimum radius 3*0.707106
        (dict(mx=0.0, my=0.0, z=0.1, su=0.1, sv=0.1), 0),        # in front of the near plane
        (dict(mx=0.0, my=0.0, z=150.0, su=0.1, sv=0.1), 0),      # beyond the far plane
        (dict(mx=40.0, my=0.0, z=2.0, su=0.1, sv=0.1), 0),       # right of the image
        (dict(mx=-40.0, my=0.0, z=2.0, su=0.1, sv=0.1), 0),      # left of the image
    ],
)
def test_radius_and_culling(case, expected):
    *_, radii = _fronto_parallel(**case)
    assert int(radii) == expected


@pytest.mark.parametrize("case", ["edge_on", "degenerate_conic"])
def test_edge_on_and_degenerate_surfels_are_culled(case):
    # q = (1,1,1,1)/2 is exactly the 120-degree turn x->y->z->x: the normal
    # is the x axis, so a surfel on the optical axis is seen exactly edge-on;
    # with unit scales and x = 0.1 the conic denominator is exactly zero.
    q = torch.full((1, 1, 4), 0.5, dtype=torch.float64)
    R = rotation_from_quaternion(q)[0, 0]
    torch.testing.assert_close(R, torch.tensor([[0.0, 0, 1], [1, 0, 0], [0, 1, 0]], dtype=torch.float64))
    x, scale = (0.1, 1.0) if case == "degenerate_conic" else (0.0, 0.2)
    means = torch.tensor([[[x, 0.0, 3.0]]], dtype=torch.float64)
    views = torch.eye(4, dtype=torch.float64)[None, None]
    K = torch.tensor([[80.0, 0, 32], [0, 80.0, 32], [0, 0, 1]], dtype=torch.float64)[None, None]
    T, xy, *_, radii = project(means, q, torch.full((1, 1, 2), scale, dtype=torch.float64), views,
                               K, 64, 64, 0.2, 100.0)
    assert int(radii) == 0
    if case == "degenerate_conic":
        assert float((torch.tensor([9.0, 9, -1], dtype=torch.float64) * T[0, 0, 0, 2] ** 2).sum()) == 0


def test_projection_gradients_match_finite_differences():
    g = torch.Generator().manual_seed(3)
    S, C, N = 1, 2, 4
    means = (torch.rand(S, N, 3, generator=g, dtype=torch.float64) - 0.5)
    means[..., 2] += 3
    quats = torch.randn(S, N, 4, generator=g, dtype=torch.float64)
    scales = torch.rand(S, N, 2, generator=g, dtype=torch.float64) * 0.2 + 0.05
    views = torch.eye(4, dtype=torch.float64).expand(S, C, 4, 4).clone()
    views[..., :3, 3] = torch.randn(S, C, 3, generator=g, dtype=torch.float64) * 0.1
    K = torch.tensor([[60.0, 1.0, 31], [0, 58.0, 29], [0, 0, 1]], dtype=torch.float64).expand(S, C, 3, 3).clone()
    inputs = [means, quats, scales, views, K]
    weights = [torch.randn(s, generator=g, dtype=torch.float64) for s in [(S, C, N, 3, 3), (S, C, N, 2), (S, C, N, 3), (S, C, N, 3)]]

    def objective(*args):
        outs = project(*args, 64, 64, 0.2, 100.0)[:4]
        return sum((o * w).sum() for o, w in zip(outs, weights))

    assert torch.autograd.gradcheck(objective, [t.clone().requires_grad_() for t in inputs],
                                    eps=1e-6, atol=1e-5, rtol=1e-4)
