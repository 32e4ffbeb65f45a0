"""The upstream-convention adapter against the direct API.

Settings are built exactly as the reference's optional upstream test builds
them (tests/test_upstream.py:23-59); the adapter must recover the camera and
render what the direct call renders, and write the screen-space gradient of
the projected centres into means2D. Agreement with the upstream packages
themselves is unpinned: they are not installed.
"""

import pytest
import torch

from diff_gabor_splatting_amd import upstream
from scenes import make_inputs


def upstream_settings(view, K, width, height, bg, near=0.2, far=100.0):
    projection = torch.zeros(4, 4, dtype=view.dtype, device=view.device)
    projection[0, 0] = 2 * K[0, 0] / width
    projection[1, 1] = 2 * K[1, 1] / height
    projection[0, 2] = (2 * K[0, 2] - (width - 1)) / width
    projection[1, 2] = (2 * K[1, 2] - (height - 1)) / height
    projection[2, 2] = far / (far - near)
    projection[2, 3] = -far * near / (far - near)
    projection[3, 2] = 1
    return upstream.GaborRasterizationSettings(
        image_height=height, image_width=width, tanfovx=width / (2 * K[0, 0].item()),
        tanfovy=height / (2 * K[1, 1].item()), bg=bg, scale_modifier=1.0,
        viewmatrix=view.T.contiguous(), projmatrix=(projection @ view).T.contiguous(),
        sh_degree=0, campos=(-view[:3, :3].T @ view[:3, 3]).contiguous(), prefiltered=False,
        debug=False)


def test_camera_round_trip():
    angle = torch.tensor(0.3, dtype=torch.float64)
    view = torch.eye(4, dtype=torch.float64)
    view[0, 0] = view[2, 2] = torch.cos(angle)
    view[0, 2], view[2, 0] = torch.sin(angle), -torch.sin(angle)
    view[:3, 3] = torch.tensor([0.2, -0.1, 0.4], dtype=torch.float64)
    K = torch.tensor([[28.0, 0, 17.25], [0, 27.0, 15.5], [0, 0, 1]], dtype=torch.float64)
    settings = upstream_settings(view, K, 35, 33, torch.zeros(3), near=0.3, far=50.0)
    got_view, got_K, near, far = upstream.camera_from_settings(settings)
    torch.testing.assert_close(got_view, view)
    torch.testing.assert_close(got_K, K)
    assert near == pytest.approx(0.3) and far == pytest.approx(50.0)


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
@pytest.mark.parametrize("method", ["classic", "neural"])
def test_adapter_matches_direct_api(method):
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    values = {k: v.cuda() for k, v in make_inputs(method, cameras=1, primitives=10).items()}
    width, height = 35, 33
    values["means"][..., 0] = torch.linspace(-1.1, 1.1, 10, device="cuda")
    values["means"][..., 1] = torch.linspace(0.6, -0.6, 10, device="cuda")
    values["intrinsics"][..., 0, 0] = 28
    values["intrinsics"][..., 1, 1] = 27
    values["intrinsics"][..., 0, 2] = (width - 1) / 2
    values["intrinsics"][..., 1, 2] = (height - 1) / 2
    for value in values.values():
        value.requires_grad_()
    render = rasterize_gabors if method == "classic" else rasterize_neural_gabors
    rgb, alpha, meta = render(**values, width=width, height=height)
    meta["projected_means"].retain_grad()

    settings = upstream_settings(values["view_matrices"][0, 0].detach(),
                                 values["intrinsics"][0, 0].detach(), width, height,
                                 values["backgrounds"][0, 0].detach())
    arguments = dict(means3D=values["means"][0], opacities=values["opacities"][0, :, None],
                     scales=values["scales"][0], rotations=values["quaternions"][0])
    means2D = torch.zeros_like(values["means"][0], requires_grad=True)
    if method == "classic":
        rasterizer = upstream.GaborRasterizer(settings)
        arguments.update(colors_precomp=values["colors"][0],
                         colors_precomp2=values["secondary_colors"][0],
                         weights_for_frequency_angle=values["frequency_weights"][0],
                         frequency_lengths=values["frequency_magnitudes"][0],
                         phases=values["phases"][0])
    else:
        rasterizer = upstream.GaussianRasterizer(upstream.GaussianRasterizationSettings(*settings))
        arguments.update(W1=values["input_weights"][0], b1=values["input_biases"][0],
                         W2=values["output_weights"][0], b2=values["output_biases"][0])
    out_rgb, radii, maps = rasterizer(means2D=means2D, **arguments)
    tolerance = dict(atol=1e-6, rtol=1e-5)
    torch.testing.assert_close(out_rgb, rgb[0, 0].permute(2, 0, 1), **tolerance)
    torch.testing.assert_close(maps[1], alpha[0, 0, ..., 0], **tolerance)
    torch.testing.assert_close(maps[0], meta["accumulated_depth"][0, 0, ..., 0], **tolerance)
    torch.testing.assert_close(maps[2:5], meta["normals"][0, 0].permute(2, 0, 1), **tolerance)
    torch.testing.assert_close(maps[6], meta["distortion"][0, 0, ..., 0], **tolerance)
    assert bool((maps[5] == 0).all())
    torch.testing.assert_close(radii, meta["radii"][0, 0])

    weights = torch.linspace(-0.5, 0.8, 9 * height * width, device="cuda").reshape(height, width, 9)
    direct = torch.cat((rgb[0, 0], alpha[0, 0], meta["accumulated_depth"][0, 0],
                        meta["normals"][0, 0], meta["distortion"][0, 0]), -1)
    (direct * weights).sum().backward()
    adapted = torch.cat((out_rgb.permute(1, 2, 0), maps[1:2].permute(1, 2, 0),
                         maps[0:1].permute(1, 2, 0), maps[2:5].permute(1, 2, 0),
                         maps[6:7].permute(1, 2, 0)), -1)
    expected_means = values["means"].grad[0].clone()
    values["means"].grad = None
    (adapted * weights).sum().backward()
    torch.testing.assert_close(values["means"].grad[0], expected_means, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(means2D.grad[:, :2], meta["projected_means"].grad,
                               atol=1e-6, rtol=1e-5)
    assert bool((means2D.grad[:, 2] == 0).all())
