"""torch.library custom operators (``torch.ops.gabor_splatting.*``).

CPU: every operator is registered with the reference's argument names where
the reference binds the function, its fake kernel gives the real kernel's
shapes and dtypes under FakeTensorMode (data-dependent sizes as new symbols),
and a CPU call raises (there is no CPU kernel). GPU: ``torch.library.opcheck``
(schema, autograd registration, fake tensors, AOT dispatch with dynamic
shapes) on small inputs, and the operators' outputs equal the direct calls'.
"""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.symbolic_shapes import ShapeEnv

from diff_gabor_splatting_amd import _native, library

ops = torch.ops.gabor_splatting

# Argument names of the four functions the reference binds into _C
# (src/gabor_splatting/csrc/rasterize.h:6-21).
REFERENCE_ARGUMENTS = {
    "rasterize_forward": ["geometry", "appearance", "opacities", "primitive_ids", "image_ids",
                          "radii", "backgrounds", "width", "height", "neural", "near_plane",
                          "far_plane"],
    "rasterize_backward": ["geometry", "appearance", "opacities", "primitive_ids", "backgrounds",
                           "point_list", "ranges", "state", "contributors", "grad_maps", "width",
                           "height", "neural", "near_plane", "far_plane"],
    "evaluate_sh_forward": ["first", "second", "directions", "degree"],
    "evaluate_sh_backward": ["first", "second", "directions", "grad_colors", "degree"],
}


def test_every_operator_is_registered():
    for name in library.OPERATORS:
        assert hasattr(ops, name), name
        assert ops.__getattr__(name).default._schema.name == f"gabor_splatting::{name}"


@pytest.mark.parametrize("name", sorted(REFERENCE_ARGUMENTS))
def test_reference_functions_keep_their_arguments(name):
    schema = ops.__getattr__(name).default._schema
    assert [a.name for a in schema.arguments] == REFERENCE_ARGUMENTS[name]


def _fake_inputs():
    f32, i32, i64 = torch.float32, torch.int32, torch.int64
    c = dict(device="cuda")
    return dict(
        geometry=torch.empty(10, 17, **c), appearance=torch.empty(10, 18, **c),
        opacities=torch.empty(10, **c), primitive_ids=torch.empty(10, dtype=i64, **c),
        image_ids=torch.empty(10, dtype=i64, **c), radii=torch.empty(10, dtype=i32, **c),
        backgrounds=torch.empty(2, 3, **c),
        means=torch.empty(1, 7, 3, **c), quaternions=torch.empty(1, 7, 4, **c),
        scales=torch.empty(1, 7, 2, **c), surfel_opacities=torch.empty(1, 7, **c),
        views=torch.empty(1, 2, 4, 4, **c), K=torch.empty(1, 2, 3, 3, **c),
        first=torch.empty(1, 7, 16, 3, **c), second=torch.empty(1, 7, 16, 3, **c),
        shared=torch.empty(1, 7, 4, **c), directions=torch.empty(1, 2, 7, 3, dtype=f32, **c),
    )


def test_fake_kernels_give_the_output_shapes():
    with FakeTensorMode(shape_env=ShapeEnv()):
        x = _fake_inputs()
        raster = (x["geometry"], x["appearance"], x["opacities"], x["primitive_ids"],
                  x["image_ids"], x["radii"], x["backgrounds"], 40, 30, False, 0.2, 100.0)
        maps, points, ranges, state, contributors = ops.rasterize_forward(*raster)
        assert maps.shape == (2, 30, 40, 9) and state.shape == (2, 30, 40, 3)
        assert contributors.shape == (2, 30, 40) and contributors.dtype == torch.int32
        assert ranges.shape == (2 * 3 * 2, 2) and ranges.dtype == torch.int32
        assert points.dtype == torch.int32 and not isinstance(points.shape[0], int)
        bounded = ops.rasterize_forward_bounded(*raster, 500)
        assert bounded[1].shape == (500,) and bounded[5].shape == (2,)
        assert bounded[5].dtype == torch.int64
        grads = ops.rasterize_backward(x["geometry"], x["appearance"], x["opacities"],
                                       x["primitive_ids"], x["backgrounds"], points, ranges,
                                       state, contributors, maps, 40, 30, False, 0.2, 100.0)
        assert [g.shape for g in grads] == [(10, 17), (10, 18), (10,), (2, 3)]
        colors = ops.evaluate_sh_forward(x["first"], x["second"], x["directions"], 3)
        assert colors.shape == (1, 2, 7, 6)
        sh = ops.evaluate_sh_backward(x["first"], x["second"], x["directions"], colors, 3)
        assert [g.shape for g in sh] == [(1, 7, 16, 3), (1, 7, 16, 3), (1, 2, 7, 3)]
        camera = (x["means"], x["quaternions"], x["scales"], x["views"], x["K"])
        transform, xy, normals, directions, radii = ops.project_forward(*camera, 40, 30, 0.2,
                                                                        100.0)
        assert transform.shape == (1, 2, 7, 3, 3) and radii.dtype == torch.int32
        assert [g.shape for g in ops.project_backward(*camera, transform, xy, None, None)] == [
            (1, 7, 3), (1, 7, 4), (1, 7, 2), (1, 2, 4, 4), (1, 2, 3, 3)]
        for packed in (False, True):
            rows = ops.records_forward(
                x["means"], x["quaternions"], x["scales"], x["surfel_opacities"], x["views"],
                x["K"], x["first"], x["second"], x["shared"], x["shared"], x["shared"], 3, 40,
                30, 0.2, 100.0, packed)
            q = rows[0].shape[0]
            assert (not isinstance(q, int)) if packed else q == 14
            assert rows[2].shape[1] == 18 and rows[7].shape[0] == 3
            assert rows[8].shape == (1, 2, 7)
            assert rows[9].shape == ((14,) if packed else (0,))
        plain = ops.records_forward(x["means"], x["quaternions"], x["scales"], None, x["views"],
                                    x["K"], None, None, None, None, None, -1, 40, 30, 0.2, 100.0,
                                    False)
        assert plain[2].shape == (14, 0) and plain[3].shape == (0,)
        back = ops.records_backward(*camera, x["first"], x["second"], 3, None, plain[0],
                                    plain[0], None, None, None)
        assert [g.shape for g in back[5:]] == [(1, 7, 16, 3), (1, 7, 16, 3), (1, 7, 4),
                                               (1, 7, 4), (1, 7, 4), (1, 7)]
        selected, row_of_pair = ops.pack_visible(radii)
        assert selected.dtype == torch.int64 and row_of_pair.shape == (1, 2, 7)
        points, ranges = ops.bin_tiles(x["geometry"], x["radii"], x["image_ids"], 2, 40, 30)
        assert ranges.shape == (12, 2) and points.dtype == torch.int32
        keys, values = ops.sort_pairs(x["image_ids"], x["radii"], 0, 64)
        assert keys.shape == (10,) and values.dtype == torch.int32


def test_cpu_tensors_have_no_kernel():
    first = torch.zeros(1, 2, 1, 3)
    with pytest.raises((NotImplementedError, RuntimeError)):
        ops.evaluate_sh_forward(first, first, torch.zeros(1, 1, 2, 3), 0)


# --------------------------------------------------------------------------
# GPU


def _scene(device):
    from scenes import random_scene

    raw = random_scene("classic", scenes=1, cameras=2, n=60, width=40, height=30, seed=11, sh=2)
    return {k: v.to(device).contiguous() for k, v in raw.items()}


def _records(scene, packed):
    return ops.records_forward(
        scene["means"], scene["quaternions"], scene["scales"], scene["opacities"],
        scene["view_matrices"], scene["intrinsics"], scene["colors"], scene["secondary_colors"],
        scene["frequency_weights"], scene["frequency_magnitudes"], scene["phases"], 2, 40, 30,
        0.2, 100.0, packed)


def _raster_inputs(scene, packed=True):
    rows = _records(scene, packed)
    geometry, _, appearance, opacity_rows, radii, primitive_ids, image_ids = rows[:7]
    return (geometry, appearance, opacity_rows, primitive_ids, image_ids, radii,
            scene["backgrounds"].reshape(-1, 3).contiguous())


def _grad(*tensors):
    return [t.detach().clone().requires_grad_() for t in tensors]




@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("name", ["evaluate_sh", "project", "records", "rasterize",
                                  "rasterize_bounded", "rasterize_backward", "pack_visible",
                                  "bin_tiles", "sort_pairs"])
@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_opcheck(name, packed):
    device = torch.device("cuda:0")
    scene = _scene(device)
    print(f"opcheck {name} packed={packed}", flush=True)
    if name == "evaluate_sh":
        directions = ops.project_forward(scene["means"], scene["quaternions"], scene["scales"],
                                         scene["view_matrices"], scene["intrinsics"], 40, 30,
                                         0.2, 100.0)[3]
        args = (*_grad(scene["colors"], scene["secondary_colors"], directions), 2)
        op = ops.evaluate_sh_forward
    elif name == "project":
        args = (*_grad(scene["means"], scene["quaternions"], scene["scales"],
                       scene["view_matrices"], scene["intrinsics"]), 40, 30, 0.2, 100.0)
        op = ops.project_forward
    elif name == "records":
        keys = ("means", "quaternions", "scales", "opacities", "view_matrices", "intrinsics",
                "colors", "secondary_colors", "frequency_weights", "frequency_magnitudes",
                "phases")
        args = (*_grad(*(scene[k] for k in keys)), 2, 40, 30, 0.2, 100.0, packed)
        op = ops.records_forward
    elif name in ("rasterize", "rasterize_bounded"):
        g, a, o, p, i, r, b = _raster_inputs(scene, packed)
        g, a, o, b = _grad(g, a, o, b)
        args = (g, a, o, p, i, r, b, 40, 30, False, 0.2, 100.0)
        op = ops.rasterize_forward
        if name == "rasterize_bounded":
            args, op = args + (4096,), ops.rasterize_forward_bounded
    elif name == "rasterize_backward":
        g, a, o, p, i, r, b = _raster_inputs(scene, packed)
        maps, points, ranges, state, contributors = ops.rasterize_forward(
            g, a, o, p, i, r, b, 40, 30, False, 0.2, 100.0)
        grad_maps = torch.randn_like(maps)
        args = (g, a, o, p, b, points, ranges, state, contributors, grad_maps, 40, 30, False,
                0.2, 100.0)
        op = ops.rasterize_backward
    elif name == "pack_visible":
        args = (_records(scene, False)[8],)
        op = ops.pack_visible
    elif name == "bin_tiles":
        g, a, o, p, i, r, b = _raster_inputs(scene, packed)
        args = (g, r, i, b.shape[0], 40, 30)
        op = ops.bin_tiles
    else:
        gen = torch.Generator(device=device).manual_seed(3)
        keys = torch.randint(0, 2**62, (5000,), generator=gen, device=device)
        values = torch.arange(5000, dtype=torch.int32, device=device)
        args, op = (keys, values, 0, 64 if packed else 40), ops.sort_pairs
    torch.library.opcheck(op, args)


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_operators_equal_the_direct_calls():
    device = torch.device("cuda:0")
    scene = _scene(device)
    inputs = _raster_inputs(scene)
    via_op = ops.rasterize_forward(*inputs, 40, 30, False, 0.2, 100.0)
    direct = _native.rasterize_forward(*inputs, 40, 30, False, 0.2, 100.0)
    for a, b in zip(via_op, direct):
        assert torch.equal(a, b)
    bounded = ops.rasterize_forward_bounded(*inputs, 40, 30, False, 0.2, 100.0, 4096)
    m = direct[1].numel()
    assert bounded[5].tolist() == [0, m]
    assert torch.equal(bounded[0], direct[0]) and torch.equal(bounded[1][:m], direct[1])
    assert bool((bounded[1][m:] == -1).all())  # defined past the live count
    small = ops.rasterize_forward_bounded(*inputs, 40, 30, False, 0.2, 100.0, max(m // 2, 1))
    assert small[5].tolist() == [_native.BINNING_OVERFLOW, m]
    # Autograd through the operator gives the direct backward's gradients
    # (equal up to the order of the backward's float atomics).
    g, a, o, p, i, r, b = inputs
    leaves = _grad(g, a, o, b)
    maps = ops.rasterize_forward(leaves[0], leaves[1], leaves[2], p, i, r, leaves[3], 40, 30,
                                 False, 0.2, 100.0)[0]
    weights = torch.randn_like(maps)
    (maps * weights).sum().backward()
    expected = _native.rasterize_backward(g, a, o, p, b, direct[1], direct[2], direct[3],
                                          direct[4], weights, 40, 30, False, 0.2, 100.0)
    for leaf, want in zip(leaves, expected):
        torch.testing.assert_close(leaf.grad, want, rtol=1e-5, atol=1e-6)
