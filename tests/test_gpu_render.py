"""Public-API parity on the GPU: the reference's own test cases
(tests/test_rendering.py) against the float64 oracle, plus drop-in contracts."""

import math

import numpy as np
import pytest
import torch

from oracle import render as oracle_render
from scenes import (assert_gradients_close, fp32_conditioned, make_inputs, maps_from_result,
                    oracle_reference, pixel_reference, random_scene)

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")
ORACLE = {"classic": oracle_render.rasterize_gabors, "neural": oracle_render.rasterize_neural_gabors}


def renderer(method):
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    return rasterize_gabors if method == "classic" else rasterize_neural_gabors


def on_gpu(values):
    return {k: v.to(DEVICE).requires_grad_() for k, v in values.items()}


def oracle_maps(method, values, width, height, **options):
    """float64 oracle maps and the leaf tensors they differentiate against."""
    leaves = {k: v.detach().cpu().double().requires_grad_() for k, v in values.items()}
    rest = dict(leaves)
    backgrounds = rest.pop("backgrounds")
    maps, meta, aux = ORACLE[method](**rest, width=width, height=height, backgrounds=backgrounds,
                                     **options)
    return maps, meta, aux, leaves


def grads(output, weights, leaves):
    out = torch.autograd.grad((output * weights).sum(), list(leaves.values()), allow_unused=True,
                              retain_graph=True)
    return [torch.zeros_like(v) if g is None else g for g, v in zip(out, leaves.values())]


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("packed", [False, True])
def test_reference_outputs_and_gradients(method, packed):
    values = on_gpu(make_inputs(method))
    actual = maps_from_result(renderer(method)(**values, width=9, height=9, packed=packed))
    expected = pixel_reference(method, {k: v.detach().cpu() for k, v in values.items()})
    torch.testing.assert_close(actual.detach().cpu().double(), expected, atol=3e-6, rtol=2e-5)
    oracle, _, _, leaves = oracle_maps(method, values, 9, 9, packed=packed)
    torch.testing.assert_close(actual.detach().cpu().double(), oracle.detach(), atol=1e-6, rtol=1e-5)
    weights = torch.linspace(-0.4, 0.7, actual.numel()).reshape(actual.shape)
    actual_grads = grads(actual, weights.to(DEVICE), values)
    expected_grads = grads(oracle, weights.double(), leaves)
    for name, a, e in zip(values, actual_grads, expected_grads):
        torch.testing.assert_close(a.cpu().double(), e, atol=2e-5, rtol=1e-4, msg=name)


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("packed", [False, True])
def test_scene_camera_batch_matches_loop(method, packed):
    values = on_gpu(make_inputs(method, scenes=2, cameras=3))
    result = maps_from_result(renderer(method)(**values, width=9, height=9, packed=packed))
    views = []
    for scene in range(2):
        per_camera = []
        for camera in range(3):
            subset = {
                k: v[scene, camera:camera + 1].contiguous()
                if k in ("view_matrices", "intrinsics", "backgrounds") else v[scene].contiguous()
                for k, v in values.items()
            }
            per_camera.append(maps_from_result(renderer(method)(**subset, width=9, height=9)))
        views.append(torch.cat(per_camera))
    repeated = torch.stack(views)
    torch.testing.assert_close(result, repeated)
    a = torch.autograd.grad(result.square().sum(), list(values.values()), retain_graph=True)
    e = torch.autograd.grad(repeated.square().sum(), list(values.values()))
    for name, x, y in zip(values, a, e):
        torch.testing.assert_close(x, y, atol=4e-3, rtol=1e-3, msg=name)


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("empty", [False, True])
def test_empty_and_invisible_scenes(method, packed, empty):
    raw = make_inputs(method, primitives=0 if empty else 3)
    if not empty:
        raw["means"][..., 2] = -2
    values = on_gpu(raw)
    rgb, alpha, meta = renderer(method)(**values, width=9, height=9, packed=packed)
    torch.testing.assert_close(rgb, values["backgrounds"][:, :, None, None, :].expand_as(rgb))
    assert alpha.count_nonzero() == 0
    maps_from_result((rgb, alpha, meta)).sum().backward()
    for name, value in values.items():
        assert value.grad is not None and torch.isfinite(value.grad).all(), name
        if name != "backgrounds":
            assert value.grad.count_nonzero() == 0, name


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_leading_dimensions_and_stream(method):
    with torch.cuda.stream(torch.cuda.Stream()):
        values = {k: v.reshape(2, 2, *v.shape[1:]) for k, v in on_gpu(make_inputs(method, scenes=4)).items()}
        rgb, alpha, _ = renderer(method)(**values, width=9, height=9, packed=True)
        (rgb.sum() + alpha.sum()).backward()
        assert rgb.shape == (2, 2, 2, 9, 9, 3)
    torch.cuda.synchronize()


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_invalid_contracts(method):
    original = on_gpu(make_inputs(method))
    for name, replacement in [
        ("means", original["means"].double()),
        ("scales", -original["scales"]),
        ("quaternions", torch.zeros_like(original["quaternions"])),
        ("opacities", torch.full_like(original["opacities"], 2)),
        ("intrinsics", original["intrinsics"].transpose(-1, -2)),
    ]:
        with pytest.raises(ValueError):
            renderer(method)(**dict(original, **{name: replacement}), width=9, height=9)
    with pytest.raises(ValueError):
        renderer(method)(**original, width=0, height=9)
    with pytest.raises(TypeError):
        renderer(method)(**original, width=9, height=9, packed=1)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_classic_sh_batches(degree):
    from diff_gabor_splatting_amd import rasterize_gabors

    raw = make_inputs("classic", scenes=2)
    g = torch.Generator().manual_seed(degree)
    for name in ("colors", "secondary_colors"):
        raw[name] = torch.rand(2, 3, (degree + 1) ** 2, 3, generator=g) * 0.4
    values = on_gpu(raw)
    dense = maps_from_result(rasterize_gabors(**values, width=9, height=9, sh_degree=degree))
    packed = maps_from_result(rasterize_gabors(**values, width=9, height=9, sh_degree=degree, packed=True))
    torch.testing.assert_close(dense, packed)
    oracle, _, _, leaves = oracle_maps("classic", values, 9, 9, sh_degree=degree)
    torch.testing.assert_close(dense.detach().cpu().double(), oracle.detach(), atol=1e-6, rtol=1e-5)
    weights = torch.linspace(-1, 1, dense.numel()).reshape(dense.shape)
    for name, a, e in zip(values, grads(dense, weights.to(DEVICE), values), grads(oracle, weights.double(), leaves)):
        torch.testing.assert_close(a.cpu().double(), e, atol=2e-5, rtol=1e-4, msg=name)
    assert values["colors"].grad is None  # grads() does not accumulate
    dense.sum().backward()
    assert values["colors"].grad.abs().sum() > 0
    assert values["secondary_colors"].grad.abs().sum() > 0


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("opacity", [0.0, 1.0])
def test_opacity_cutoff_and_saturation(method, opacity):
    raw = make_inputs(method, cameras=1, primitives=7)
    raw["opacities"].fill_(0.85 if opacity == 1.0 else opacity)
    raw["opacities"][..., 0] = opacity
    raw["quaternions"].zero_()
    raw["quaternions"][..., 0] = 1
    raw["means"][..., :2] = 0
    values = on_gpu(raw)
    actual = maps_from_result(renderer(method)(**values, width=9, height=9))
    oracle, _, _, leaves = oracle_maps(method, values, 9, 9)
    torch.testing.assert_close(actual.detach().cpu().double(), oracle.detach(), atol=3e-6, rtol=3e-5)
    ones = torch.ones(actual.shape)
    for name, a, e in zip(values, grads(actual, ones.to(DEVICE), values), grads(oracle, ones.double(), leaves)):
        torch.testing.assert_close(a.cpu().double(), e, atol=2e-4, rtol=1e-3, msg=name)


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_tiny_surfaces_use_lowpass_filter(method):
    raw = make_inputs(method, cameras=1, primitives=1)
    raw["scales"].fill_(0.02)
    raw["quaternions"].zero_()
    raw["quaternions"][..., 0] = 1
    values = on_gpu(raw)
    actual = maps_from_result(renderer(method)(**values, width=9, height=9))
    oracle, _, _, leaves = oracle_maps(method, values, 9, 9)
    torch.testing.assert_close(actual.detach().cpu().double(), oracle.detach(), atol=2e-6, rtol=2e-5)
    ones = torch.ones(actual.shape)
    for name, a, e in zip(values, grads(actual, ones.to(DEVICE), values), grads(oracle, ones.double(), leaves)):
        torch.testing.assert_close(a.cpu().double(), e, atol=5e-4, rtol=1e-3, msg=name)


@pytest.mark.parametrize("degree", [0, 3])
def test_empty_sh_scene(degree):
    from diff_gabor_splatting_amd import rasterize_gabors

    values = on_gpu(make_inputs("classic", primitives=0))
    for name in ("colors", "secondary_colors"):
        values[name] = torch.empty((1, 0, (degree + 1) ** 2, 3), device=DEVICE, requires_grad=True)
    result = rasterize_gabors(**values, width=9, height=9, sh_degree=degree, packed=True)
    maps_from_result(result).sum().backward()
    assert values["colors"].grad.shape == values["colors"].shape


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_parameter_finite_differences(method):
    values = on_gpu(make_inputs(method, cameras=1, primitives=1))
    names = ["means", "scales", "opacities", "phases" if method == "classic" else "input_biases"]
    weights = torch.linspace(-0.2, 0.4, 81 * 9, device=DEVICE).reshape(1, 1, 9, 9, 9)

    def objective():
        maps = maps_from_result(renderer(method)(**values, width=9, height=9))
        return (maps.double() * weights).sum()

    gradients = torch.autograd.grad(objective(), [values[n] for n in names])
    for name, gradient in zip(names, gradients):
        parameter = values[name]
        index = (0,) * parameter.ndim
        step = 5e-4
        original = parameter[index].item()
        with torch.no_grad():
            parameter[index] = original + step
            plus = objective().item()
            parameter[index] = original - step
            minus = objective().item()
            parameter[index] = original
        torch.testing.assert_close(gradient[index].double().cpu(),
                                   torch.tensor((plus - minus) / (2 * step), dtype=torch.float64),
                                   atol=3e-3, rtol=8e-3, msg=name)


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_float32_inputs_ignore_global_default_dtype(method):
    values = on_gpu(make_inputs(method, cameras=1, primitives=1))
    previous = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.float64)
        rgb, alpha, _ = renderer(method)(**values, width=9, height=9)
        (rgb.sum() + alpha.sum()).backward()
        assert rgb.dtype == torch.float32 and alpha.dtype == torch.float32
    finally:
        torch.set_default_dtype(previous)


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("case", ["edge_on", "degenerate_conic"])
def test_degenerate_surfaces_have_finite_zero_gradients(method, case):
    raw = make_inputs(method, cameras=1, primitives=1)
    raw["view_matrices"].copy_(torch.eye(4))
    raw["means"][0, 0] = torch.tensor([0.0, 0.0, 3.0])
    raw["quaternions"].fill_(0.5)
    if case == "degenerate_conic":
        raw["scales"].fill_(1.0)
        raw["means"][..., 0] = 0.1
    values = on_gpu(raw)
    rgb, alpha, meta = renderer(method)(**values, width=9, height=9, packed=True)
    assert alpha.count_nonzero() == 0
    maps_from_result((rgb, alpha, meta)).sum().backward()
    for name, value in values.items():
        assert value.grad is not None and torch.isfinite(value.grad).all(), name
        if name != "backgrounds":
            assert value.grad.count_nonzero() == 0, name


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_trusted_input_path_skips_only_value_checks(method, monkeypatch):
    import gabor_splatting.rendering as rendering

    values = on_gpu(make_inputs(method))
    expected = maps_from_result(renderer(method)(**values, width=9, height=9))

    def unexpected(*args):
        raise AssertionError("check_values should not be called")

    monkeypatch.setattr(rendering, "check_values", unexpected)
    actual = maps_from_result(renderer(method)(**values, width=9, height=9, validate=False))
    torch.testing.assert_close(actual, expected)
    a = torch.autograd.grad(actual.sum(), list(values.values()), retain_graph=True)
    e = torch.autograd.grad(expected.sum(), list(values.values()))
    for x, y in zip(a, e):
        torch.testing.assert_close(x, y, atol=2e-3, rtol=1e-3)
    with pytest.raises(ValueError, match="scales must be float32"):
        renderer(method)(**dict(values, scales=values["scales"].double()), width=9, height=9,
                         validate=False)


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_shared_batch_boundary_matches_reference(method):
    raw = make_inputs(method, cameras=1, primitives=65)
    raw["opacities"].fill_(0.03)
    values = on_gpu(raw)
    actual = maps_from_result(renderer(method)(**values, width=9, height=9))
    oracle, _, _, leaves = oracle_maps(method, values, 9, 9)
    torch.testing.assert_close(actual.detach().cpu().double(), oracle.detach(), atol=4e-6, rtol=3e-5)
    weights = torch.linspace(-0.4, 0.7, actual.numel()).reshape(actual.shape)
    for name, a, e in zip(values, grads(actual, weights.to(DEVICE), values), grads(oracle, weights.double(), leaves)):
        torch.testing.assert_close(a.cpu().double(), e, atol=2e-4, rtol=1e-3, msg=name)


@pytest.mark.parametrize("packed", [False, True])
def test_projected_means_gradient_is_the_screen_filter_term(packed):
    from diff_gabor_splatting_amd import rasterize_gabors

    values = on_gpu(make_inputs("classic", scenes=1, cameras=2, primitives=3))
    rgb, alpha, meta = rasterize_gabors(**values, width=9, height=9, packed=packed)
    meta["projected_means"].retain_grad()
    maps_from_result((rgb, alpha, meta)).square().sum().backward()
    oracle, oracle_meta, _, leaves = oracle_maps("classic", values, 9, 9, packed=packed)
    oracle_meta["projected_means"].retain_grad()
    oracle.square().sum().backward()
    torch.testing.assert_close(meta["projected_means"].grad.cpu().double(),
                               oracle_meta["projected_means"].grad, atol=2e-5, rtol=1e-4)
    for key in ("scene_ids", "camera_ids", "primitive_ids", "radii"):
        np.testing.assert_array_equal(meta[key].cpu().numpy(), oracle_meta[key].numpy())


@pytest.mark.parametrize("method, sh", [("classic", None), ("classic", 2), ("neural", None)])
@pytest.mark.parametrize("packed", [False, True])
def test_multi_tile_scenes_match_oracle(method, sh, packed):
    width, height = 45, 37  # partial edge tiles
    raw = random_scene(method, scenes=2, cameras=2, n=150, width=width, height=height, seed=11, sh=sh)
    values = on_gpu(raw)
    options = dict(packed=packed) if sh is None else dict(packed=packed, sh_degree=sh)
    rgb, alpha, meta = renderer(method)(**values, width=width, height=height, **options)
    actual = maps_from_result((rgb, alpha, meta))
    # Radii must agree with the float32 oracle; the float64 oracle then
    # composites with the same radii.
    oracle32 = ORACLE[method](**{k: v.detach().cpu() for k, v in values.items() if k != "backgrounds"},
                              width=width, height=height,
                              backgrounds=values["backgrounds"].detach().cpu(), **options)
    np.testing.assert_array_equal(meta["radii"].cpu().numpy(), oracle32[1]["radii"].numpy())
    oracle, _, aux, leaves = oracle_maps(method, values, width, height, **options)
    # Random orientations: compare on pixels that are well conditioned at
    # float32 precision (see scenes.fp32_conditioned).
    rest = {k: v for k, v in values.items() if k != "backgrounds"}
    _, mask = fp32_conditioned(
        lambda backgrounds, **kw: ORACLE[method](**kw, backgrounds=backgrounds),
        {**rest, "backgrounds": values["backgrounds"]}, width=width, height=height, **options)
    assert float((~mask).float().mean()) <= 0.03
    torch.testing.assert_close(actual.detach().cpu().double()[mask], oracle.detach()[mask],
                               atol=1e-5, rtol=1e-4)
    weights = torch.randn(actual.shape, generator=torch.Generator().manual_seed(3)) * mask[..., None]
    _, expected, sensitivity = oracle_reference(ORACLE[method], values, weights, width=width,
                                                height=height, **options)
    for name, a in zip(values, grads(actual, weights.to(DEVICE), values)):
        assert_gradients_close(a, expected[name], name, sensitivity[name])


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_extreme_views_match_oracle(method):
    """Surfels that straddle the camera plane, lie nearly edge-on, or are huge
    and thin: the per-wave footprint cull must keep every pixel the oracle
    accepts, forward and backward."""
    width, height, n = 48, 40, 160
    g = torch.Generator().manual_seed(23)
    raw = random_scene(method, n=n, width=width, height=height, seed=23)
    raw["means"][..., :2] = (torch.rand(1, n, 2, generator=g) * 2 - 1) * 1.2
    raw["means"][..., 2] = torch.rand(1, n, generator=g) * 3.9 + 0.1
    raw["scales"] = torch.exp(torch.rand(1, n, 2, generator=g) * math.log(200) + math.log(0.01))
    # A quarter nearly edge-on: normal (local z) close to the image plane.
    tilt = torch.rand(n // 4, generator=g) * 0.02 + math.pi / 2 - 0.01
    axis = torch.zeros(n // 4, 3)
    axis[:, 0] = 1.0
    half = tilt / 2
    raw["quaternions"][0, : n // 4] = torch.cat(
        [half.cos()[:, None], axis * half.sin()[:, None]], -1)
    values = on_gpu(raw)
    actual = maps_from_result(renderer(method)(**values, width=width, height=height))
    oracle, _, _, _ = oracle_maps(method, values, width, height)
    rest = {k: v for k, v in values.items() if k != "backgrounds"}
    _, mask = fp32_conditioned(
        lambda backgrounds, **kw: ORACLE[method](**kw, backgrounds=backgrounds),
        {**rest, "backgrounds": values["backgrounds"]}, width=width, height=height)
    assert float((~mask).float().mean()) <= 0.05
    torch.testing.assert_close(actual.detach().cpu().double()[mask], oracle.detach()[mask],
                               atol=1e-5, rtol=1e-4)
    weights = torch.randn(actual.shape, generator=torch.Generator().manual_seed(4)) * mask[..., None]
    _, expected, sensitivity = oracle_reference(ORACLE[method], values, weights, width=width,
                                                height=height)
    for name, a in zip(values, grads(actual, weights.to(DEVICE), values)):
        assert_gradients_close(a, expected[name], name, sensitivity[name])


def test_unaligned_inputs_match_aligned():
    """Contiguous inputs need not start on a 16-byte boundary: vector loads
    are only used when every array allows them."""
    from diff_gabor_splatting_amd import rasterize_gabors

    values = on_gpu(random_scene("classic", n=200, width=40, height=32, seed=9, sh=3))
    shifted = {}
    for key, value in values.items():
        storage = torch.empty(value.numel() + 1, dtype=value.dtype, device=value.device)
        view = storage[1:].view(value.shape)  # 4 bytes past an aligned start
        view.copy_(value.detach())
        shifted[key] = view.requires_grad_(value.requires_grad)
    first = maps_from_result(rasterize_gabors(**values, width=40, height=32, sh_degree=3))
    second = maps_from_result(rasterize_gabors(**shifted, width=40, height=32, sh_degree=3))
    assert torch.equal(first, second)
    weights = torch.randn(first.shape, generator=torch.Generator().manual_seed(2)).to(DEVICE)
    for name, a, b in zip(values, grads(first, weights, values), grads(second, weights, shifted)):
        assert_gradients_close(a, b, name)


def test_forward_is_bitwise_deterministic():
    from diff_gabor_splatting_amd import rasterize_gabors

    values = on_gpu(random_scene("classic", n=400, width=64, height=64, seed=5, sh=3))
    first = maps_from_result(rasterize_gabors(**values, width=64, height=64, sh_degree=3))
    second = maps_from_result(rasterize_gabors(**values, width=64, height=64, sh_degree=3))
    assert torch.equal(first, second)


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_retained_graph_backward_twice(method):
    """The compositor's accumulators are cleared ahead of the first backward;
    a second backward through a retained graph must see fresh ones."""
    values = on_gpu(make_inputs(method, cameras=2, primitives=9))
    maps = maps_from_result(renderer(method)(**values, width=19, height=13))
    weights = torch.linspace(-1.0, 1.0, maps.numel(), device=DEVICE).reshape(maps.shape)
    first = torch.autograd.grad((maps * weights).sum(), list(values.values()), retain_graph=True)
    second = torch.autograd.grad((maps * weights).sum(), list(values.values()))
    for name, a, b in zip(values, first, second):
        # float atomics: compare at the scale of the tensor
        scale = max(float(b.abs().max()), 1.0)
        torch.testing.assert_close(a, b, atol=1e-6 * scale, rtol=1e-5, msg=name)
    with torch.no_grad():
        plain = maps_from_result(renderer(method)(**values, width=19, height=13))
    torch.testing.assert_close(plain, maps.detach())


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_fixed_cameras_skip_camera_gradients(method):
    """Cameras that do not require gradients get none, and the surfel
    gradients equal those of a render whose cameras do (to the order of the
    compositor's float atomics)."""
    inputs = make_inputs(method, cameras=2, primitives=9)
    fixed = on_gpu(inputs)
    for key in ("view_matrices", "intrinsics"):
        fixed[key] = fixed[key].detach()
    full = on_gpu(inputs)
    for values in (fixed, full):
        maps = maps_from_result(renderer(method)(**values, width=19, height=13))
        weights = torch.linspace(-1.0, 1.0, maps.numel(), device=DEVICE).reshape(maps.shape)
        (maps * weights).sum().backward()
    assert fixed["view_matrices"].grad is None and fixed["intrinsics"].grad is None
    assert full["view_matrices"].grad is not None and full["intrinsics"].grad is not None
    for name, value in fixed.items():
        if not value.requires_grad:
            continue
        want = full[name].grad
        scale = max(float(want.abs().max()), 1.0)
        torch.testing.assert_close(value.grad, want, atol=1e-6 * scale, rtol=1e-5, msg=name)


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_single_map_storage_is_the_reference_layout(method):
    """Inside single_map_storage() rgb, alpha and the three meta maps are
    views of one [..., C, H, W, 9] tensor, as in the reference
    (rendering.py:375-400): the same values as the grouped layout, bit for
    bit, the same gradients (atomic order aside), the reference's strides
    and shared base, and an in-place change of a view reaches the base."""
    from diff_gabor_splatting_amd import single_map_storage

    width, height = 45, 37
    print(f"single map storage: {method}", flush=True)
    raw = random_scene(method, scenes=2, cameras=2, n=150, width=width, height=height, seed=17)
    values = on_gpu(raw)
    grouped = renderer(method)(**values, width=width, height=height)
    with single_map_storage():
        rgb, alpha, meta = renderer(method)(**values, width=width, height=height)
    base = rgb._base
    assert base is not None and tuple(base.shape) == tuple(rgb.shape[:-1]) + (9,)
    for view in (alpha, meta["accumulated_depth"], meta["normals"], meta["distortion"]):
        assert view._base is base
    assert rgb.stride()[-2:] == (9, 1) and alpha.storage_offset() - rgb.storage_offset() == 3
    single_maps = maps_from_result((rgb, alpha, meta))
    grouped_maps = maps_from_result(grouped)
    assert torch.equal(single_maps, grouped_maps)
    assert torch.equal(base, grouped_maps)
    weights = torch.randn(single_maps.shape, generator=torch.Generator().manual_seed(6))
    weights = weights.to(DEVICE)
    for name, a, b in zip(values, grads(single_maps, weights, values),
                          grads(grouped_maps, weights, values)):
        assert torch.isfinite(a).all(), name
        assert_gradients_close(a, b, name)
    # The reference objective over the views, through an in-place change.
    with single_map_storage():
        rgb, alpha, meta = renderer(method)(**values, width=width, height=height)
    rgb.mul_(2.0)
    assert torch.equal(rgb._base[..., :3], 2 * grouped[0].detach())
    loss = torch.cat((rgb, alpha, meta["accumulated_depth"], meta["normals"],
                      meta["distortion"]), -1).square().mean()
    loss.backward()
    assert all(torch.isfinite(v.grad).all() for v in values.values())


@pytest.mark.parametrize("packed", [False, True])
def test_neural_gradients_by_parameter_group_equal_row_gradients(packed):
    """The neural renderer's backward writes the SIREN parameter groups'
    gradients in place (gs_render_backward's grad_appearance_columns); they
    equal the gradients of the concatenated rows that autograd slices back
    into the groups (the reference's path), up to the order of float
    atomics, and each arrives contiguous in its parameter's layout."""
    from diff_gabor_splatting_amd import rasterize_neural_gabors, rendering
    from scenes import random_scene

    values = {k: v.to(DEVICE) for k, v in random_scene(
        "neural", scenes=2, cameras=2, n=400, width=70, height=45, seed=21).items()}

    def run():
        leaves = {k: v.detach().clone().requires_grad_() for k, v in values.items()}
        maps = maps_from_result(rasterize_neural_gabors(**leaves, width=70, height=45,
                                                        packed=packed))
        weights = torch.linspace(-1, 1, maps.numel(), device=DEVICE).view_as(maps)
        (maps * weights).sum().backward()
        return maps.detach(), {k: v.grad for k, v in leaves.items()}

    saved = rendering._NEURAL_COLUMNS
    try:
        rendering._NEURAL_COLUMNS = False
        row_maps, row_grads = run()
        rendering._NEURAL_COLUMNS = True
        maps, grads = run()
    finally:
        rendering._NEURAL_COLUMNS = saved
    assert torch.equal(maps, row_maps)
    for name in ("input_weights", "input_biases", "output_weights", "output_biases"):
        assert grads[name].is_contiguous(), name
        assert bool(grads[name].abs().sum() > 0), name
    for name, grad in grads.items():
        scale = float(row_grads[name].abs().max()) if grad.numel() else 0.0
        torch.testing.assert_close(grad, row_grads[name], atol=1e-5 * max(scale, 1e-3),
                                   rtol=1e-5, msg=lambda m, name=name: f"{name}: {m}")


def test_default_backgrounds_are_kept_zeros():
    """Without backgrounds the renderers use kept zeros (no fill per call):
    made outside inference mode, so that a render under inference mode
    followed by a differentiated one works, and equal to explicit zeros."""
    from diff_gabor_splatting_amd import rasterize_gabors, rendering
    from scenes import random_scene

    values = {k: v.to(DEVICE) for k, v in random_scene(
        "classic", scenes=1, cameras=2, n=200, width=40, height=30, seed=23).items()}
    values["backgrounds"] = torch.zeros_like(values["backgrounds"])
    explicit = maps_from_result(rasterize_gabors(**values, width=40, height=30))
    del values["backgrounds"]
    rendering._ZERO_BACKGROUNDS.clear()
    with torch.inference_mode():
        first = maps_from_result(rasterize_gabors(**values, width=40, height=30))
    leaves = {k: v.detach().clone().requires_grad_() for k, v in values.items()}
    maps = maps_from_result(rasterize_gabors(**leaves, width=40, height=30))
    maps.sum().backward()
    assert torch.equal(first, explicit) and torch.equal(maps.detach(), explicit)
    assert all(v.grad is not None for v in leaves.values())
    kept = list(rendering._ZERO_BACKGROUNDS.values())
    assert len(kept) == 1 and not kept[0].is_inference() and not bool(kept[0].any())
