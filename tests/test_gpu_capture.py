"""Rendering without host synchronisation, and inside a captured HIP graph.

Within ``fixed_capacity`` the point list has a fixed capacity and the
intersection count stays on the device (gs_bin_tiles_bounded), value checks
are deferred to ``check()``, and a whole forward + backward can be captured
in a graph. Each graph replay is compared with an eager render of the same
inputs, with eager work and synchronisations between the replays.
"""

import math

import pytest
import torch

from scenes import maps_from_result, random_scene

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")


def renderer(method):
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    return rasterize_gabors if method == "classic" else rasterize_neural_gabors


def scene(method, seed, n=300, width=70, height=45):
    raw = random_scene(method, scenes=1, cameras=2, n=n, width=width, height=height, seed=seed)
    return {k: v.to(DEVICE) for k, v in raw.items()}, dict(width=width, height=height)


def assert_grads_close(actual, expected, names, what):
    """Float atomics sum the gradients in a run-dependent order, and a render
    into a fixed-capacity point list picks its split-tile segment length
    from that capacity rather than from the intersection count, so the
    segments of a split tile (each starting from a checkpoint's prefix sums)
    can differ from the synchronised render's. Elements are compared at the
    scale of their tensor: 1e-4 of its largest value, ten times inside the
    oracle gradient bar."""
    for name, a, e in zip(names, actual, expected):
        scale = float(e.abs().max()) if e.numel() else 0.0
        torch.testing.assert_close(a, e, atol=1e-4 * max(scale, 1e-2), rtol=1e-4,
                                   msg=lambda m, name=name: f"{name} {what}: {m}")


def maps_and_grads(method, values, options, weights, **kwargs):
    leaves = {k: v.detach().clone().requires_grad_() for k, v in values.items()}
    maps = maps_from_result(renderer(method)(**leaves, **options, **kwargs))
    grads = torch.autograd.grad(maps, list(leaves.values()), grad_outputs=weights)
    return maps.detach(), grads


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_bounded_render_matches_synchronised_render(method):
    from diff_gabor_splatting_amd import fixed_capacity

    values, options = scene(method, seed=3)
    plain = maps_from_result(renderer(method)(**values, **options))
    weights = torch.linspace(-1, 1, plain.numel(), device=DEVICE).reshape(plain.shape)
    expected, expected_grads = maps_and_grads(method, values, options, weights)
    with fixed_capacity(1 << 20) as capacity:
        actual, grads = maps_and_grads(method, values, options, weights)
    peak = capacity.check()
    assert 0 < peak < 1 << 20
    with fixed_capacity(peak) as exact:  # a capacity of exactly M suffices
        tight, _ = maps_and_grads(method, values, options, weights)
    assert exact.check() == peak
    assert torch.equal(tight, expected)
    assert torch.equal(actual, expected)
    assert_grads_close(grads, expected_grads, list(values), "bounded")


@pytest.mark.parametrize("method, sh", [("classic", None), ("classic", 2), ("neural", None)])
def test_bounded_packed_render_keeps_one_row_per_pair(method, sh):
    """packed=True at a fixed capacity: the visible count stays on the device,
    so the packed outputs keep S*C*N rows, the packed rows first."""
    from diff_gabor_splatting_amd import fixed_capacity

    raw = random_scene(method, scenes=2, cameras=2, n=300, width=70, height=45, seed=21, sh=sh)
    raw["means"][:, ::5, 2] = -3.0  # a fifth of the surfels behind every camera
    values = {k: v.to(DEVICE) for k, v in raw.items()}
    options = dict(width=70, height=45, packed=True)
    if sh is not None:
        options["sh_degree"] = sh
    rgb, alpha, meta = renderer(method)(**values, **options)
    plain = maps_from_result((rgb, alpha, meta))
    weights = torch.linspace(-1, 1, plain.numel(), device=DEVICE).reshape(plain.shape)
    expected, expected_grads = maps_and_grads(method, values, options, weights)
    with fixed_capacity(1 << 20) as capacity:
        result = renderer(method)(**values, **options)
        actual, grads = maps_and_grads(method, values, options, weights)
    assert capacity.check() > 0
    assert torch.equal(actual, expected) and torch.equal(maps_from_result(result), expected)
    assert_grads_close(grads, expected_grads, list(values), "bounded packed")

    padded = result[2]
    visible, pairs = meta["radii"].numel(), 2 * 2 * 300
    assert 0 < visible <= pairs * 4 // 5 and padded["packed"] is True
    assert padded["radii"].shape == (pairs,) and padded["projected_means"].shape == (pairs, 2)
    for key in ("radii", "projected_means", "scene_ids", "camera_ids", "primitive_ids"):
        assert torch.equal(padded[key][:visible], meta[key]), key
    assert int(padded["radii"][visible:].abs().sum()) == 0
    assert int(padded["projected_means"][visible:].abs().sum()) == 0
    for key in ("scene_ids", "camera_ids", "primitive_ids"):
        assert bool((padded[key][visible:] == -1).all()), key


def test_overflow_is_reported_by_check():
    from diff_gabor_splatting_amd import fixed_capacity

    values, options = scene("classic", seed=5)
    with fixed_capacity(7) as capacity:
        renderer("classic")(**values, **options)
    with pytest.raises(RuntimeError, match=r"tile intersections \(\d+\) exceeded the fixed capacity of 7"):
        capacity.check()
    assert capacity.check() == 0  # the flags were consumed


def test_value_checks_are_deferred():
    from diff_gabor_splatting_amd import fixed_capacity

    values, options = scene("classic", seed=6)
    values["scales"][0, 3, 1] = -1.0
    values["means"][0, 7, 0] = math.nan
    with fixed_capacity(1 << 20) as capacity:
        renderer("classic")(**values, **options)  # does not raise here
        renderer("classic")(**values, **options, packed=True)
    with pytest.raises(ValueError) as error:
        capacity.check()
    assert str(error.value) == ("means must contain only finite values; "
                                "scales must be strictly positive")


@pytest.mark.parametrize("method, packed", [("classic", False), ("neural", False),
                                            ("classic", True)])
def test_graph_replays_match_eager(method, packed):
    from diff_gabor_splatting_amd import fixed_capacity

    base, options = scene(method, seed=11)
    options["packed"] = packed
    static = {k: v.detach().clone().requires_grad_() for k, v in base.items()}
    probe = maps_from_result(renderer(method)(**base, **options))
    weights = torch.linspace(-1, 1, probe.numel(), device=DEVICE).reshape(probe.shape)

    def step():
        maps = maps_from_result(renderer(method)(**static, **options, validate=False))
        grads = torch.autograd.grad(maps, list(static.values()), grad_outputs=weights)
        return maps, grads

    capacity = fixed_capacity(1 << 20)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with capacity, torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with capacity, torch.cuda.graph(graph):
        static_maps, static_grads = step()
    capacity.check()

    for replay, seed in enumerate((11, 12, 13)):
        values, _ = scene(method, seed=seed)
        with torch.no_grad():
            for name, value in values.items():
                static[name].copy_(value)
        print(f"graph replay {method} packed={packed} {replay}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        expected, expected_grads = maps_and_grads(method, values, options, weights)
        assert torch.equal(static_maps, expected), replay
        assert_grads_close(static_grads, expected_grads, list(values), f"replay {replay}")
        capacity.check()


def test_forward_captured_alone():
    """A render whose inputs require gradients also clears the backward's
    accumulators (on a side stream outside fixed_capacity); inside it
    nothing is left unjoined, so a forward can be captured alone and its
    replays render the eager maps."""
    from diff_gabor_splatting_amd import fixed_capacity

    method = "classic"
    base, options = scene(method, seed=14)
    static = {k: v.detach().clone().requires_grad_() for k, v in base.items()}
    capacity = fixed_capacity(1 << 20)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with capacity, torch.cuda.stream(side):
        maps_from_result(renderer(method)(**static, **options))
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with capacity, torch.cuda.graph(graph):
        static_maps = maps_from_result(renderer(method)(**static, **options))
    capacity.check()
    for replay, seed in enumerate((14, 15)):
        values, _ = scene(method, seed=seed)
        with torch.no_grad():
            for name, value in values.items():
                static[name].copy_(value)
        print(f"forward-only replay {replay}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        expected = maps_from_result(renderer(method)(**values, **options))
        assert torch.equal(static_maps.detach(), expected), replay
        capacity.check()


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_bounded_render_of_an_empty_view(method):
    """No surfel in front of the camera: zero intersections on the device."""
    from diff_gabor_splatting_amd import fixed_capacity

    values, options = scene(method, seed=8, n=20)
    values["means"][..., 2] = -3.0  # behind every camera
    expected = maps_from_result(renderer(method)(**values, **options))
    with fixed_capacity(64) as capacity:
        actual = maps_from_result(renderer(method)(**values, **options))
    assert capacity.check() == 0
    assert torch.equal(actual, expected)
    background = values["backgrounds"][:, :, None, None, :].expand_as(actual[..., :3])
    torch.testing.assert_close(actual[..., :3], background)


def test_check_reports_each_replay_of_a_captured_graph():
    """A check right after capture reads nothing (no kernel ran yet); every
    later check reports the replays since the one before: within capacity
    it returns the intersection count, a replay that overflows the capacity
    or carries a violated value contract raises."""
    from diff_gabor_splatting_amd import fixed_capacity

    method = "classic"
    base, options = scene(method, seed=11)
    static = {k: v.detach().clone() for k, v in base.items()}
    probe = fixed_capacity(1 << 20)
    with probe:
        renderer(method)(**static, **options)
    exact = probe.check()
    assert exact > 0

    def step():
        return maps_from_result(renderer(method)(**static, **options, validate=True))

    capacity = fixed_capacity(exact)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with capacity, torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    assert capacity.check() == exact  # the eager warm-up render
    graph = torch.cuda.CUDAGraph()
    with capacity, torch.cuda.graph(graph):
        static_maps = step()
    assert capacity.check() == 0  # captured, not yet replayed

    print("replay within capacity", flush=True)
    graph.replay()
    expected = maps_from_result(renderer(method)(**base, **options))
    assert torch.equal(static_maps, expected)
    assert capacity.check() == exact
    assert capacity.check() == 0  # nothing replayed since

    print("replay past capacity", flush=True)
    with torch.no_grad():
        static["scales"].mul_(3.0)  # larger footprints: more tile intersections
    graph.replay()
    with pytest.raises(RuntimeError, match=rf"exceeded the fixed capacity of {exact}"):
        capacity.check()

    print("replay within capacity again", flush=True)
    with torch.no_grad():
        static["scales"].copy_(base["scales"])
    graph.replay()
    assert capacity.check() == exact

    print("replay with invalid values", flush=True)
    with torch.no_grad():
        static["opacities"][0, 4] = 1.5
    graph.replay()
    with pytest.raises(ValueError, match="opacities must lie in"):
        capacity.check()
    assert capacity.check() == 0
