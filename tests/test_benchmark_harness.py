"""The loop / fused-dense / fused-packed benchmark harness.

CPU: command-line defaults and errors, the synthetic scene's distributions,
and that the parity gate rejects an implementation whose maps or gradients
differ from the per-camera loop (strategies replaced by a small
differentiable CPU function). GPU: a tiny end-to-end run whose report
carries the reference harness's keys, and the compositor kernels' names.
"""

import json

import pytest
import torch

from diff_gabor_splatting_amd import benchmark_rasterization as harness


def test_defaults_follow_the_reference_harness():
    work, output = harness.parse_workload([])
    assert (work.method, work.num_primitives, work.num_scenes, work.num_cameras) == (
        "both", 10_000, 1, 4)
    assert (work.image_width, work.image_height) == (256, 256)
    assert (work.warmup_iterations, work.measurement_iterations, work.seed) == (5, 20, 42)
    assert work.profile_iterations == 0 and not work.skip_validation
    assert output is None and work.methods == ("classic", "neural")


@pytest.mark.parametrize("flag", ["--num-primitives", "--num-cameras", "--image-width",
                                  "--measurement-iterations"])
def test_nonpositive_sizes_are_rejected(flag):
    with pytest.raises(SystemExit):
        harness.parse_workload([flag, "0"])


def test_timed_regions_pause_the_garbage_collector():
    import gc

    from diff_gabor_splatting_amd.timing import paused_collector

    was = gc.isenabled()
    try:
        gc.enable()
        with paused_collector():
            assert not gc.isenabled()
        assert gc.isenabled()
        gc.disable()
        with paused_collector():
            pass
        assert not gc.isenabled()  # a caller's own pause is kept
    finally:
        (gc.enable if was else gc.disable)()


@pytest.mark.parametrize("flag", ["--warmup-iterations", "--profile-iterations"])
def test_negative_counts_are_rejected(flag):
    with pytest.raises(SystemExit):
        harness.parse_workload([flag, "-1"])
    harness.parse_workload([flag, "0"])


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_scene_follows_the_reference_distributions(method):
    """The reference harness's scene (benchmarks/benchmark_rasterization.py:
    16-64), drawn on the CPU: the same seed gives the same tensors."""
    work, _ = harness.parse_workload(["--num-primitives", "3000", "--num-scenes", "2",
                                      "--num-cameras", "3", "--image-width", "80",
                                      "--image-height", "48", "--method", method])
    scene = harness.synthesize(work, method, torch.device("cpu"))
    again = harness.synthesize(work, method, torch.device("cpu"))
    assert all(torch.equal(scene[k], again[k]) for k in scene)
    means = scene["means"]
    assert means.shape == (2, 3000, 3)
    assert float(means[..., 2].min()) >= 3 and float(means[..., 2].max()) <= 5
    assert abs(float(means[..., :2].std()) - 0.6) < 0.03
    q = scene["quaternions"]
    torch.testing.assert_close(q.norm(dim=-1), torch.ones(2, 3000))
    assert float(q[..., 0].min()) > 0.5
    assert bool((scene["scales"] == 0.025).all()) and bool((scene["opacities"] == 0.3).all())
    views, K = scene["view_matrices"], scene["intrinsics"]
    assert views.shape == (2, 3, 4, 4)
    torch.testing.assert_close(views[0, :, 0, 3], torch.tensor([-0.2, 0.0, 0.2]))
    torch.testing.assert_close(K[0, 0], torch.tensor([[64.0, 0, 39.5], [0, 38.4, 23.5],
                                                      [0, 0, 1.0]]))
    assert bool((scene["backgrounds"] == 0.05).all())
    optimised = {k for k, v in scene.items() if v.requires_grad}
    assert optimised == set(scene) - set(harness.CAMERA_INPUTS)
    if method == "classic":
        assert bool((scene["frequency_weights"] == 0.25).all())
        assert bool((scene["frequency_magnitudes"] == 1).all())
        assert not scene["phases"].any()
        assert 0 <= float(scene["colors"].min()) and float(scene["colors"].max()) <= 1
    else:
        for name, bound in (("input_weights", 0.2), ("input_biases", 0.2),
                            ("output_weights", 1 / 30), ("output_biases", 0.1)):
            assert float(scene[name].abs().max()) <= bound, name
        assert scene["input_weights"].shape == (2, 3000, 6, 5)


class _FakeStrategy:
    """Stand-in renderer: maps = f(parameters), plus a small term
    offset * sum(sin(wiggle * means)) whose value stays tiny while its
    derivative is wiggle times larger."""

    def __init__(self, offset=0.0, wiggle=1.0, name="fake"):
        self.offset, self.wiggle, self.name = offset, wiggle, name

    def maps(self, scene):
        base = torch.outer(scene["means"].sin(), scene["scales"].exp())
        return base + self.offset * (self.wiggle * scene["means"]).sin().sum()


def _fake_scene():
    gen = torch.Generator().manual_seed(3)
    scene = {
        "means": torch.rand(5, generator=gen, dtype=torch.float64),
        "scales": torch.rand(4, generator=gen, dtype=torch.float64),
        "backgrounds": torch.rand(3, generator=gen, dtype=torch.float64),
    }
    for name, value in scene.items():
        value.requires_grad_(name != "backgrounds")
    return scene


def test_parity_gate_accepts_equal_implementations():
    candidates = {"loop": _FakeStrategy(), "fused_dense": _FakeStrategy(), "fused_packed": _FakeStrategy()}
    record = harness.parity_gate(_fake_scene(), candidates, "loop")
    assert set(record) == {"fused_dense", "fused_packed"}
    assert all(row["max_map_error"] == 0 and row["max_gradient_error"] == 0
               for row in record.values())


@pytest.mark.parametrize("offset, wiggle, what", [(1e-3, 1.0, "maps differ"),
                                                  (1e-6, 5000.0, "means gradient error")])
@pytest.mark.parametrize("implementation", ["fused_dense", "fused_packed"])
def test_parity_gate_rejects_a_differing_implementation(implementation, offset, wiggle, what):
    """Maps off by 1e-3, or maps within 1e-5 but the means gradient off by
    about 1e-2 of its scale: both are rejected."""
    candidates = {"loop": _FakeStrategy(), "fused_dense": _FakeStrategy(),
                  "fused_packed": _FakeStrategy()}
    candidates[implementation] = _FakeStrategy(offset, wiggle)
    with pytest.raises(harness.ParityError, match=rf"{implementation} differs from loop: .*{what}"):
        harness.parity_gate(_fake_scene(), candidates, "loop")


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_tiny_run_reports_every_implementation(tmp_path):
    output = tmp_path / "report.json"
    harness.run([
        "--num-primitives", "1500", "--num-scenes", "2", "--num-cameras", "2",
        "--image-width", "80", "--image-height", "48", "--warmup-iterations", "1",
        "--measurement-iterations", "2", "--profile-iterations", "1",
        "--output-json", str(output),
    ])
    report = json.loads(output.read_text())
    assert set(report) >= {"environment", "workload", "timing", "profiling", "memory", "parity",
                           "results"}
    assert report["workload"]["num_primitives"] == 1500
    for method in ("classic", "neural"):
        parity = report["parity"][method]
        assert set(parity) == {"fused_dense", "fused_packed"}
        assert all(row["map_excess"] == 0 for row in parity.values())
    rows = {(r["method"], r["implementation"]): r for r in report["results"]}
    assert set(rows) == {(m, i) for m in ("classic", "neural") for i in harness.IMPLEMENTATIONS}
    for (method, implementation), row in rows.items():
        for key in ("forward_ms", "backward_ms", "forward_backward_ms", "images_per_second",
                    "peak_allocated_memory_mb", "forward_kernel_ms", "backward_kernel_ms"):
            assert row[key] > 0, (method, implementation, key)
        assert row["forward_backward_ms"] == pytest.approx(row["forward_ms"] + row["backward_ms"])
        assert row["images_per_second"] == pytest.approx(4000 / row["forward_backward_ms"])
    for method in ("classic", "neural"):
        assert rows[(method, "single_view_loop")]["speedup_vs_single_view_loop"] == 1.0


def test_bench_reads_committed_counter_summaries():
    import bench

    workload = bench.CONFIGS[4]["name"]
    traffic = bench.measured_traffic("render_backward", workload)
    assert traffic is None or traffic > 0
    valu = bench.measured_valu("render_backward", workload, 1.9)
    if valu is not None:
        assert valu["issue_ms"] == pytest.approx(valu["instructions"] / bench.VALU_ISSUE_PER_S * 1e3,
                                                 rel=1e-3)
        assert valu["frac"] == pytest.approx(valu["issue_ms"] / 1.9, rel=1e-3)
    assert bench.measured_valu("render_backward", "another workload", 1.9) is None
    assert bench.measured_traffic("render_backward", "another workload") is None


@pytest.mark.parametrize("channels", [9, 5])
def test_bench_loss_is_the_reference_objective(channels):
    import bench

    g = torch.Generator().manual_seed(3)
    shape = (1, 2, 5, 7)
    groups = [torch.randn(shape + (k,), generator=g, dtype=torch.float64, requires_grad=True)
              for k in (3, 1, 1, 3, 1)]
    rgb, alpha, depth, normals, distortion = groups
    meta = {"accumulated_depth": depth, "normals": normals, "distortion": distortion}
    loss = bench._loss(rgb, alpha, meta, channels)
    got = torch.autograd.grad(loss, groups, allow_unused=True)
    # The reference benchmark's form: concatenate, keep the channels, mean of squares.
    expected = torch.cat(groups, -1)[..., :channels].square().mean()
    want = torch.autograd.grad(expected, groups)
    assert loss.item() == pytest.approx(expected.item(), rel=1e-12)
    for g_got, g_want in zip(got, want):
        if g_got is None:  # groups past `channels` get no gradient (zero in the reference form)
            assert not g_want.any()
        else:
            torch.testing.assert_close(g_got, g_want, rtol=1e-12, atol=0)


def test_compositor_kernels_carry_the_reference_names():
    """The compositor kernels are named renderForward / renderBackward as in
    the reference (rasterize.cu:230, :284), so trace tools that split kernel
    time by those names find them."""
    import shutil
    import subprocess

    from diff_gabor_splatting_amd import _native

    if shutil.which("nm") is None:
        pytest.skip("needs nm")
    symbols = subprocess.run(["nm", "-C", str(_native._LIBRARY_PATH)], capture_output=True,
                             text=True).stdout
    for name in ("renderForward<", "renderBackward<"):
        assert name in symbols, name


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_profiler_finds_the_compositor_kernels():
    """A torch.profiler trace of one step holds kernels whose names contain
    "renderForward<" and "renderBackward<", the split the reference's
    benchmark makes (benchmarks/benchmark_rasterization.py:152-178)."""
    import gabor_splatting
    from scenes import maps_from_result, random_scene

    raw = random_scene("classic", scenes=1, cameras=2, n=200, width=40, height=30, seed=4)
    values = {k: v.cuda().requires_grad_() for k, v in raw.items()}
    gabor_splatting.rasterize_gabors(**values, width=40, height=30)  # warm-up
    torch.cuda.synchronize()
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU,
                                            torch.profiler.ProfilerActivity.CUDA]) as trace:
        maps = maps_from_result(gabor_splatting.rasterize_gabors(**values, width=40, height=30))
        maps.square().mean().backward()
        torch.cuda.synchronize()
    names = {event.name for event in trace.events()
             if event.device_type == torch.autograd.DeviceType.CUDA}
    assert any("renderForward<" in name for name in names), sorted(names)[:20]
    assert any("renderBackward<" in name for name in names), sorted(names)[:20]
