"""The loop / fused-dense / fused-packed benchmark harness.

CPU: command-line defaults and errors, and that the parity gate rejects an
implementation whose maps or gradients differ from the per-camera loop (the
renderer replaced by a small differentiable CPU function). GPU: a tiny
end-to-end run whose report carries the reference harness's keys.
"""

import json

import pytest
import torch

from diff_gabor_splatting_amd import benchmark_rasterization as harness


def test_defaults_follow_the_reference_harness():
    args = harness._parse([])
    assert (args.method, args.num_primitives, args.num_scenes, args.num_cameras) == (
        "both", 10_000, 1, 4)
    assert (args.image_width, args.image_height) == (256, 256)
    assert (args.warmup_iterations, args.measurement_iterations, args.seed) == (5, 20, 42)
    assert args.profile_iterations == 0 and not args.skip_validation
    assert args.output_json is None


@pytest.mark.parametrize("flag", ["--num-primitives", "--num-cameras", "--image-width",
                                  "--measurement-iterations"])
def test_nonpositive_sizes_are_rejected(flag):
    with pytest.raises(SystemExit):
        harness._parse([flag, "0"])


def test_negative_warmup_is_rejected():
    with pytest.raises(SystemExit):
        harness._parse(["--warmup-iterations", "-1"])


def _fake_renderer(offsets):
    """Stand-in for render_maps: maps = f(parameters) + an implementation offset."""
    def render(scene, args, method, implementation):
        base = torch.outer(scene["means"].sin(), scene["scales"].exp())
        return base + offsets.get(implementation, 0.0) * scene["means"].sum()
    return render


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


def test_parity_gate_accepts_equal_implementations(monkeypatch):
    monkeypatch.setattr(harness, "render_maps", _fake_renderer({}))
    harness.check_parity(_fake_scene(), harness._parse([]), "classic")


@pytest.mark.parametrize("implementation", ["fused_dense", "fused_packed"])
def test_parity_gate_rejects_a_differing_implementation(monkeypatch, implementation):
    monkeypatch.setattr(harness, "render_maps", _fake_renderer({implementation: 1e-3}))
    with pytest.raises(AssertionError):
        harness.check_parity(_fake_scene(), harness._parse([]), "classic")


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
    assert set(report) >= {"environment", "workload", "timing", "results"}
    assert report["workload"]["num_primitives"] == 1500
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
