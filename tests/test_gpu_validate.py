"""The HIP value-contract kernel against the oracle and the planted answers.

Every planted violation of tests/contract_cases.py must produce exactly its
messages, in the reference's order, through ``rendering.check_values`` (one
launch of gs_check_values) and through the public renderers, which raise
ValueError before drawing anything. Larger scenes put violations in the
first and last element of every tensor, so that each job's first and tail
block is exercised, and an empty scene checks nothing.
"""

import math

import pytest
import torch

from contract_cases import FINITE, check_arguments, contract_cases, planted_inputs
from oracle.validate import value_violations
from scenes import make_inputs

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")


def on_gpu(values):
    return {name: value.to(DEVICE) for name, value in values.items()}


def hip_messages(values, method):
    from diff_gabor_splatting_amd import rendering

    try:
        rendering.check_values(*check_arguments(values, method))
    except ValueError as error:
        return str(error).split("; ")
    return []


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_planted_violations_match_the_oracle(method):
    for label, mutate, expected in contract_cases(method):
        values = planted_inputs(method, mutate)
        assert value_violations(*check_arguments(values, method)) == expected, label
        print(f"check_values {method} {label}", flush=True)
        assert hip_messages(on_gpu(values), method) == expected, label


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_renderer_raises_every_violation_before_drawing(method):
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    render = rasterize_gabors if method == "classic" else rasterize_neural_gabors
    values = on_gpu(make_inputs(method, cameras=2, primitives=5))
    values["scales"][0, 1, 0] = -1.0
    values["means"][0, 4, 2] = math.nan
    values["intrinsics"][0, 1, 2, 2] = 2.0
    with pytest.raises(ValueError) as error:
        render(**values, width=17, height=9)
    assert str(error.value) == "; ".join([
        FINITE.format("means"), "scales must be strictly positive",
        "intrinsics must have last row [0, 0, 1]",
    ])


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("where", ["first", "last"])
def test_multi_block_scenes_find_edge_violations(method, where):
    base = make_inputs(method, scenes=3, cameras=300, primitives=9000, seed=11)
    for name in base:
        planted = {k: v.clone() for k, v in base.items()}
        flat = planted[name].view(-1)
        flat[0 if where == "first" else flat.numel() - 1] = math.inf
        expected = value_violations(*check_arguments(planted, method))
        assert FINITE.format(name) in expected
        values = on_gpu(planted)
        print(f"check_values {method} {where} {name}", flush=True)
        assert hip_messages(values, method) == expected, name
    assert hip_messages(on_gpu(base), method) == []


def test_empty_scene_checks_nothing():
    values = on_gpu(make_inputs("classic", primitives=0))
    assert hip_messages(values, "classic") == []


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("packed", [False, True])
def test_renderer_reports_each_planted_violation(method, packed):
    """The renderers read the check's verdict back with the intersection
    count and raise it before compositing: the oracle's messages, every case."""
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    render = rasterize_gabors if method == "classic" else rasterize_neural_gabors
    for label, mutate, expected in contract_cases(method):
        values = on_gpu(planted_inputs(method, mutate))
        print(f"render {method} packed={packed} {label}", flush=True)
        if not expected:
            render(**values, width=17, height=9, packed=packed)
            continue
        with pytest.raises(ValueError) as error:
            render(**values, width=17, height=9, packed=packed)
        assert str(error.value).split("; ") == expected, label


def test_validated_render_synchronises_once(monkeypatch):
    """validate=True never takes the check's own read-back, and still raises."""
    from diff_gabor_splatting_amd import _native, rasterize_gabors

    def separate_read_back(*args, **kwargs):
        raise AssertionError("the value check was read back on its own")

    monkeypatch.setattr(_native, "check_values", separate_read_back)
    values = on_gpu(make_inputs("classic", cameras=2, primitives=5))
    rgb, _, _ = rasterize_gabors(**values, width=17, height=9)
    assert bool(torch.isfinite(rgb).all())
    values["opacities"][0, 2] = 1.5
    with pytest.raises(ValueError, match="opacities must lie in"):
        rasterize_gabors(**values, width=17, height=9)


def test_replaced_check_values_runs_in_place_of_the_kernel(monkeypatch):
    """A caller's replacement of rendering.check_values is called, as the
    reference calls it, once per validated render."""
    from diff_gabor_splatting_amd import rasterize_gabors, rendering

    calls = []
    monkeypatch.setattr(rendering, "check_values", lambda *args: calls.append(len(args)))
    values = on_gpu(make_inputs("classic", cameras=2, primitives=5))
    values["opacities"][0, 2] = 1.5  # the replacement accepts it
    rasterize_gabors(**values, width=17, height=9)
    rasterize_gabors(**values, width=17, height=9, validate=False)
    assert calls == [8]
