"""Golden fixtures (tests/golden/*.npz): the oracle reproduces them on the CPU
and the HIP path reproduces them on the GPU."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import binning

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_case(name):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    data = np.load(GOLDEN / f"{name}.npz")
    inputs = {k[3:]: data[k] for k in data.files if k.startswith("in_")}
    outputs = {k[4:]: data[k] for k in data.files if k.startswith("out_")}
    return module, module.CASES[name], inputs, outputs


CASES = ["classic_tile", "neural_tile", "classic_sh2_multitile", "neural_multitile_packed"]


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    module, spec, inputs, expected = load_case(name)
    actual = module.render_case(spec, inputs)
    for key, value in expected.items():
        if value.dtype.kind in "iu":
            np.testing.assert_array_equal(actual[key], value, err_msg=key)
        else:
            np.testing.assert_allclose(actual[key], value, atol=1e-12, rtol=1e-10, err_msg=key)


def test_oracle_reproduces_binning_fixture():
    data = np.load(GOLDEN / "binning_random.npz")
    width, height, images = (int(v) for v in data["meta"])
    keys, point_list, ranges = binning.bin_pairs(data["geometry"], data["radii"], data["image_ids"],
                                                 images, width, height)
    np.testing.assert_array_equal(keys, data["sorted_keys"])
    np.testing.assert_array_equal(point_list, data["point_list"])
    np.testing.assert_array_equal(ranges, data["ranges"])


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
@pytest.mark.parametrize("name", CASES)
def test_hip_reproduces_fixture(name):
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors
    from scenes import assert_gradients_close, describe_mismatch, maps_from_result

    module, spec, inputs, expected = load_case(name)
    device = torch.device("cuda:0")
    values = {k: torch.from_numpy(v).to(device).requires_grad_() for k, v in inputs.items()}
    fn = rasterize_gabors if spec["method"] == "classic" else rasterize_neural_gabors
    options = {k: spec[k] for k in ("sh_degree", "packed") if k in spec}
    result = fn(**values, width=spec["width"], height=spec["height"], **options)
    maps = maps_from_result(result)
    np.testing.assert_array_equal(result[2]["radii"].cpu().numpy(), expected["radii"])
    # 1e-5 / 1e-4 plus four times each value's float32-scale sensitivity.
    actual = maps.detach().cpu().double().numpy()
    bound = 1e-5 + 1e-4 * np.abs(expected["maps"]) + 4 * expected["maps_sensitivity"]
    worst = np.abs(actual - expected["maps"]) - bound
    assert (worst <= 0).all(), describe_mismatch(torch.from_numpy(actual), torch.from_numpy(expected["maps"]))
    weights = module.weights_for(maps.shape).float().to(device)
    grads = torch.autograd.grad((maps * weights).sum(), list(values.values()), allow_unused=True)
    for key, grad in zip(values, grads):
        e = torch.from_numpy(expected[f"grad_{key}"])
        a = torch.zeros_like(e) if grad is None else grad.cpu()
        assert_gradients_close(a, e, key, torch.from_numpy(expected[f"gradsens_{key}"]))


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_hip_reproduces_binning_fixture():
    from diff_gabor_splatting_amd import _native

    data = np.load(GOLDEN / "binning_random.npz")
    width, height, images = (int(v) for v in data["meta"])
    device = torch.device("cuda:0")
    g, r, ids = (torch.from_numpy(data[k]).to(device) for k in ("geometry", "radii", "image_ids"))
    offsets = _native.count_tiles(g, r, width, height)
    keys, values = _native.emit_tiles(g, r, ids, offsets, width, height, int(offsets[-1]))
    tw, th = _native.tile_grid(width, height)
    sorted_keys, point_list = _native.sort_pairs(keys, values, 0, _native.sort_end_bit(images * tw * th))
    np.testing.assert_array_equal(sorted_keys.cpu().numpy().view(np.uint64), data["sorted_keys"])
    np.testing.assert_array_equal(point_list.cpu().numpy(), data["point_list"])
    np.testing.assert_array_equal(_native.find_ranges(sorted_keys, images * tw * th).cpu().numpy(),
                                  data["ranges"])
