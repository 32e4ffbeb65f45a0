"""Host-side contracts of the public API that fail before any GPU work."""

import pytest
import torch

from diff_gabor_splatting_amd import _native, rasterize_gabors, rasterize_neural_gabors
from diff_gabor_splatting_amd import rendering
from scenes import make_inputs


def test_drop_in_module_paths():
    import gabor_splatting
    import gabor_splatting.rendering as alias

    assert alias is rendering
    assert gabor_splatting.rasterize_gabors is rasterize_gabors
    assert alias.SHColors is rendering.SHColors
    assert callable(alias.check_values)


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_cpu_tensors_are_rejected(method):
    values = make_inputs(method)
    function = rasterize_gabors if method == "classic" else rasterize_neural_gabors
    with pytest.raises(ValueError, match="CUDA float32"):
        function(**values, width=9, height=9)


def test_scalar_option_errors():
    values = make_inputs("classic")
    bad_means = dict(values, means=values["means"][..., :2])
    with pytest.raises(ValueError, match=r"\[..., N, 3\]"):
        rasterize_gabors(**bad_means, width=9, height=9)


def test_check_tensor_messages():
    device = torch.device("cpu")
    with pytest.raises(TypeError):
        rendering.check_tensor("scales", [1.0], (1,), device)
    with pytest.raises(ValueError, match="scales must be float32"):
        rendering.check_tensor("scales", torch.zeros(2, dtype=torch.float64), (2,), device)


def test_quaternion_matrix_is_a_rotation():
    q = torch.randn(10, 4, dtype=torch.float64)
    R = rendering.quaternion_matrix(q)
    torch.testing.assert_close(R @ R.transpose(-1, -2), torch.eye(3, dtype=torch.float64).expand(10, 3, 3))


def test_overflow_guards_are_pure_host_functions():
    _native.check_intersections(2**31 - 1)
    with pytest.raises(RuntimeError, match="intersection count exceeds int32"):
        _native.check_intersections(2**31)
    _native.check_image_tiles(1, 16, 16)
    with pytest.raises(RuntimeError, match="image tile count exceeds int32"):
        _native.check_image_tiles(2**20, 2**16, 2**16)
    assert _native.tile_grid(1920, 1080) == (120, 68)
    assert _native.sort_end_bit(120 * 68) == 45


def test_fixed_capacity_arguments_and_nesting():
    from diff_gabor_splatting_amd import fixed_capacity

    for bad in (0, -5, 2**31, 3.0, True):
        with pytest.raises(ValueError, match="max_intersections"):
            fixed_capacity(bad)
    outer, inner = fixed_capacity(10), fixed_capacity(20)
    with outer:
        assert rendering._FIXED_CAPACITY[-1] is outer
        with inner:
            assert rendering._FIXED_CAPACITY[-1] is inner
        assert rendering._FIXED_CAPACITY[-1] is outer
    assert rendering._FIXED_CAPACITY == []
    outer.check()  # nothing recorded: no synchronisation, no error
