"""gs_render_forward_static: the forward compositor without a caller workspace.

Its only scratch, the tiles' dispatch order, lives in a static device array
instead of a workspace the caller allocates. Called through the C ABI on the
same inputs as gs_render_forward, it must produce the same maps, state,
contributor counts and replay lists, bit for bit, on consecutive calls of
different sizes (the second smaller, so stale scratch from the first call
would show). Its refusal of more tiles than the scratch holds returns before
any HIP call, so that case runs on the CPU (test_abi.py).
"""

import pytest
import torch

from scenes import random_scene

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")


def _library():
    from diff_gabor_splatting_amd import _native

    return _native


def compositor_inputs(method, seed, n, width, height, scenes, cameras):
    """The inputs the public API hands to the forward compositor: records,
    point list and ranges of a random scene."""
    native = _library()
    raw = random_scene(method, scenes=scenes, cameras=cameras, n=n, width=width,
                       height=height, seed=seed)
    values = {k: v.to(DEVICE) for k, v in raw.items()}
    captured = {}
    original = native.rasterize_forward

    def spy(*args, **kwargs):
        out = original(*args, **kwargs)
        captured["args"] = args
        captured["lists"] = out[1:3]
        return out

    native.rasterize_forward = spy
    try:
        from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

        render = rasterize_gabors if method == "classic" else rasterize_neural_gabors
        with torch.no_grad():
            render(**values, width=width, height=height)
    finally:
        native.rasterize_forward = original
    return captured["args"], captured["lists"]


def call(entry, args, lists):
    """Run one forward entry point through the C ABI; returns its outputs."""
    native = _library()
    (geometry, appearance, opacities, primitive_ids, _, _, backgrounds, width, height, neural,
     near_plane, far_plane) = args[:12]
    point_list, ranges = lists
    images = backgrounds.shape[0]
    tw, th = native.tile_grid(width, height)
    maps = torch.full((images, height, width, 9), float("nan"), device=DEVICE)
    state = torch.full((images, height, width, 3), float("nan"), device=DEVICE)
    contributors = torch.full((images, height, width), -7, dtype=torch.int32, device=DEVICE)
    replay = torch.full((max(point_list.numel(), 1), 2), -1, dtype=torch.int32, device=DEVICE)
    counts = torch.full((images * tw * th,), -1, dtype=torch.int32, device=DEVICE)
    groups, strides = native._map_group_args(native.split_map_groups(maps), "maps")
    common = (int(bool(neural)), geometry.data_ptr(), appearance.data_ptr(),
              opacities.data_ptr(), primitive_ids.data_ptr(), backgrounds.data_ptr(),
              point_list.data_ptr(), ranges.data_ptr(), images, width, height, near_plane,
              far_plane, groups, strides, state.data_ptr(), contributors.data_ptr(),
              replay.data_ptr(), point_list.numel(), counts.data_ptr())
    stream = torch.cuda.current_stream(DEVICE).cuda_stream
    if entry == "static":
        status = native.lib.gs_render_forward_static(*common, stream)
    else:
        workspace = torch.empty(native.lib.gs_render_workspace_size(images, width, height),
                                dtype=torch.uint8, device=DEVICE)
        status = native.lib.gs_render_forward(*common, 0, None, None, 0, workspace.data_ptr(),
                                              workspace.numel(), stream)
    assert status == 0, native.lib.gs_last_error()
    torch.cuda.synchronize()
    return maps, state, contributors, replay, counts


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_static_forward_equals_workspace_forward(method):
    # Two calls in a row, the second with fewer images and tiles.
    for seed, n, width, height, scenes, cameras in ((31, 900, 150, 97, 2, 2),
                                                    (32, 300, 61, 40, 1, 1)):
        print(f"static forward {method} {scenes}x{cameras} {width}x{height}", flush=True)
        args, lists = compositor_inputs(method, seed, n, width, height, scenes, cameras)
        expected = call("workspace", args, lists)
        actual = call("static", args, lists)
        for name, a, e in zip(("maps", "state", "contributors", "replay", "counts"), actual,
                              expected):
            assert torch.equal(a, e) or (a.is_floating_point() and
                                         torch.equal(a.nan_to_num(9.0), e.nan_to_num(9.0))), name
        assert torch.isfinite(actual[0]).all()
        assert int(actual[2].min()) >= 0

