"""Tile dispatch orders cover every tile exactly once.

The compositors dispatch whole tiles longest first: the forward by list
length, or by the probed walk lengths of its pixels where the image holds
few rounds of workgroups (tile_probe_kernel), the backward by replay-list
length. No order changes any result, but each must be a permutation of the
tiles. Checked on images large enough not to be split into segments (2048
tiles or more): one 1080p image (list-length order), three images of 2079
tiles in all (probed order) and one image of 65,750 tiles:

* forward: every pixel of maps pre-filled with NaN, and every contributor
  count pre-filled with -7, is overwritten;
* backward: with dL/drgb = 1 and no other map gradient, each tile adds
  sum T (final transmittance) of its pixels to each background channel's
  gradient once, so that gradient equals H W - sum(alpha) per image.
"""

import pytest
import torch

from scenes import random_scene

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")

# (scenes, cameras, width, height)
SHAPES = [
    (1, 1, 1920, 1080),  # 8160 tiles: ordered by list length
    (3, 1, 515, 333),    # 3 x 693 = 2079 tiles: ordered by the probed walk lengths
    (1, 1, 4200, 4000),  # 65750 tiles
]


def scene(scenes, cameras, width, height, seed):
    raw = random_scene("classic", scenes=scenes, cameras=cameras, n=3000, width=width,
                       height=height, seed=seed, focal=0.35 * width)
    return {k: v.to(DEVICE) for k, v in raw.items()}


@pytest.mark.parametrize("shape", SHAPES)
def test_forward_writes_every_tile(shape):
    from diff_gabor_splatting_amd import _native, rasterize_gabors

    scenes, cameras, width, height = shape
    print(f"forward coverage {shape}", flush=True)
    values = scene(scenes, cameras, width, height, seed=41)
    captured = {}
    original = _native.rasterize_forward

    def spy(*args, **kwargs):
        captured["args"] = args
        return original(*args, **kwargs)

    _native.rasterize_forward = spy
    try:
        with torch.no_grad():
            rasterize_gabors(**values, width=width, height=height)
    finally:
        _native.rasterize_forward = original
    args = captured["args"]
    images = scenes * cameras
    groups = [torch.full((images, height, width, k), float("nan"), device=DEVICE)
              for k in _native.MAP_GROUPS]
    out = _native.rasterize_forward(*args[:12], outputs=groups)
    maps, _, ranges, state, contributors = out[:5]
    tw, th = _native.tile_grid(width, height)
    assert ranges.shape[0] == images * tw * th >= _native.SPLIT_MAX_TILES
    for group in maps:
        assert torch.isfinite(group).all()
    assert torch.isfinite(state).all()
    assert int(contributors.min()) >= 0


@pytest.mark.parametrize("shape", SHAPES[:2])
def test_backward_visits_every_tile_once(shape):
    from diff_gabor_splatting_amd import rasterize_gabors

    scenes, cameras, width, height = shape
    print(f"backward coverage {shape}", flush=True)
    values = scene(scenes, cameras, width, height, seed=43)
    backgrounds = values.pop("backgrounds").clone().requires_grad_()
    rgb, alpha, _ = rasterize_gabors(**values, backgrounds=backgrounds, width=width,
                                     height=height)
    rgb.sum().backward()
    transmittance = (width * height - alpha.detach().double().sum((-3, -2, -1)))
    expected = transmittance[..., None].expand(scenes, cameras, 3)
    torch.testing.assert_close(backgrounds.grad.double(), expected, rtol=1e-5, atol=1e-2)
