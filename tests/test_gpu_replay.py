"""Replay lists on the GPU.

The forward compositor can write, per tile, the point-list entries that at
least one of its pixels took, each with the bits of the 8x8 quadrants that
took it; the backward then replays only those. Checked here:
  * maps, state and contributors are bitwise the same with and without the
    lists;
  * the lists' structure at full config sizes (ascending positions inside
    the tile's list, entry ids equal to the point list's, a quadrant bit
    set, each pixel's last contributor listed in its quadrant, no record
    listed beyond the quadrant's largest contributor count);
  * on small scenes, the lists equal the float64 oracle's taken quadrants
    on every tile whose pixels are well-conditioned (in practice more than
    half of them, all of which must agree);
  * gradients with the lists equal those without (float atomic sums differ
    only in order).
"""

import numpy as np
import pytest
import torch

import bench
from oracle import composite as oracle_composite
from scenes import assert_gradients_close, random_scene

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")


def compositor_inputs(function, values, opts):
    """The public renderer's call into rasterize_forward: its 12 arguments."""
    from diff_gabor_splatting_amd import _native

    captured = {}
    original = _native.rasterize_forward

    def spy(*args, **kwargs):
        captured["args"] = args[:12]
        return original(*args, **kwargs)

    _native.rasterize_forward = spy
    try:
        with torch.no_grad():
            function(**values, **opts)
    finally:
        _native.rasterize_forward = original
    return captured["args"]


def renderer(neural):
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    return rasterize_neural_gabors if neural else rasterize_gabors


def decode(lists, counts, ranges):
    """Flat arrays over every listed entry: tile, position, id, quadrant bits."""
    lists, counts, ranges = (t.cpu().numpy() for t in (lists, counts, ranges))
    tiles = np.repeat(np.arange(len(counts)), counts)
    index = ranges[tiles, 0] + (np.arange(len(tiles)) - np.repeat(np.cumsum(counts) - counts, counts))
    words = lists[index, 1].astype(np.int64) & 0xFFFFFFFF
    return tiles, words & ((1 << 28) - 1), lists[index, 0], words >> 28


def quadrant_last(contributors, width, height):
    """Largest contributor count per (tile, quadrant): [tiles, 4]."""
    c = contributors.cpu().numpy()
    images = c.shape[0]
    tw, th = (width + 15) // 16, (height + 15) // 16
    py, px = np.meshgrid(np.arange(height), np.arange(width), indexing="ij")
    tile = (py // 16) * tw + px // 16
    quad = 2 * ((py % 16) >= 8) + ((px % 16) >= 8)
    out = np.zeros((images * tw * th, 4), dtype=np.int64)
    for image in range(images):
        np.maximum.at(out, (image * tw * th + tile, quad), c[image])
    return out, tile, quad


def check_structure(point_list, ranges, contributors, lists, counts, width, height):
    tiles, pos, ids, quads = decode(lists, counts, ranges)
    r = ranges.cpu().numpy()
    lengths = r[:, 1] - r[:, 0]
    assert np.all(counts.cpu().numpy() <= lengths)
    assert np.all(pos < lengths[tiles])
    same = tiles[1:] == tiles[:-1]
    assert np.all(pos[1:][same] > pos[:-1][same]), "positions ascend within a tile"
    np.testing.assert_array_equal(ids, point_list.cpu().numpy()[r[tiles, 0] + pos])
    assert np.all((quads >= 1) & (quads <= 15))
    last, tile, quad = quadrant_last(contributors, width, height)
    for q in range(4):
        listed = (quads >> q) & 1 == 1
        assert np.all(pos[listed] < last[tiles[listed], q]), "listed beyond every contributor"
    # Every pixel's last contributor is listed with the pixel's quadrant bit.
    bits = np.zeros(max(point_list.numel(), 1), dtype=np.int64)
    bits[r[tiles, 0] + pos] = quads
    c = contributors.cpu().numpy()
    tw, th = (width + 15) // 16, (height + 15) // 16
    for image in range(c.shape[0]):
        has = c[image] > 0
        t = image * tw * th + tile[has]
        at = r[t, 0] + c[image][has] - 1
        assert np.all((bits[at] >> quad[has]) & 1 == 1), "a last contributor is missing"
    return tiles, pos, quads


def forward_both(args):
    from diff_gabor_splatting_amd import _native

    # Unsplit tiles on both sides (split tiles, checked in test_gpu_split.py,
    # are independent of the replay lists too).
    plain = _native.rasterize_forward(*args, split=0)
    replayed = _native.rasterize_forward(*args, replay=True, split=0)
    assert replayed[5] is not None
    for a, b in zip(plain, replayed[:5]):
        assert torch.equal(a, b)
    return replayed


def backward_both(args, forward, seed):
    from diff_gabor_splatting_amd import _native

    geometry, appearance, opacities, primitive_ids, _, _, backgrounds = args[:7]
    width, height, neural, near, far = args[7:12]
    maps, point_list, ranges, state, contributors, replay = forward
    generator = torch.Generator().manual_seed(seed)
    grad_maps = torch.randn(maps.shape, generator=generator).to(DEVICE)
    saved = (geometry, appearance, opacities, primitive_ids, backgrounds, point_list, ranges,
             state, contributors, grad_maps, width, height, neural, near, far)
    plain = _native.rasterize_backward(*saved)
    replayed = _native.rasterize_backward(*saved, replay=replay)
    for name, a, b in zip(("geometry", "appearance", "opacities", "backgrounds"), plain,
                          replayed):
        assert torch.isfinite(b).all(), name
        assert_gradients_close(b, a, name)
    return plain


@pytest.mark.parametrize("index", [1, 2, 3, 4])
def test_config_replay_lists(index):
    cfg = bench.CONFIGS[index]
    print(f"replay lists: config {index}", flush=True)
    values = {k: v.to(DEVICE) for k, v in bench.make_scene(index).items()}
    opts = dict(width=cfg["width"], height=cfg["height"], packed=cfg["packed"])
    if not cfg["neural"]:
        opts["sh_degree"] = cfg["sh"]
    args = compositor_inputs(renderer(cfg["neural"]), values, opts)
    forward = forward_both(args)
    _, point_list, ranges, _, contributors, (lists, counts, _) = forward
    tiles, _, quads = check_structure(point_list, ranges, contributors, lists, counts,
                                      cfg["width"], cfg["height"])
    # The lists are much shorter than the tiles' lists up to their last contributor.
    assert 0 < len(tiles) < point_list.numel()
    backward_both(args, forward, seed=index)


@pytest.mark.parametrize("neural", [False, True])
@pytest.mark.parametrize("seed", [0, 1])
def test_replay_lists_match_oracle(neural, seed):
    method = "neural" if neural else "classic"
    width, height = 48, 40
    values = random_scene(method, scenes=2, cameras=2, n=160, width=width, height=height,
                          seed=seed)
    print(f"replay lists vs oracle: {method} seed {seed}", flush=True)
    gpu = {k: v.to(DEVICE) for k, v in values.items()}
    args = compositor_inputs(renderer(neural), gpu, dict(width=width, height=height))
    forward = forward_both(args)
    _, point_list, ranges, _, contributors, (lists, counts, _) = forward
    tiles, pos, quads = check_structure(point_list, ranges, contributors, lists, counts,
                                        width, height)
    geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds = (
        a.detach().cpu() for a in args[:7])
    taken, margins = {}, {}
    oracle_composite.composite(
        geometry.double(), appearance.double(), opacities.double(), primitive_ids, image_ids,
        radii, backgrounds.double(), width, height, neural, args[10], args[11],
        lists=(point_list.cpu().numpy(), ranges.cpu().numpy()), margins=margins, taken=taken,
    )
    expected = taken["quadrants"]
    actual = np.zeros_like(expected)
    actual[tiles, pos] = quads
    # Tiles whose every pixel keeps its discrete decisions away from their
    # thresholds (relative margin 1e-5, ~80 float32 ulps) must agree exactly.
    _, tile, _ = quadrant_last(contributors, width, height)
    margin = margins["pixels"].numpy()
    tw, th = (width + 15) // 16, (height + 15) // 16
    clean = np.ones(len(expected), dtype=bool)
    for image in range(margin.shape[0]):
        np.logical_and.at(clean, image * tw * th + tile, margin[image] > 1e-5)
    assert clean.sum() >= len(clean) // 2, (clean.sum(), len(clean))
    np.testing.assert_array_equal(actual[clean], expected[clean])
    backward_both(args, forward, seed=seed)


def test_empty_tiles_have_empty_lists():
    values = random_scene("classic", n=8, width=64, height=64, seed=4)
    values["opacities"].zero_()  # nothing reaches alpha 1/255: no pixel takes a record
    gpu = {k: v.to(DEVICE) for k, v in values.items()}
    args = compositor_inputs(renderer(False), gpu, dict(width=64, height=64))
    forward = forward_both(args)
    assert int(forward[5][1].sum()) == 0
    gg, ga, go, gb = backward_both(args, forward, seed=5)
    assert not gg.any() and not ga.any() and not go.any()


@pytest.mark.parametrize("neural", [False, True])
def test_lists_only_when_a_backward_can_follow(neural):
    """Under torch.no_grad the renderer prepares no replay lists, even when
    leaves that require gradients (the neural opacities) reach the
    compositor directly; with gradients recorded it does."""
    from diff_gabor_splatting_amd import _native

    method = "neural" if neural else "classic"
    values = random_scene(method, n=16, width=32, height=32, seed=6)
    gpu = {k: v.to(DEVICE).requires_grad_() for k, v in values.items()}
    requested = []
    original = _native.rasterize_forward

    def spy(*args, **kwargs):
        requested.append(kwargs.get("replay", False))
        return original(*args, **kwargs)

    _native.rasterize_forward = spy
    try:
        with torch.no_grad():
            renderer(neural)(**gpu, width=32, height=32)
        rgb, _, _ = renderer(neural)(**gpu, width=32, height=32)
    finally:
        _native.rasterize_forward = original
    assert requested == [False, True]
    rgb.sum().backward()
    assert gpu["opacities"].grad is not None
