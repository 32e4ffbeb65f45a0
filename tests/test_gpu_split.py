"""Split tiles: long tile lists are composited in segments (one workgroup
each, merged per pixel afterwards) and their backward replayed in segments,
each from a checkpoint the merge wrote.

* Maps agree with the unsplit forward to float32 rounding (merged segments
  reassociate the sums) and the contributor counts are identical (the stop
  rule is decided exactly); gradients agree with the unsplit backward to
  float32 rounding (each segment's running suffix is derived from prefix-sum
  differences instead of accumulated).
* The checkpoint layout: slot bases in tile order for exactly the tiles
  longer than the segment length, non-decreasing replay lengths ending at
  the tile's replay count, and a last checkpoint equal to the saved state.
* Gradients of a scene whose tiles are split match the float64 oracle.
"""

import pytest
import torch

from diff_gabor_splatting_amd import _native
from oracle import render as oracle_render
from scenes import (assert_gradients_close, fp32_conditioned, maps_from_result,
                    oracle_reference, random_scene)

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")
ORACLE = {"classic": oracle_render.rasterize_gabors, "neural": oracle_render.rasterize_neural_gabors}


def renderer(method):
    from diff_gabor_splatting_amd import rasterize_gabors, rasterize_neural_gabors

    return rasterize_gabors if method == "classic" else rasterize_neural_gabors


def heavy_scene(method, opacity, n=900, width=40, height=36, seed=5):
    raw = random_scene(method, scenes=1, cameras=2, n=n, width=width, height=height, seed=seed)
    raw["opacities"] = torch.full_like(raw["opacities"], opacity)
    return {k: v.to(DEVICE).requires_grad_() for k, v in raw.items()}


def spy_forward(monkeypatch):
    """Records every rasterize_forward result."""
    seen = []
    original = _native.rasterize_forward

    def spy(*args, **kwargs):
        out = original(*args, **kwargs)
        seen.append(out)
        return out

    monkeypatch.setattr(_native, "rasterize_forward", spy)
    return seen


def run(method, values, weights, width, height):
    maps = maps_from_result(renderer(method)(**values, width=width, height=height))
    grads = torch.autograd.grad((maps * weights).sum(), list(values.values()), allow_unused=True)
    return maps.detach(), [torch.zeros_like(v) if g is None else g
                           for g, v in zip(grads, values.values())]


@pytest.mark.parametrize("method", ["classic", "neural"])
@pytest.mark.parametrize("opacity", [0.3, 0.97])
def test_split_backward_matches_unsplit(method, opacity, monkeypatch):
    width, height = 40, 36
    values = heavy_scene(method, opacity, width=width, height=height)
    weights = torch.randn((1, 2, height, width, 9), generator=torch.Generator().manual_seed(8))
    weights = weights.to(DEVICE)
    print(f"split vs unsplit: {method} opacity {opacity}", flush=True)
    seen = spy_forward(monkeypatch)
    split_maps, split_grads = run(method, values, weights, width, height)
    segments = seen[-1][5][2]
    assert segments is not None, "the scene was not split"
    tiles = seen[-1][2].shape[0]
    assert int((segments[2][:tiles] >= 0).sum()) > 0
    monkeypatch.setattr(_native, "SPLIT_MAX_TILES", 0)
    split_contributors = seen[-1][4]
    plain_maps, plain_grads = run(method, values, weights, width, height)
    assert seen[-1][5][2] is None
    assert torch.equal(split_contributors, seen[-1][4])
    torch.testing.assert_close(split_maps, plain_maps, atol=2e-6, rtol=2e-5)
    # Both sides round differently (atomic order, reassociated sums), as any
    # float32 implementation does against the float64 oracle: the oracle's
    # gradient bar, 1e-3 of the tensor's largest value, with a wrong term
    # off by far more.
    for name, a, b in zip(values, split_grads, plain_grads):
        scale = float(b.abs().max())
        err = float((a - b).abs().max())
        assert err <= 1e-3 * scale + 1e-12, f"{name}: max error {err:.3e}, scale {scale:.3e}"


@pytest.mark.parametrize("opacity", [0.3, 0.97])
def test_checkpoint_layout(opacity, monkeypatch):
    width, height = 40, 36
    values = heavy_scene("classic", opacity, width=width, height=height)
    seen = spy_forward(monkeypatch)
    renderer("classic")(**values, width=width, height=height)
    maps, point_list, ranges, state, contributors, (lists, counts, segments) = seen[-1]
    length, checkpoints, index = segments
    tiles = ranges.shape[0]
    lengths = (ranges[:, 1] - ranges[:, 0]).long().cpu()
    base = index[:tiles].long().cpu()
    split = lengths > length
    assert bool(((base >= 0) == split).all())
    # Slots in tile order: each split tile takes ceil(L / length) of them.
    need = (lengths + length - 1) // length
    expected_base = torch.cumsum(torch.where(split, need, 0), 0) - torch.where(split, need, 0)
    assert torch.equal(base[split], expected_base[split])
    replayed = index[tiles:].long().cpu()
    counts = counts.long().cpu()
    state_cpu = state.cpu()
    ck = checkpoints.cpu()
    tw, th = _native.tile_grid(width, height)
    for t in torch.nonzero(split).flatten().tolist():
        n = replayed[base[t]:base[t] + need[t]]
        assert bool((n[1:] >= n[:-1]).all()) and int(n[-1]) == int(counts[t]) and int(n[0]) >= 0
        image, local = divmod(t, tw * th)
        ty, tx = divmod(local, tw)
        last = ck[base[t] + need[t] - 1]  # [10, 256]: the final state of the tile's pixels
        pix = torch.arange(256)
        wave, lane = pix // 64, pix % 64
        px = tx * 16 + (wave % 2) * 8 + lane % 8
        py = ty * 16 + (wave // 2) * 8 + lane // 8
        inside = (px < width) & (py < height)
        saved = state_cpu[image, py[inside], px[inside]]
        assert torch.equal(last[0, inside], saved[:, 0])
        assert torch.equal(last[8, inside], saved[:, 1])
        assert torch.equal(last[9, inside], saved[:, 2])


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_split_scene_matches_oracle(method, monkeypatch):
    width, height = 36, 20
    raw = random_scene(method, scenes=1, cameras=2, n=260, width=width, height=height, seed=21)
    values = {k: v.to(DEVICE).requires_grad_() for k, v in raw.items()}
    seen = spy_forward(monkeypatch)
    rgb, alpha, meta = renderer(method)(**values, width=width, height=height)
    actual = maps_from_result((rgb, alpha, meta))
    segments = seen[-1][5][2]
    assert segments is not None and int((segments[2][:seen[-1][2].shape[0]] >= 0).sum()) > 0
    rest = {k: v for k, v in values.items() if k != "backgrounds"}
    oracle_maps, mask = fp32_conditioned(
        lambda backgrounds, **kw: ORACLE[method](**kw, backgrounds=backgrounds),
        {**rest, "backgrounds": values["backgrounds"]}, width=width, height=height)
    assert float((~mask).float().mean()) <= 0.03
    torch.testing.assert_close(actual.detach().cpu().double()[mask], oracle_maps[mask],
                               atol=1e-5, rtol=1e-4)
    weights = torch.randn(actual.shape, generator=torch.Generator().manual_seed(4)) * mask[..., None]
    _, expected, sensitivity = oracle_reference(ORACLE[method], values, weights, width=width,
                                                height=height)
    grads = torch.autograd.grad((actual * weights.to(DEVICE)).sum(), list(values.values()),
                                allow_unused=True)
    for (name, v), g in zip(values.items(), grads):
        g = torch.zeros_like(v) if g is None else g
        assert_gradients_close(g, expected[name], name, sensitivity[name])


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_forward_bits_do_not_depend_on_grad_mode(method):
    """Tiles are split whether or not a backward follows (the replay lists
    are only written when one can), so a render's maps are the same bits
    with and without gradient recording."""
    width, height = 40, 36
    values = heavy_scene(method, 0.5, width=width, height=height)
    with torch.no_grad():
        frozen = maps_from_result(renderer(method)(**values, width=width, height=height))
    recorded = maps_from_result(renderer(method)(**values, width=width, height=height))
    assert recorded.requires_grad
    assert torch.equal(frozen, recorded.detach())


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_slots_past_capacity_leave_later_tiles_unsplit(method, monkeypatch):
    """With fewer checkpoint slots than the long tiles need, the first long
    tiles (in tile order) are split and later ones are walked whole inside
    the split launch; the forward's work list and the backward's segment
    order then mix split and unsplit long tiles. Contributor counts equal
    the unsplit render's, maps and gradients agree with it to float32
    rounding."""
    width, height = 40, 36
    values = heavy_scene(method, 0.5, width=width, height=height)
    weights = torch.randn((1, 2, height, width, 9), generator=torch.Generator().manual_seed(9))
    weights = weights.to(DEVICE)
    print(f"slots past capacity: {method}", flush=True)
    seen = spy_forward(monkeypatch)
    with torch.no_grad():
        renderer(method)(**values, width=width, height=height)
    ranges = seen[-1][2]
    lengths = (ranges[:, 1] - ranges[:, 0]).long().cpu()
    need = (lengths + _native.SPLIT_LENGTH - 1) // _native.SPLIT_LENGTH
    long_need = need[lengths > _native.SPLIT_LENGTH]
    assert len(long_need) >= 2, "the scene needs two long tiles"
    # Slots for the first long tile (in tile order) only.
    capacity = int(long_need[0])
    monkeypatch.setattr(_native, "SPLIT_MAX_SLOTS", capacity)
    capped_maps, capped_grads = run(method, values, weights, width, height)
    ranges, contributors, (_, _, segments) = seen[-1][2], seen[-1][4], seen[-1][5]
    length, checkpoints, index = segments
    assert checkpoints.shape[0] == capacity
    tiles = ranges.shape[0]
    lengths = (ranges[:, 1] - ranges[:, 0]).long().cpu()
    base = index[:tiles].long().cpu()
    long_tiles = lengths > length
    split = base >= 0
    assert int(split.sum()) > 0, "no tile was split"
    assert int((long_tiles & ~split).sum()) > 0, "every long tile was split"
    assert bool((split <= long_tiles).all())
    monkeypatch.setattr(_native, "SPLIT_MAX_TILES", 0)
    plain_maps, plain_grads = run(method, values, weights, width, height)
    assert seen[-1][5][2] is None
    assert torch.equal(contributors, seen[-1][4])
    torch.testing.assert_close(capped_maps, plain_maps, atol=2e-6, rtol=2e-5)
    for name, a, b in zip(values, capped_grads, plain_grads):
        scale = float(b.abs().max())
        err = float((a - b).abs().max())
        assert err <= 1e-3 * scale + 1e-12, f"{name}: max error {err:.3e}, scale {scale:.3e}"
