"""Pins oracle/binning.py against brute force over every tile."""

import numpy as np
import pytest

from oracle import binning


def _brute_force(xy, radii, depth, image_ids, images, width, height):
    """Per tile, every pair whose float32 rectangle covers it, ordered by
    (depth bits, pair index): the stable-sort contract."""
    tw, th = binning.tile_grid(width, height)
    f16, one = np.float32(16), np.float32(1)

    def to_int(v):
        v = float(v)
        if v != v:
            return 0
        return int(max(min(np.trunc(v), 2**31 - 1), -(2**31)))

    lists = {}
    for i in range(len(radii)):
        if radii[i] <= 0:
            continue
        r = np.float32(radii[i])
        x, y = np.float32(xy[i, 0]), np.float32(xy[i, 1])
        x0 = min(max(to_int((x - r) / f16), 0), tw)
        y0 = min(max(to_int((y - r) / f16), 0), th)
        x1 = min(max(to_int((((x + r) + f16) - one) / f16), 0), tw)
        y1 = min(max(to_int((((y + r) + f16) - one) / f16), 0), th)
        for ty in range(y0, y1):
            for tx in range(x0, x1):
                tile = int(image_ids[i]) * tw * th + ty * tw + tx
                lists.setdefault(tile, []).append((int(np.float32(depth[i]).view(np.uint32)), i))
    point_list, ranges = [], np.zeros((images * tw * th, 2), np.int32)
    for tile in sorted(lists):
        entries = sorted(lists[tile])
        ranges[tile] = (len(point_list), len(point_list) + len(entries))
        point_list += [i for _, i in entries]
    return np.array(point_list, np.int32), ranges


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_binning_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    images, width, height, q = 3, 70, 45, 300
    geometry = np.zeros((q, 17), np.float32)
    geometry[:, 9] = rng.uniform(-40, width + 40, q)
    geometry[:, 10] = rng.uniform(-40, height + 40, q)
    # Depths with deliberate ties to exercise the stable order.
    geometry[:, 8] = rng.choice(rng.uniform(0.3, 20, 40).astype(np.float32), q)
    radii = rng.integers(-2, 40, q).astype(np.int32)
    image_ids = rng.integers(0, images, q).astype(np.int64)
    keys, point_list, ranges = binning.bin_pairs(geometry, radii, image_ids, images, width, height)
    expected_list, expected_ranges = _brute_force(
        geometry[:, 9:11], radii, geometry[:, 8], image_ids, images, width, height
    )
    np.testing.assert_array_equal(point_list, expected_list)
    np.testing.assert_array_equal(ranges, expected_ranges)
    assert np.all(np.diff(keys.astype(np.float64)) >= 0) or np.all(keys[:-1] <= keys[1:])
    counts = binning.tile_counts(geometry, radii, width, height)
    assert counts.sum() == len(point_list)


def test_rectangles_saturate_and_truncate():
    xy = np.array([[np.nan, 5.0], [3e9, -3e9], [-7.5, 7.5]], np.float32)
    radii = np.array([1, 1, 2], np.int32)
    x0, y0, x1, y1 = binning.tile_rects(xy, radii, 10, 10)
    # NaN -> 0, huge values clamp to the grid, truncation is toward zero:
    # (-7.5 - 2) / 16 = -0.59 -> 0 and (-7.5 + 2 + 15) / 16 = 0.59 -> 0.
    assert (x0[0], x1[0]) == (0, 0)
    assert (x0[1], y1[1]) == (10, 0)
    assert (x0[2], x1[2]) == (0, 0)


def test_pack_visible_and_sort_bits():
    radii = np.array([0, 3, -1, 5, 0, 1], np.int32)
    np.testing.assert_array_equal(binning.pack_visible(radii), [1, 3, 5])
    assert binning.sort_end_bit(1) == 32
    assert binning.sort_end_bit(2) == 33
    assert binning.sort_end_bit(8160) == 45
