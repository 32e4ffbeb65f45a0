"""Tile binning in numpy (reference: rasterize.cu:24-69, rendering.py:362-364).

All rectangle arithmetic is float32, evaluated in the reference's order, so
counts, keys, the stable sort and the tile ranges are bit-exact. int(float)
truncates toward zero and saturates (NaN -> 0), the conversion the
reference's hardware performs.
"""

from __future__ import annotations

import numpy as np

TILE = 16
INT_MIN, INT_MAX = -(2**31), 2**31 - 1


def tile_grid(width: int, height: int) -> tuple[int, int]:
    return (width + TILE - 1) // TILE, (height + TILE - 1) // TILE


def _to_int(values: np.ndarray) -> np.ndarray:
    """C int(float) with truncation and saturation."""
    values = np.asarray(values, dtype=np.float32)
    out = np.zeros(values.shape, dtype=np.int64)
    finite = ~np.isnan(values)
    clipped = np.clip(np.trunc(values[finite]).astype(np.float64), INT_MIN, INT_MAX)
    out[finite] = clipped.astype(np.int64)
    return out


def tile_rects(xy: np.ndarray, radii: np.ndarray, tw: int, th: int):
    """Rectangles [x0, x1) x [y0, y1) of tiles a pair may touch (rasterize.cu:24-30)."""
    xy = np.asarray(xy, dtype=np.float32)
    r = np.asarray(radii).astype(np.float32)
    sixteen, one = np.float32(16), np.float32(1)
    with np.errstate(invalid="ignore", over="ignore"):
        x0 = _to_int((xy[:, 0] - r) / sixteen)
        y0 = _to_int((xy[:, 1] - r) / sixteen)
        x1 = _to_int((((xy[:, 0] + r) + sixteen) - one) / sixteen)
        y1 = _to_int((((xy[:, 1] + r) + sixteen) - one) / sixteen)
    clamp_x = lambda v: np.clip(v, 0, tw)  # noqa: E731
    clamp_y = lambda v: np.clip(v, 0, th)  # noqa: E731
    return clamp_x(x0), clamp_y(y0), clamp_x(x1), clamp_y(y1)


def tile_counts(geometry: np.ndarray, radii: np.ndarray, width: int, height: int) -> np.ndarray:
    """Per-pair tile counts (countTiles, rasterize.cu:33-40), int64."""
    tw, th = tile_grid(width, height)
    radii = np.asarray(radii, dtype=np.int64)
    x0, y0, x1, y1 = tile_rects(geometry[:, 9:11], radii, tw, th)
    counts = (x1 - x0) * (y1 - y0)
    return np.where(radii > 0, counts, 0).astype(np.int64)


def emit(geometry: np.ndarray, radii: np.ndarray, image_ids: np.ndarray, width: int,
         height: int):
    """Unsorted keys (uint64) and values (int32) in pair order, tiles row-major
    within each pair (emitTiles, rasterize.cu:43-56)."""
    geometry = np.asarray(geometry, dtype=np.float32)
    tw, th = tile_grid(width, height)
    radii = np.asarray(radii, dtype=np.int64)
    x0, y0, x1, y1 = tile_rects(geometry[:, 9:11], radii, tw, th)
    counts = np.where(radii > 0, (x1 - x0) * (y1 - y0), 0)
    total = int(counts.sum())
    pair = np.repeat(np.arange(len(radii), dtype=np.int64), counts)
    first = np.concatenate([[0], np.cumsum(counts)[:-1]]) if len(counts) else np.zeros(0, np.int64)
    local = np.arange(total, dtype=np.int64) - np.repeat(first, counts)
    row_width = (x1 - x0)[pair]
    ty = y0[pair] + local // np.maximum(row_width, 1)
    tx = x0[pair] + local % np.maximum(row_width, 1)
    tile = np.asarray(image_ids, dtype=np.uint64)[pair] * np.uint64(tw * th) + (
        ty * tw + tx
    ).astype(np.uint64)
    depth_bits = geometry[:, 8].view(np.uint32).astype(np.uint64)[pair]
    keys = (tile << np.uint64(32)) | depth_bits
    return keys.astype(np.uint64), pair.astype(np.int32)


def sort_pairs(keys: np.ndarray, values: np.ndarray):
    """Stable ascending sort by the full 64-bit key."""
    order = np.argsort(keys, kind="stable")
    return keys[order], values[order]


def find_ranges(sorted_keys: np.ndarray, tiles: int) -> np.ndarray:
    """[tiles, 2] int32 [first, last) runs; empty tiles stay (0, 0)."""
    ranges = np.zeros((tiles, 2), dtype=np.int32)
    if len(sorted_keys) == 0:
        return ranges
    tile_of = (sorted_keys >> np.uint64(32)).astype(np.int64)
    boundaries = np.flatnonzero(np.diff(tile_of)) + 1
    starts = np.concatenate([[0], boundaries])
    ends = np.concatenate([boundaries, [len(sorted_keys)]])
    ranges[tile_of[starts], 0] = starts
    ranges[tile_of[starts], 1] = ends
    return ranges


def bin_pairs(geometry: np.ndarray, radii: np.ndarray, image_ids: np.ndarray, images: int,
              width: int, height: int):
    """Full binning: (sorted keys, point_list, ranges)."""
    tw, th = tile_grid(width, height)
    keys, values = emit(geometry, radii, image_ids, width, height)
    sorted_keys, point_list = sort_pairs(keys, values)
    return sorted_keys, point_list, find_ranges(sorted_keys, images * tw * th)


def pack_visible(radii: np.ndarray) -> np.ndarray:
    """Ascending indices of visible pairs (rendering.py:362-364)."""
    return np.flatnonzero(np.asarray(radii).reshape(-1) > 0).astype(np.int64)


def sort_end_bit(tiles: int) -> int:
    return 32 + max(int(tiles) - 1, 0).bit_length()
