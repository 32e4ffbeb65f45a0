"""Kernel-level parity: binning, sort and ranges bit-exact; projection and SH
within float tolerance of the float64 oracle."""

import math

import numpy as np
import pytest
import torch

from oracle import binning as oracle_binning
from oracle.projection import project, radius_before_ceil
from oracle.sh import sh_colors
from scenes import assert_gradients_close, describe_mismatch, perturbation_sensitivity

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEVICE = torch.device("cuda:0")


@pytest.fixture(scope="module")
def native():
    from diff_gabor_splatting_amd import _native

    return _native


def to_u64(t):
    return t.cpu().numpy().view(np.uint64)


@pytest.mark.parametrize("m", [1, 255, 1000, 2048, 2049, 8192, 8193, 100_003, 1_000_003,
                               4_194_305])
@pytest.mark.parametrize("bits, with_values", [
    ((0, 32), True), ((19, 32), False), ((0, 13), True), ((5, 12), False),
    ((16, 25), True), ((3, 14), False), ((0, 22), True),
])
def test_sort32_is_stable_radix_order(native, m, bits, with_values):
    """The 32-bit sort of the binning stages against numpy's stable argsort:
    the one-workgroup sort (up to 8192 keys) and the reduce-then-scan digit
    passes (from 8193), partial last spans, both span sizes (4,194,305 keys
    take 4096-key spans), keys alone and with values, partial bit ranges,
    many ties and skewed digits. Digit widths: 8 bits or fewer (256 bins),
    and 9 bits in one 512-bin pass (16, 25), which saves a pass; 11 and 22
    bits take two and three passes of at most 8 bits."""
    rng = np.random.default_rng(m + 7 * bits[0])
    keys = rng.integers(0, 2**32, m, dtype=np.uint64).astype(np.uint32)
    keys[rng.integers(0, m, m // 3)] = keys[0]  # many exact ties
    keys[: m // 5] = rng.integers(0, 5, m // 5).astype(np.uint32)  # skewed low digits
    values = np.arange(m, dtype=np.int32)[::-1].copy()
    print(f"sort32 m={m} bits={bits} values={with_values}", flush=True)
    sk, sv = native.sort_pairs32(torch.from_numpy(keys.view(np.int32)).to(DEVICE),
                                 torch.from_numpy(values).to(DEVICE) if with_values else None,
                                 *bits)
    begin, end = bits
    digit = (keys.astype(np.uint64) >> np.uint64(begin)) & np.uint64((1 << (end - begin)) - 1)
    order = np.argsort(digit, kind="stable")
    np.testing.assert_array_equal(sk.cpu().numpy().view(np.uint32), keys[order])
    if with_values:
        np.testing.assert_array_equal(sv.cpu().numpy(), values[order])
    else:
        assert sv is None


@pytest.mark.parametrize("m", [1, 5, 4095, 4096, 4097, 8192, 8193, 100_003, 2_000_000])
@pytest.mark.parametrize("bits", [(0, 64), (0, 45), (32, 45), (3, 17)])
def test_sort_is_stable_radix_order(native, m, bits):
    rng = np.random.default_rng(m + bits[0])
    keys = rng.integers(0, 2**63, m, dtype=np.uint64) | (rng.integers(0, 2, m, dtype=np.uint64) << np.uint64(63))
    keys[rng.integers(0, m, m // 3)] = keys[0]  # many exact ties
    values = np.arange(m, dtype=np.int32)[::-1].copy()
    sk, sv = native.sort_pairs(torch.from_numpy(keys.view(np.int64)).to(DEVICE),
                               torch.from_numpy(values).to(DEVICE), *bits)
    begin, end = bits
    digit = (keys >> np.uint64(begin)) & np.uint64((1 << (end - begin)) - 1 if end - begin < 64 else 2**64 - 1)
    order = np.argsort(digit, kind="stable")
    np.testing.assert_array_equal(to_u64(sk), keys[order])
    np.testing.assert_array_equal(sv.cpu().numpy(), values[order])


def random_geometry(seed, q, width, height, images):
    rng = np.random.default_rng(seed)
    geometry = rng.normal(size=(q, 17)).astype(np.float32)
    geometry[:, 9] = rng.uniform(-60, width + 60, q)
    geometry[:, 10] = rng.uniform(-60, height + 60, q)
    geometry[:, 8] = rng.choice(rng.uniform(0.3, 50, max(q // 3, 1)).astype(np.float32), q)
    radii = rng.integers(-3, 70, q).astype(np.int32)
    image_ids = np.sort(rng.integers(0, images, q)).astype(np.int64)
    return geometry, radii, image_ids


@pytest.mark.parametrize("seed, q, width, height, images", [
    (0, 1, 16, 16, 1), (1, 700, 100, 61, 3), (2, 20_000, 640, 480, 2), (3, 5000, 1920, 1080, 1),
])
def test_binning_pipeline_is_bit_exact(native, seed, q, width, height, images):
    geometry, radii, image_ids = random_geometry(seed, q, width, height, images)
    g, r, ids = (torch.from_numpy(a).to(DEVICE) for a in (geometry, radii, image_ids))
    offsets = native.count_tiles(g, r, width, height)
    expected_counts = oracle_binning.tile_counts(geometry, radii, width, height)
    np.testing.assert_array_equal(offsets.cpu().numpy(), np.cumsum(expected_counts))
    m = int(offsets[-1])
    keys, values = native.emit_tiles(g, r, ids, offsets, width, height, m)
    expected_keys, expected_values = oracle_binning.emit(geometry, radii, image_ids, width, height)
    np.testing.assert_array_equal(to_u64(keys), expected_keys)
    np.testing.assert_array_equal(values.cpu().numpy(), expected_values)
    tw, th = native.tile_grid(width, height)
    tiles = images * tw * th
    sorted_keys, point_list = native.sort_pairs(keys, values, 0, native.sort_end_bit(tiles))
    ok_keys, ok_list, ok_ranges = oracle_binning.bin_pairs(geometry, radii, image_ids, images, width, height)
    np.testing.assert_array_equal(to_u64(sorted_keys), ok_keys)
    np.testing.assert_array_equal(point_list.cpu().numpy(), ok_list)
    np.testing.assert_array_equal(native.find_ranges(sorted_keys, tiles).cpu().numpy(), ok_ranges)
    # The renderer's depth-first pipeline gives the same list and ranges.
    bin_list, bin_ranges = native.bin_depth_first(g, r, ids, images, width, height)
    np.testing.assert_array_equal(bin_list.cpu().numpy(), ok_list)
    np.testing.assert_array_equal(bin_ranges.cpu().numpy(), ok_ranges)


def test_depth_first_binning_propagates_callback_errors(native):
    """An exception from the callback run while the host waits for the
    intersection count propagates as raised, and the next binning on the
    same thread (which reuses its pinned read-back buffer) is unaffected; a
    pending value-check word reaches its callback before the count is used."""
    geometry, radii, image_ids = random_geometry(11, 2000, 64, 64, 1)
    g, r, ids = (torch.from_numpy(a).to(DEVICE) for a in (geometry, radii, image_ids))

    def boom():
        raise KeyError("overlap failed")

    with pytest.raises(KeyError, match="overlap failed"):
        native.bin_depth_first(g, r, ids, 1, 64, 64, overlap=boom)
    _, ok_list, ok_ranges = oracle_binning.bin_pairs(geometry, radii, image_ids, 1, 64, 64)
    point_list, ranges = native.bin_depth_first(g, r, ids, 1, 64, 64)
    np.testing.assert_array_equal(point_list.cpu().numpy(), ok_list)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ok_ranges)
    word = torch.full((1,), 5, dtype=torch.int32, device=DEVICE)
    seen = []

    def report(value):
        seen.append(value)
        raise ValueError("values violated")

    with pytest.raises(ValueError, match="values violated"):
        native.bin_depth_first(g, r, ids, 1, 64, 64, violations=(word, report))
    assert seen == [5]


@pytest.mark.parametrize("seed, q, width, height, images, culled", [
    (5, 3000, 64, 64, 1, 1.0),          # every pair culled: m = 0
    (6, 40_000, 1920, 1080, 40, 0.0),   # 326,400 tiles: 19 id bits, three tile passes
    (7, 300_000, 512, 512, 32, 0.0),    # config-3-like: 32,768 tiles, 1e5+ equal depths
    # 8,160 tiles (13 bits) and V < 2^19 visible pairs: packed 32-bit keys
    # with the true V, (tile id, pair) pairs when V is unknown (2^21 pairs).
    (8, 1_100_000, 1920, 1080, 1, 0.6),
])
def test_depth_first_binning_is_bit_exact(native, seed, q, width, height, images, culled):
    geometry, radii, image_ids = random_geometry(seed, q, width, height, images)
    radii[: int(culled * q)] = np.minimum(radii[: int(culled * q)], 0)
    if seed == 7:
        geometry[:, 8] = np.float32(3.5)  # all depths tie: order is by pair index
        geometry[::5, 8] = np.float32(2.0)
    g, r, ids = (torch.from_numpy(a).to(DEVICE) for a in (geometry, radii, image_ids))
    offsets = native.count_tiles(g, r, width, height)
    m = int(offsets[-1])
    assert (m == 0) == (culled == 1.0)
    counts = np.diff(np.concatenate([[0], offsets.cpu().numpy()]))
    visible = int(np.count_nonzero(counts))
    _, ok_list, ok_ranges = oracle_binning.bin_pairs(geometry, radii, image_ids, images, width,
                                                     height)
    order, starts, rects, totals = native.bin_order(g, r, ids, width, height)
    assert totals.tolist() == [m, visible]
    # The one-call entry point (gs_bin_order) gives the same stage-1 outputs
    # as the renderer's two calls (gs_bin_order_count, gs_bin_order_sort).
    lib = native.lib
    single = [torch.full_like(t, -9) for t in (order, starts, rects, totals)]
    space = torch.empty(lib.gs_bin_order_workspace_size(q), dtype=torch.uint8, device=DEVICE)
    status = lib.gs_bin_order(g.data_ptr(), r.data_ptr(), ids.data_ptr(), q, width, height,
                              single[0].data_ptr(), single[1].data_ptr(), single[2].data_ptr(),
                              single[3].data_ptr(), single[3].data_ptr() + 8, space.data_ptr(),
                              space.numel(), torch.cuda.current_stream(DEVICE).cuda_stream)
    assert status == 0, lib.gs_last_error()
    torch.cuda.synchronize()
    for name, a, b in zip(("order", "starts", "rects", "totals"), single,
                          (order, starts, rects, totals)):
        assert torch.equal(a, b), name
    for known in (visible, -1):
        point_list, ranges = native.bin_tiles(order, starts, rects, images, width, height, m,
                                              known)
        np.testing.assert_array_equal(point_list.cpu().numpy(), ok_list)
        np.testing.assert_array_equal(ranges.cpu().numpy(), ok_ranges)
    if seed == 8:
        tile_bits = (images * 120 * 68 - 1).bit_length()
        assert tile_bits + visible.bit_length() <= 32 < tile_bits + q.bit_length()


def test_bin_tiles_flags_sort_outputs_out_of_range(native):
    """The binning consumers range-check what the depth sort produced: an
    `order` entry outside [0, count) - planted on the host here - is
    replaced by pair 0 and reported as GS_BIN_BAD_INDEX instead of being
    dereferenced, with packed (tile, rank) keys (V known) and with (tile,
    pair) pairs (V unknown, bits(tiles) + bits(count) > 32)."""
    width, height, images, q = 1920, 1080, 1, 600_000
    geometry, radii, image_ids = random_geometry(9, q, width, height, images)
    radii[: int(0.6 * q)] = np.minimum(radii[: int(0.6 * q)], 0)
    g, r, ids = (torch.from_numpy(a).to(DEVICE) for a in (geometry, radii, image_ids))
    order, starts, rects, totals = native.bin_order(g, r, ids, width, height)
    m, visible = totals.tolist()
    tile_bits = (120 * 68 - 1).bit_length()
    assert tile_bits + visible.bit_length() <= 32 < tile_bits + q.bit_length()
    _, ok_list, ok_ranges = oracle_binning.bin_pairs(geometry, radii, image_ids, images, width,
                                                     height)
    status = torch.full((1,), -1, dtype=torch.int32, device=DEVICE)
    corrupt = order.clone()
    corrupt[5], corrupt[visible // 2] = q + 7, -3
    for known in (visible, -1):
        print(f"bin_tiles guard visible={known}", flush=True)
        point_list, ranges = native.bin_tiles(order, starts, rects, images, width, height, m,
                                              known, status=status)
        assert int(status) == 0
        np.testing.assert_array_equal(point_list.cpu().numpy(), ok_list)
        np.testing.assert_array_equal(ranges.cpu().numpy(), ok_ranges)
        point_list, ranges = native.bin_tiles(corrupt, starts, rects, images, width, height, m,
                                              known, status=status)
        assert int(status) == native.BINNING_BAD_INDEX
        listed = point_list.cpu().numpy()
        assert listed.min() >= 0 and listed.max() < q
        bounds = ranges.cpu().numpy()
        assert bounds.min() >= 0 and bounds.max() <= m


def block_entries(geometry, radii, width, height):
    """(pair, tile block) entries of the block path: the 4 x 4-tile blocks
    each pair's tile rectangle meets."""
    tw, th = native_tile_grid(width, height)
    x0, y0, x1, y1 = oracle_binning.tile_rects(geometry[:, 9:11], radii.astype(np.int64), tw, th)
    met = (radii > 0) & (x1 > x0) & (y1 > y0)
    blocks = ((((x1 - 1) >> 2) - (x0 >> 2) + 1) * (((y1 - 1) >> 2) - (y0 >> 2) + 1))
    return int(np.where(met, blocks, 0).sum())


def native_tile_grid(width, height):
    return (width + 15) // 16, (height + 15) // 16


@pytest.mark.parametrize("seed, q, width, height, images, culled, radius", [
    (20, 1, 16, 16, 1, 0.0, None),            # one tile, one block
    (21, 3000, 64, 64, 1, 1.0, None),         # every pair culled: M = E = 0
    (22, 700, 100, 61, 3, 0.0, None),         # 7 x 4 tiles: partial blocks at both edges
    (23, 20_000, 515, 333, 5, 0.3, None),     # 33 x 21 tiles per image, five images
    (24, 2000, 1920, 1080, 2, 0.0, 2000),     # every pair covers its whole image
    (25, 300_000, 512, 512, 32, 0.0, None),   # config-3-like: 2,048 blocks, equal depths
    (26, 1_100_000, 1920, 1080, 1, 0.6, None),  # config-4-like: 510 blocks
])
def test_block_binning_is_bit_exact(native, seed, q, width, height, images, culled, radius):
    """The block path (gs_bin_blocks_count, gs_bin_order_sort,
    gs_bin_blocks_tiles) gives the oracle's point list and ranges bit for
    bit, the totals (M, V, E), and the same lists as the tile sort through
    bin_depth_first."""
    geometry, radii, image_ids = random_geometry(seed, q, width, height, images)
    radii[: int(culled * q)] = np.minimum(radii[: int(culled * q)], 0)
    if radius is not None:
        radii[:] = radius
    if seed == 25:
        geometry[:, 8] = np.float32(3.5)  # all depths tie: order is by pair index
        geometry[::5, 8] = np.float32(2.0)
    print(f"block binning seed={seed} q={q} {images}x{width}x{height}", flush=True)
    g, r, ids = (torch.from_numpy(a).to(DEVICE) for a in (geometry, radii, image_ids))
    _, ok_list, ok_ranges = oracle_binning.bin_pairs(geometry, radii, image_ids, images, width,
                                                     height)
    counts = oracle_binning.tile_counts(geometry, radii, width, height)
    m, visible = int(counts.sum()), int(np.count_nonzero(counts))
    entries = block_entries(geometry, radii, width, height)
    assert native.lib.gs_bin_blocks_fit(images, width, height) == 1
    status = torch.full((1,), -1, dtype=torch.int32, device=DEVICE)
    # Raw depth keys, and keys relative to the near plane (all depths of
    # random_geometry lie in (0.2, 100): 27-bit keys, three 9-bit passes).
    for planes in ((0.0, 0.0), (0.2, 100.0)):
        order, starts, rects, totals = native.bin_blocks_order(g, r, ids, width, height, *planes)
        assert totals.tolist() == [m, visible, entries]
        for known in (visible, -1):
            point_list, ranges = native.bin_blocks_tiles(order, starts, rects, images, width,
                                                         height, m, entries, known, status=status)
            assert int(status) == 0
            np.testing.assert_array_equal(point_list.cpu().numpy(), ok_list)
            np.testing.assert_array_equal(ranges.cpu().numpy(), ok_ranges)
    assert native.binning_path() == "blocks"
    try:
        for path, planes in (("tiles", (0.0, 0.0)), ("blocks", (0.0, 0.0)),
                             ("blocks", (0.2, 100.0))):
            native.set_binning_path(path)
            point_list, ranges = native.bin_depth_first(g, r, ids, images, width, height,
                                                        near_plane=planes[0],
                                                        far_plane=planes[1])
            np.testing.assert_array_equal(point_list.cpu().numpy(), ok_list)
            np.testing.assert_array_equal(ranges.cpu().numpy(), ok_ranges)
    finally:
        native.set_binning_path("blocks")


@pytest.mark.parametrize("near, far", [(0.25, 0.5), (1e-3, 1e6), (-1.0, 10.0)])
def test_block_binning_depth_keys(native, near, far):
    """Depth keys relative to the near plane keep the raw bits' order: depths
    packed into a narrow range (24-bit keys, many ties), a wide one (28-bit
    keys), and a non-positive near plane (raw keys); pairs without tiles
    still sort after every pair with tiles."""
    width, height, images, q = 640, 480, 2, 60_000
    geometry, radii, image_ids = random_geometry(28, q, width, height, images)
    rng = np.random.default_rng(29)
    low, high = max(near, 0.0), far
    depths = rng.uniform(low, high, q // 7).astype(np.float32)
    depths = np.clip(depths, np.nextafter(np.float32(low), np.float32(high)),
                     np.nextafter(np.float32(high), np.float32(low)))
    geometry[:, 8] = rng.choice(depths, q)
    print(f"block depth keys near={near} far={far}", flush=True)
    g, r, ids = (torch.from_numpy(a).to(DEVICE) for a in (geometry, radii, image_ids))
    _, ok_list, ok_ranges = oracle_binning.bin_pairs(geometry, radii, image_ids, images, width,
                                                     height)
    point_list, ranges = native.bin_depth_first(g, r, ids, images, width, height,
                                                near_plane=near, far_plane=far)
    np.testing.assert_array_equal(point_list.cpu().numpy(), ok_list)
    np.testing.assert_array_equal(ranges.cpu().numpy(), ok_ranges)


def test_block_binning_flags_sort_outputs_out_of_range(native):
    """An `order` entry outside [0, count), planted on the host, is replaced
    by pair 0 and reported as GS_BIN_BAD_INDEX by the block path's emission;
    no point-list entry or range leaves its bounds."""
    width, height, images, q = 1920, 1080, 1, 200_000
    geometry, radii, image_ids = random_geometry(27, q, width, height, images)
    g, r, ids = (torch.from_numpy(a).to(DEVICE) for a in (geometry, radii, image_ids))
    order, starts, rects, totals = native.bin_blocks_order(g, r, ids, width, height)
    m, visible, entries = totals.tolist()
    status = torch.full((1,), -1, dtype=torch.int32, device=DEVICE)
    corrupt = order.clone()
    corrupt[5], corrupt[visible // 2] = q + 7, -3
    point_list, ranges = native.bin_blocks_tiles(corrupt, starts, rects, images, width, height, m,
                                                 entries, visible, status=status)
    assert int(status) & native.BINNING_BAD_INDEX
    listed = point_list.cpu().numpy()
    written = listed[: int(ranges[:, 1].max())]
    assert written.min() >= 0 and written.max() < q
    bounds = ranges.cpu().numpy()
    assert bounds.min() >= 0 and bounds.max() <= m


def _is_subsequence(part, whole):
    it = iter(whole.tolist())
    return all(any(v == w for w in it) for v in part.tolist())


@pytest.mark.parametrize("seed, q, width, height, images, culled", [
    (40, 0, 64, 48, 1, 0.0),                # no pairs
    (41, 3000, 64, 64, 1, 1.0),             # every pair culled: M = E = 0
    (42, 700, 100, 61, 3, 0.0),             # partial blocks at both edges
    (43, 20_000, 515, 333, 5, 0.3),         # five images
    (44, 1_100_000, 1920, 1080, 1, 0.6),    # config-4-like
])
def test_bounded_block_binning(native, seed, q, width, height, images, culled):
    """gs_bin_blocks_tiles_bounded reads M and E on the device. Within the
    capacity it gives gs_bin_blocks_tiles' point list and ranges bit for bit
    and -1 past M. Past it (GS_BIN_OVERFLOW): with all block entries kept,
    the list is the synchronised list cut at the capacity and the ranges
    are clamped to it (a tile wholly past it keeps (C, C)); with block
    entries dropped too, every tile's list is a subsequence of its
    synchronised list, inside the capacity, made of valid pairs."""
    geometry, radii, image_ids = random_geometry(seed, max(q, 1), width, height, images)
    geometry, radii, image_ids = geometry[:q], radii[:q], image_ids[:q]
    radii[: int(culled * q)] = np.minimum(radii[: int(culled * q)], 0)
    print(f"bounded block binning seed={seed} q={q} {images}x{width}x{height}", flush=True)
    g, r, ids = (torch.from_numpy(np.ascontiguousarray(a)).to(DEVICE)
                 for a in (geometry, radii, image_ids))
    order, starts, rects, totals = native.bin_blocks_order(g, r, ids, width, height, 0.2, 100.0)
    m, visible, entries = totals.tolist()
    status = torch.full((1,), -1, dtype=torch.int32, device=DEVICE)
    full_list, full_ranges = native.bin_blocks_tiles(order, starts, rects, images, width, height,
                                                     m, entries, visible, status=status)
    assert int(status) == 0
    full_list, full_ranges = full_list.cpu().numpy(), full_ranges.cpu().numpy()
    capacities = sorted({m, m + 1000, m // 2, entries // 2, 0})
    for capacity in capacities:
        print(f"  capacity {capacity} (M {m}, E {entries})", flush=True)
        point_list, ranges, overflow = native.bin_blocks_tiles_bounded(
            order, starts, rects, images, width, height, capacity, totals)
        point_list, ranges = point_list.cpu().numpy(), ranges.cpu().numpy()
        assert point_list.shape == (capacity,) and ranges.shape == full_ranges.shape
        if capacity >= m:
            assert int(overflow) == 0
            np.testing.assert_array_equal(point_list[:m], full_list)
            assert (point_list[m:] == -1).all()
            np.testing.assert_array_equal(ranges, full_ranges)
            continue
        assert int(overflow) == native.BINNING_OVERFLOW
        assert ranges.min() >= 0 and ranges.max() <= capacity
        assert (ranges[:, 1] >= ranges[:, 0]).all()
        covered = np.concatenate([point_list[a:b] for a, b in ranges] + [np.zeros(0, np.int32)])
        assert covered.size == 0 or (covered.min() >= 0 and covered.max() < q)
        if capacity >= entries:
            expected = np.where(
                (full_ranges[:, 1:] > full_ranges[:, :1]),
                np.minimum(full_ranges, capacity), 0)
            np.testing.assert_array_equal(ranges, expected)
            np.testing.assert_array_equal(point_list, full_list[:capacity])
        else:
            for t in np.flatnonzero(ranges[:, 1] > ranges[:, 0])[::97]:
                a, b = ranges[t]
                fa, fb = full_ranges[t]
                assert b - a <= fb - fa
                assert _is_subsequence(point_list[a:b], full_list[fa:fb])
    # bin_depth_first with a capacity takes the same path, and the tile
    # path gives the same lists within the capacity.
    try:
        for path in ("blocks", "tiles"):
            native.set_binning_path(path)
            seen = []
            point_list, ranges = native.bin_depth_first(
                g, r, ids, images, width, height, capacity=m + 64,
                flags=lambda word, total: seen.append((int(word), int(total))),
                near_plane=0.2, far_plane=100.0)
            assert seen == [(0, m)]
            np.testing.assert_array_equal(point_list[:m].cpu().numpy(), full_list)
            assert bool((point_list[m:] == -1).all())
            np.testing.assert_array_equal(ranges.cpu().numpy(), full_ranges)
    finally:
        native.set_binning_path("blocks")


def test_ranges_of_empty_list_are_zero(native):
    ranges = native.find_ranges(torch.empty(0, dtype=torch.int64, device=DEVICE), 37)
    assert ranges.shape == (37, 2) and int(ranges.abs().sum()) == 0


@pytest.mark.parametrize("count", [0, 1, 4096, 4097, 8192, 8193, 1_000_000])
def test_pack_visible(native, count):
    rng = np.random.default_rng(count)
    radii = rng.integers(-1, 3, count).astype(np.int32)
    selected = native.pack_visible(torch.from_numpy(radii).to(DEVICE))
    np.testing.assert_array_equal(selected.cpu().numpy(), oracle_binning.pack_visible(radii))


def projection_inputs(seed, S=2, C=3, N=777, width=64, height=48, z_low=-0.5):
    g = torch.Generator().manual_seed(seed)
    means = torch.cat([torch.rand(S, N, 2, generator=g) * 3 - 1.5,
                       torch.rand(S, N, 1, generator=g) * (5.5 - z_low) + z_low], -1)
    quats = torch.randn(S, N, 4, generator=g)
    quats = quats / quats.norm(dim=-1, keepdim=True)
    scales = torch.exp(torch.rand(S, N, 2, generator=g) * math.log(10) + math.log(0.02))
    views = torch.eye(4).expand(S, C, 4, 4).clone()
    angle = torch.rand(S, C, generator=g) * 0.4 - 0.2
    views[..., 0, 0], views[..., 0, 2] = angle.cos(), angle.sin()
    views[..., 2, 0], views[..., 2, 2] = -angle.sin(), angle.cos()
    views[..., :3, 3] = torch.randn(S, C, 3, generator=g) * 0.2
    K = torch.tensor([[50.0, 0.5, (width - 1) / 2], [0, 52.0, (height - 1) / 2], [0, 0, 1]])
    return [means, quats, scales, views, K.expand(S, C, 3, 3).clone()], width, height


def test_projection_forward_matches_oracle(native):
    inputs, width, height = projection_inputs(0)
    gpu = native.project_forward(*(t.to(DEVICE) for t in inputs), width, height, 0.2, 100.0)
    ref = project(*(t.double() for t in inputs), width, height, 0.2, 100.0)
    # Per-element bound: 1e-6 relative plus four times the float64 output's
    # sensitivity to float32-sized input perturbations (the conic centre of a
    # nearly edge-on surfel is ill-conditioned).
    sens = perturbation_sensitivity(lambda *x: project(*x, width, height, 0.2, 100.0)[:4], inputs)
    for name, a, b, d in zip(("transform", "xy", "normals", "directions"), gpu[:4], ref[:4], sens):
        a = a.cpu().double()
        ok = (a - b).abs() <= 1e-6 * (1 + b.abs()) + 4 * d
        assert bool(ok.all()), f"{name}: {describe_mismatch(a, b)}"
    # Radii are integers from a ceiling: they must agree except where the
    # float64 pre-ceiling radius lies within 1e-4 of an integer (margin rule),
    # and the float32 oracle must agree exactly off those margins too.
    radii32 = project(*inputs, width, height, 0.2, 100.0)[4]
    before = radius_before_ceil(*(t.double() for t in inputs))
    wobble = perturbation_sensitivity(radius_before_ceil, inputs)[0]
    margin = (before - before.round()).abs() <= 4 * wobble + 1e-4
    differ = gpu[4].cpu() != radii32
    assert not bool((differ & ~margin).any()), int(differ.sum())
    assert int((gpu[4].cpu() > 0).sum()) > 100


def test_projection_backward_matches_autograd(native):
    # Depths in [1, 5.5]: away from the camera plane, where the conic centre
    # and its derivatives blow up.
    inputs, width, height = projection_inputs(1, S=2, C=2, N=300, z_low=1.0)
    leaves = [t.double().requires_grad_() for t in inputs]
    outs = project(*leaves, width, height, 0.2, 100.0)[:4]
    g = torch.Generator().manual_seed(5)
    grads = [torch.randn(o.shape, generator=g, dtype=torch.float64) for o in outs]
    expected = torch.autograd.grad(sum((o * w).sum() for o, w in zip(outs, grads)), leaves,
                                   retain_graph=True)
    actual = native.project_backward(*(t.to(DEVICE) for t in inputs),
                                     *(w.float().to(DEVICE) for w in grads))
    for name, a, e in zip(("means", "quaternions", "scales", "views", "intrinsics"), actual, expected):
        assert_gradients_close(a, e, name, rel_norm=1e-5, elem=1e-5, rtol=1e-5)
    # Missing output gradients are treated as zero.
    partial = native.project_backward(*(t.to(DEVICE) for t in inputs), None, grads[1].float().to(DEVICE), None, None)
    expected_partial = torch.autograd.grad((outs[1] * grads[1]).sum(), leaves)
    torch.testing.assert_close(partial[0].cpu().double(), expected_partial[0], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
@pytest.mark.parametrize("cameras", [1, 3])
def test_sh_values_and_derivatives(native, degree, cameras):
    g = torch.Generator().manual_seed(31)
    k = (degree + 1) ** 2
    first = torch.randn(2, 7, k, 3, generator=g)
    second = torch.randn(2, 7, k, 3, generator=g)
    d = torch.randn(2, cameras, 7, 3, generator=g)
    d = d / d.norm(dim=-1, keepdim=True)
    colors = native.evaluate_sh_forward(first.to(DEVICE), second.to(DEVICE), d.to(DEVICE), degree)
    leaves = [t.double().requires_grad_() for t in (first, second, d)]
    expected = sh_colors(*leaves, degree)
    torch.testing.assert_close(colors.cpu().double(), expected, atol=3e-6, rtol=3e-5)
    weights = torch.randn(expected.shape, generator=g, dtype=torch.float64)
    eg = torch.autograd.grad((expected * weights).sum(), leaves, allow_unused=True)
    ag = native.evaluate_sh_backward(first.to(DEVICE), second.to(DEVICE), d.to(DEVICE),
                                     weights.float().to(DEVICE), degree)
    for a, e, leaf in zip(ag, eg, leaves):
        e = torch.zeros_like(leaf) if e is None else e
        torch.testing.assert_close(a.cpu().double(), e, atol=3e-5, rtol=2e-4)


@pytest.mark.parametrize("n", [300, 301])  # 301: dense row runs start off 16-byte boundaries
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("sh", [None, 0, 3])
def test_records_match_oracle(native, packed, sh, n):
    from oracle import render as oracle_render
    from scenes import random_scene

    width, height = 48, 40
    v = random_scene("classic", scenes=2, cameras=3, n=n, width=width, height=height, seed=8,
                     sh=sh)
    v["view_matrices"][..., 2, 3] = torch.linspace(-1.0, 0.5, 3)  # some surfels behind near
    S, N = v["means"].shape[:2]
    C = v["view_matrices"].shape[1]
    gpu = {k: t.to(DEVICE) for k, t in v.items()}
    sh_args = None if sh is None else (gpu["colors"], gpu["secondary_colors"])
    shared = None if sh is None else (gpu["frequency_weights"], gpu["frequency_magnitudes"],
                                      gpu["phases"])
    out = native.records_forward(gpu["means"], gpu["quaternions"], gpu["scales"],
                                 gpu["opacities"], gpu["view_matrices"], gpu["intrinsics"],
                                 sh_args, shared, sh, width, height, 0.2, 100.0, packed)
    radii = out["dense_radii"].cpu()
    leaves = {k: t.double().requires_grad_() for k, t in v.items() if k != "backgrounds"}
    appearance = tuple(leaves[k] for k in ("colors", "secondary_colors", "frequency_weights",
                                          "frequency_magnitudes", "phases"))
    rec = oracle_render.records(leaves["means"], leaves["quaternions"], leaves["scales"],
                                leaves["opacities"], appearance, leaves["view_matrices"],
                                leaves["intrinsics"], width, height, packed=packed,
                                sh_degree=sh, radii=radii)
    oracle32 = oracle_render.records(*(v[k] for k in ("means", "quaternions", "scales", "opacities")),
                                     tuple(v[k] for k in ("colors", "secondary_colors",
                                                          "frequency_weights",
                                                          "frequency_magnitudes", "phases")),
                                     v["view_matrices"], v["intrinsics"], width, height,
                                     packed=packed, sh_degree=sh)
    before = radius_before_ceil(*(v[k].double() for k in ("means", "quaternions", "scales",
                                                         "view_matrices", "intrinsics")))
    wobble = perturbation_sensitivity(radius_before_ceil, [v[k] for k in (
        "means", "quaternions", "scales", "view_matrices", "intrinsics")])[0]
    margin = (before - before.round()).abs() <= 4 * wobble + 1e-4
    assert not bool(((radii != oracle32["dense_radii"]) & ~margin).any())
    selected = rec["selected"].numpy()
    if packed:
        np.testing.assert_array_equal(out["selected"].cpu().numpy(), selected)
        rows = out["row_of_pair"].cpu().numpy()
        expect_rows = np.full(S * C * N, -1)
        expect_rows[selected] = np.arange(len(selected))
        np.testing.assert_array_equal(rows, expect_rows)
    np.testing.assert_array_equal(out["image_ids"].cpu().numpy(), rec["image_ids"].numpy())
    np.testing.assert_array_equal(out["row_radii"].cpu().numpy(), rec["radii"].numpy())
    expect_prims = np.arange(len(selected)) if sh is not None else rec["primitive_ids"].numpy()
    np.testing.assert_array_equal(out["primitive_ids"].cpu().numpy(), expect_prims)
    # Rows of culled pairs (radius 0) are referenced by no tile list: their
    # radius, projected mean and ids are compared with the oracle, and in
    # dense mode their geometry and appearance rows are zero.
    if not packed:
        culled = out["row_radii"].cpu() == 0
        assert bool(culled.any())
        assert bool((out["geometry"].cpu()[culled] == 0).all())
        if sh is not None:
            assert bool((out["appearance"].cpu()[culled] == 0).all())
    visible = rec["radii"] > 0
    geometry = rec["geometry"].detach()
    sens = perturbation_sensitivity(
        lambda *x: oracle_render.records(*x[:4], tuple(x[4:9]), x[9], x[10], width, height,
                                         packed=packed, sh_degree=sh, radii=radii)["geometry"],
        [v[k] for k in ("means", "quaternions", "scales", "opacities", "colors",
                        "secondary_colors", "frequency_weights", "frequency_magnitudes",
                        "phases", "view_matrices", "intrinsics")])[0]
    a = out["geometry"].cpu().double()
    xy = out["projected_means"].cpu().double()
    xy_ok = (xy - geometry[:, 9:11]).abs() <= 1e-6 * (1 + geometry[:, 9:11].abs()) + 4 * sens[:, 9:11]
    assert bool((xy_ok | (xy == geometry[:, 9:11])).all()), describe_mismatch(xy, geometry[:, 9:11])
    a_vis, g_vis, s_vis = a[visible], geometry[visible], sens[visible]
    assert bool(((a_vis - g_vis).abs() <= 1e-6 * (1 + g_vis.abs()) + 4 * s_vis).all()), \
        describe_mismatch(a_vis, g_vis)
    if sh is not None:
        rows_ref = rec["appearance"].detach()[selected] if packed else rec["appearance"].detach()
        torch.testing.assert_close(out["appearance"].cpu().double()[visible], rows_ref[visible],
                                   atol=2e-6, rtol=1e-5)
        op_ref = rec["opacities"].detach()[selected] if packed else rec["opacities"].detach()
        torch.testing.assert_close(out["opacity_rows"].cpu().double()[visible], op_ref[visible])
    # Adjoint: random row gradients (geometry xy columns excluded: that
    # gradient enters through the projected means).
    g = torch.Generator().manual_seed(4)
    Q = a.shape[0]
    g_geometry = torch.randn(Q, 17, generator=g, dtype=torch.float64)
    g_geometry[:, 9:11] = 0
    g_geometry[~visible] = 0  # the compositor never writes culled rows
    g_projected = torch.randn(Q, 2, generator=g, dtype=torch.float64)
    loss = (rec["geometry"] * g_geometry).sum() + (rec["projected_means"] * g_projected).sum()
    g_app = g_op = None
    if sh is not None:
        g_app = torch.randn(Q, 18, generator=g, dtype=torch.float64) * visible[:, None]
        g_op = torch.randn(Q, generator=g, dtype=torch.float64) * visible
        app = rec["appearance"][selected] if packed else rec["appearance"]
        ops = rec["opacities"][selected] if packed else rec["opacities"]
        loss = loss + (app * g_app).sum() + (ops * g_op).sum()
    names = ["means", "quaternions", "scales", "view_matrices", "intrinsics"]
    if sh is not None:
        names += ["colors", "secondary_colors", "frequency_weights", "frequency_magnitudes",
                  "phases", "opacities"]
    expected = torch.autograd.grad(loss, [leaves[k] for k in names], allow_unused=True)
    to_gpu = lambda t: None if t is None else t.float().to(DEVICE)  # noqa: E731
    got = native.records_backward(
        gpu["means"], gpu["quaternions"], gpu["scales"], gpu["view_matrices"],
        gpu["intrinsics"], sh_args, sh, out["row_of_pair"], out["geometry"],
        to_gpu(g_geometry), to_gpu(g_projected), to_gpu(g_app), to_gpu(g_op))
    order = [0, 1, 2, 3, 4] + ([5, 6, 7, 8, 9, 10] if sh is not None else [])
    for name, index, e in zip(names, order, expected):
        e = torch.zeros_like(leaves[name]) if e is None else e
        assert_gradients_close(got[index], e.reshape(got[index].shape), name, rel_norm=1e-4,
                               elem=1e-4, rtol=1e-4)
    # Cameras that take no gradient: the camera adjoint is skipped, the
    # camera gradients are None and every surfel gradient is the same bits
    # (the projection adjoint sums over cameras without atomics).
    plain = native.records_backward(
        gpu["means"], gpu["quaternions"], gpu["scales"], gpu["view_matrices"],
        gpu["intrinsics"], sh_args, sh, out["row_of_pair"], out["geometry"],
        to_gpu(g_geometry), to_gpu(g_projected), to_gpu(g_app), to_gpu(g_op),
        camera_grads=False)
    assert plain[3] is None and plain[4] is None
    for index in [0, 1, 2] + order[5:]:
        assert torch.equal(plain[index], got[index]), names[order.index(index)]
