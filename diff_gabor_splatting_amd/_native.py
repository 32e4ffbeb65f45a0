"""Host side of the HIP library: the reference's ``_C`` operators over the C ABI.

The reference binds four pybind11 functions (``src/gabor_splatting/csrc/
bindings.cpp:5-10``): ``rasterize_forward``, ``rasterize_backward``,
``evaluate_sh_forward`` and ``evaluate_sh_backward``. This module exposes the
same names, argument meaning and error behaviour (structural violations raise
``RuntimeError`` like ``TORCH_CHECK``), implemented by allocating outputs with
the torch caching allocator and calling ``libgabor_hip.so`` on the current
HIP stream. It adds the projection operators (the reference runs projection
as PyTorch ops) and visible-pair packing.

The functions a render calls - the record front end, value checks, binning,
the compositor operators and their accumulators - are implemented in C++
(``csrc/host.cpp``, the ``_host`` extension module, as the reference's host
functions are); here they only keep their Python signatures and docstrings.
The rest call the C ABI through ctypes. Both reach the library loaded here:
the extension receives its entry point addresses at load.

The library and the extension are loaded at import; there is no fallback path.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

_LIBRARY_PATH = Path(__file__).resolve().parent / "libgabor_hip.so"

TILE = 16
GEOMETRY_SIZE = 17
# Binning status bits (GS_BIN_* in include/gabor_hip.h).
BINNING_OVERFLOW = 1
BINNING_BAD_INDEX = 2
MAP_SIZE = 9
INT_MAX = 2**31 - 1
# Replay-list entries carry a tile-list position in 28 bits.
REPLAY_MAX_ENTRIES = 2**28 - 1
# Split tiles (gs_render_forward's segment_* arguments): images with fewer
# tiles than SPLIT_MAX_TILES have too few workgroups to hide a long tile
# list, so tiles longer than SPLIT_LENGTH records are composited (and their
# backward replayed) in segments of that many records, one workgroup each.
# The segment length does not depend on the intersection count, and the
# checkpoint slots are at most SPLIT_MAX_SLOTS, so a render into a
# fixed-capacity point list splits its tiles exactly as the synchronised
# render does and gives the same bits.
SPLIT_MAX_TILES = 2048
SPLIT_LENGTH = 64
SPLIT_MAX_SLOTS = 16384


def split_length(tiles: int, intersections: int) -> int:
    """List records per segment of a split tile (a multiple of 64), or 0 to
    split none."""
    if tiles >= SPLIT_MAX_TILES or intersections <= 0:
        return 0
    return SPLIT_LENGTH


def split_slots(intersections: int, length: int, tiles: int) -> int:
    """Checkpoint slots: a tile of L > length records needs ceil(L / length)
    <= floor(L / length) + 1 of them, and at most min(tiles, M / (length +
    1)) tiles are that long, so floor(M / length) + min(tiles, floor(M /
    (length + 1))) + 1 suffice; capped at SPLIT_MAX_SLOTS (the slots go to
    tiles in tile order; later tiles past the cap are not split)."""
    if not length:
        return 0
    return min(intersections // length + min(tiles, intersections // (length + 1)) + 1,
               SPLIT_MAX_SLOTS)


CHECKPOINT_FLOATS = 13


def split_index_length(tiles: int, slots: int) -> int:
    """Length (int32) of gs_render_forward's segment_index buffer: slot bases
    per tile, replay lengths per slot, then the forward's (tile, segment)
    work list at an even offset."""
    return (tiles + slots + 1) // 2 * 2 + 2 * (tiles + slots)


_c_int = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float
_c_ptr = ctypes.c_void_p

_SIGNATURES = {
    "gs_last_error": (ctypes.c_char_p, []),
    "gs_abi_version": (_c_int, []),
    "gs_project_forward": (
        _c_int,
        [_c_ptr] * 5 + [_c_i64] * 3 + [_c_int, _c_int, _c_float, _c_float] + [_c_ptr] * 6,
    ),
    "gs_project_backward_workspace_size": (_c_size, [_c_i64] * 3),
    "gs_project_backward": (
        _c_int,
        [_c_ptr] * 5 + [_c_i64] * 3 + [_c_ptr] * 9 + [_c_ptr, _c_size, _c_ptr],
    ),
    "gs_sh_forward": (_c_int, [_c_ptr] * 4 + [_c_i64] * 3 + [_c_int, _c_ptr]),
    "gs_sh_backward": (_c_int, [_c_ptr] * 7 + [_c_i64] * 3 + [_c_int, _c_ptr]),
    "gs_check_values": (
        _c_int,
        [_c_ptr, _c_ptr, _c_int] + [_c_ptr] * 5 + [_c_i64] + [_c_ptr] * 2 + [_c_i64]
        + [_c_ptr, _c_ptr],
    ),
    "gs_scan_workspace_size": (_c_size, [_c_i64]),
    "gs_pack_visible": (_c_int, [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "gs_records_forward": (
        _c_int,
        [_c_ptr] * 11
        + [_c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_float, _c_float]
        + [_c_ptr] * 13,
    ),
    "gs_records_backward_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int]),
    "gs_records_backward": (
        _c_int,
        [_c_ptr] * 7 + [_c_int, _c_i64, _c_i64, _c_i64] + [_c_ptr] * 4 + [_c_i64]
        + [_c_ptr] * 14 + [_c_size, _c_ptr],
    ),
    "gs_count_tiles": (
        _c_int,
        [_c_ptr, _c_ptr, _c_i64, _c_int, _c_int, _c_ptr, _c_ptr, _c_size, _c_ptr],
    ),
    "gs_emit_tiles": (
        _c_int,
        [_c_ptr] * 4 + [_c_i64, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr],
    ),
    "gs_sort_workspace_size": (_c_size, [_c_i64]),
    "gs_sort_pairs": (
        _c_int,
        [_c_ptr] * 4 + [_c_i64, _c_int, _c_int, _c_ptr, _c_size, _c_ptr],
    ),
    "gs_sort32_workspace_size": (_c_size, [_c_i64]),
    "gs_sort_pairs32": (
        _c_int,
        [_c_ptr] * 4 + [_c_i64, _c_int, _c_int, _c_ptr, _c_size, _c_ptr],
    ),
    "gs_find_ranges": (_c_int, [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr]),
    "gs_bin_order_workspace_size": (_c_size, [_c_i64]),
    "gs_bin_order": (
        _c_int,
        [_c_ptr] * 3 + [_c_i64, _c_int, _c_int] + [_c_ptr] * 6 + [_c_size, _c_ptr],
    ),
    "gs_bin_order_count": (
        _c_int,
        [_c_ptr] * 3 + [_c_i64, _c_int, _c_int] + [_c_ptr] * 4 + [_c_size, _c_ptr],
    ),
    "gs_bin_order_sort": (_c_int, [_c_i64, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "gs_bin_tiles_workspace_size": (_c_size, [_c_i64]),
    "gs_bin_tiles": (
        _c_int,
        [_c_ptr] * 3 + [_c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr,
                        _c_ptr, _c_size, _c_ptr],
    ),
    "gs_bin_tiles_bounded": (
        _c_int,
        [_c_ptr] * 3 + [_c_i64, _c_i64, _c_ptr, _c_i64, _c_int, _c_int] + [_c_ptr] * 4
        + [_c_size, _c_ptr],
    ),
    "gs_bin_blocks_fit": (_c_int, [_c_i64, _c_int, _c_int]),
    "gs_bin_blocks_count": (
        _c_int,
        [_c_ptr] * 3 + [_c_i64, _c_int, _c_int, _c_float, _c_float] + [_c_ptr] * 3
        + [_c_size, _c_ptr],
    ),
    "gs_bin_blocks_sort": (
        _c_int, [_c_i64, _c_float, _c_float, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr],
    ),
    "gs_bin_blocks_tiles_workspace_size": (_c_size, [_c_i64, _c_i64, _c_int, _c_int]),
    "gs_bin_blocks_tiles": (
        _c_int,
        [_c_ptr] * 3 + [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int] + [_c_ptr] * 4
        + [_c_size, _c_ptr],
    ),
    "gs_bin_blocks_tiles_bounded": (
        _c_int,
        [_c_ptr] * 3 + [_c_i64, _c_i64, _c_ptr, _c_i64, _c_int, _c_int] + [_c_ptr] * 4
        + [_c_size, _c_ptr],
    ),
    "gs_render_workspace_size": (_c_size, [_c_i64, _c_int, _c_int]),
    "gs_render_backward_workspace_size": (_c_size, [_c_i64, _c_int, _c_int, _c_i64]),
    "gs_render_forward": (
        _c_int,
        [_c_int]
        + [_c_ptr] * 7
        + [_c_i64, _c_int, _c_int, _c_float, _c_float]
        + [_c_ptr] * 5
        + [_c_i64]
        + [_c_ptr]
        + [_c_int, _c_ptr, _c_ptr, _c_i64]
        + [_c_ptr, _c_size, _c_ptr],
    ),
    "gs_render_forward_static": (
        _c_int,
        [_c_int]
        + [_c_ptr] * 7
        + [_c_i64, _c_int, _c_int, _c_float, _c_float]
        + [_c_ptr] * 5
        + [_c_i64]
        + [_c_ptr] * 2,
    ),
    "gs_render_backward": (
        _c_int,
        [_c_int]
        + [_c_ptr] * 11
        + [_c_int, _c_ptr, _c_ptr, _c_i64]
        + [_c_ptr] * 2
        + [_c_i64, _c_int, _c_int, _c_float, _c_float]
        + [_c_ptr] * 6
        + [_c_size, _c_ptr],
    ),
    "gs_profile_enable": (_c_int, [_c_int]),
    "gs_profile_read": (_c_int, [_c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_i64)]),
    "gs_diagnostics_query": (_c_int, [ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)]),
    "gs_diagnostics_set": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr]),
}

PROFILE_FAMILIES = {
    "project_forward": 0,
    "project_backward": 1,
    "sh_forward": 2,
    "sh_backward": 3,
    "binning": 4,
    "sort": 5,
    "render_forward": 6,
    "render_backward": 7,
    "validate": 8,
}


try:
    from . import _host
except ImportError as error:
    raise ImportError(
        "the _host extension (csrc/host.cpp) is not built; run `python -m "
        "diff_gabor_splatting_amd.build` (or __graft_entry__.build()) first. There is no "
        "Python fallback."
    ) from error


def _load(path: Path = _LIBRARY_PATH) -> ctypes.CDLL:
    if not path.exists():
        raise ImportError(
            f"{path.name} is not built; run `python -m diff_gabor_splatting_amd.build` "
            "(or __graft_entry__.build()) first. There is no CPU fallback."
        )
    library = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in _SIGNATURES.items():
        function = getattr(library, name)
        function.restype = restype
        function.argtypes = argtypes
    return library


def _bind_host(library: ctypes.CDLL) -> None:
    """Hand the extension the addresses of the entry points it calls."""
    _host.bind({name: ctypes.cast(getattr(library, name), ctypes.c_void_p).value
                for name in _host.entry_points()})


lib = _load()
_bind_host(lib)
_library_path = _LIBRARY_PATH


def use_library(path: Path) -> None:
    """Route every later call of this module through the library at ``path``,
    a build of the same sources with the same entry points (the diagnostics
    build). Tensors and streams are unaffected; kernels already queued keep
    running from the library that launched them. The switch is process-wide
    and not synchronised with renders: call it while no other thread
    renders."""
    global lib, _library_path
    lib = _load(Path(path))
    _bind_host(lib)
    _library_path = Path(path)


def library_path() -> Path:
    """The library every call of this module currently goes through."""
    return _library_path


def exported_symbols() -> list[str]:
    """Names of every C-ABI entry point this module binds."""
    return list(_SIGNATURES)


def _check(status: int) -> None:
    if status != 0:
        message = lib.gs_last_error().decode(errors="replace")
        raise RuntimeError(message or f"gabor HIP call failed with status {status}")


def _ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def tile_grid(width: int, height: int) -> tuple[int, int]:
    """Tiles per row and per column: ceil(W/16) x ceil(H/16)."""
    return (width + TILE - 1) // TILE, (height + TILE - 1) // TILE


def sort_end_bit(tile_count: int) -> int:
    """Highest key bit that can be set: 32 depth bits plus the tile-id width."""
    return 32 + max(int(tile_count) - 1, 0).bit_length()


def check_intersections(count: int) -> None:
    """Intersection-count guard of rasterizeForward (rasterize.cu:469)."""
    _require(count <= INT_MAX, "tile intersection count exceeds int32")


def check_image_tiles(images: int, width: int, height: int) -> None:
    """Image-tile guard of rasterizeForward (rasterize.cu:443-445)."""
    tw, th = tile_grid(width, height)
    _require(images * tw * th <= INT_MAX, "image tile count exceeds int32")


# --------------------------------------------------------------------------
# Binning primitives (exposed separately for bit-exact tests).


def count_tiles(geometry: torch.Tensor, radii: torch.Tensor, width: int, height: int):
    """Inclusive prefix sum of per-pair tile counts (int64 [Q])."""
    device = geometry.device
    count = geometry.size(0)
    offsets = torch.empty(count, dtype=torch.int64, device=device)
    if count:
        workspace = _workspace(lib.gs_scan_workspace_size(count), device)
        _check(
            lib.gs_count_tiles(
                _ptr(geometry), _ptr(radii), count, width, height, _ptr(offsets),
                _ptr(workspace), workspace.numel(), _stream(device),
            )
        )
    return offsets


def emit_tiles(geometry, radii, image_ids, offsets, width, height, intersections):
    """Unsorted (key, value) pairs, one per covered tile (rasterize.cu:43-56)."""
    device = geometry.device
    keys = torch.empty(intersections, dtype=torch.int64, device=device)
    values = torch.empty(intersections, dtype=torch.int32, device=device)
    if intersections:
        _check(
            lib.gs_emit_tiles(
                _ptr(geometry), _ptr(radii), _ptr(image_ids), _ptr(offsets), geometry.size(0),
                width, height, _ptr(keys), _ptr(values), _stream(device),
            )
        )
    return keys, values


def sort_pairs(keys: torch.Tensor, values: torch.Tensor, begin_bit: int = 0, end_bit: int = 64):
    """Stable LSD radix sort of uint64 keys (stored as int64) with int32 values."""
    device = keys.device
    m = keys.numel()
    sorted_keys = torch.empty_like(keys)
    sorted_values = torch.empty_like(values)
    if m:
        workspace = _workspace(lib.gs_sort_workspace_size(m), device)
        _check(
            lib.gs_sort_pairs(
                _ptr(keys), _ptr(sorted_keys), _ptr(values), _ptr(sorted_values), m, begin_bit,
                end_bit, _ptr(workspace), workspace.numel(), _stream(device),
            )
        )
    return sorted_keys, sorted_values


def sort_pairs32(keys: torch.Tensor, values: torch.Tensor | None = None, begin_bit: int = 0,
                 end_bit: int = 32):
    """Stable LSD radix sort of uint32 keys (stored as int32) with int32
    values, or of the keys alone: (sorted keys, sorted values or None)."""
    device = keys.device
    m = keys.numel()
    sorted_keys = torch.empty_like(keys)
    sorted_values = None if values is None else torch.empty_like(values)
    if m:
        workspace = _workspace(lib.gs_sort32_workspace_size(m), device)
        _check(
            lib.gs_sort_pairs32(
                _ptr(keys), _ptr(sorted_keys), _ptr(values), _ptr(sorted_values), m, begin_bit,
                end_bit, _ptr(workspace), workspace.numel(), _stream(device),
            )
        )
    return sorted_keys, sorted_values


def find_ranges(sorted_keys: torch.Tensor, tiles: int) -> torch.Tensor:
    """Per-tile [first, last) runs of the sorted keys (int32 [tiles, 2])."""
    device = sorted_keys.device
    ranges = torch.empty((tiles, 2), dtype=torch.int32, device=device)
    _check(
        lib.gs_find_ranges(
            _ptr(sorted_keys), sorted_keys.numel(), _ptr(ranges), tiles, _stream(device)
        )
    )
    return ranges


def bin_order(geometry: torch.Tensor, radii: torch.Tensor, image_ids: torch.Tensor,
              width: int, height: int):
    """Depth-first binning, stage 1: (order int32 [Q], starts int64 [Q], rects
    int32 [Q, 4], totals int64 [2] on the device = (M, V): the intersection
    count and the number of pairs with tiles). No host synchronisation."""
    return _host.bin_order(geometry, radii, image_ids, width, height)


def bin_tiles(order, starts, rects, images, width, height, intersections, visible=-1,
              status=None):
    """Depth-first binning, stage 2: (point_list int32 [M], ranges int32
    [I*tw*th, 2]), the result of emit_tiles + sort_pairs + find_ranges
    (rasterize.cu:43-69, 470-501). ``visible`` is stage 1's count of pairs
    with tiles (-1: unknown), which selects the packed-key tile sort when it
    fits. ``status`` (an int32 [1] device tensor, or None) receives the
    BINNING_* bits: BINNING_BAD_INDEX when a sort output failed its range
    check (see gs_bin_tiles)."""
    return _host.bin_tiles(order, starts, rects, images, width, height, intersections, visible,
                           status)


def bin_blocks_order(geometry, radii, image_ids, width, height, near_plane=0.0,
                     far_plane=0.0):
    """Stage 1 of the block path: (order int32 [Q], starts int64 [Q], rects
    int32 [Q, 4], totals int64 [3] on the device = (M, V, E)). starts[j] is
    the first (pair, tile block) entry of depth rank j, rects hold each
    pair's tile rectangle with the images' tile rows stacked, and E is the
    number of (pair, block) entries. With clipping planes (near > 0) the
    depth sort runs on fewer bits (see gs_bin_blocks_count); the pairs with
    tiles must then have their depths between them."""
    return _host.bin_blocks_order(geometry, radii, image_ids, width, height, near_plane,
                                  far_plane)


def bin_blocks_tiles(order, starts, rects, images, width, height, intersections, entries,
                     visible=-1, status=None):
    """Stage 2 of the block path: (point_list, ranges), bit for bit those of
    bin_tiles, from bin_blocks_order's outputs and totals (M, V, E)."""
    return _host.bin_blocks_tiles(order, starts, rects, images, width, height, intersections,
                                  entries, visible, status)


def set_binning_path(name: str) -> None:
    """Stage 2 of the binning, synchronised or bounded: "blocks" (the
    default: the block path wherever gs_bin_blocks_fit) or "tiles" (always
    the tile sort). Both give the same point list and ranges (within a
    bounded render's capacity); process-wide."""
    _host.set_binning_path(name)


def binning_path() -> str:
    return _host.binning_path()


def bin_tiles_bounded(order, starts, rects, images, width, height, capacity, intersections):
    """Depth-first binning, stage 2, without reading M on the host: a point
    list of `capacity` entries (those past the live count are -1) and the
    live count `intersections` (int64 [1] on the device). Returns (point_list, ranges, overflow) with overflow an
    int32 [1] device word of BINNING_* bits: BINNING_OVERFLOW when M
    exceeded the capacity, BINNING_BAD_INDEX as in bin_tiles."""
    return _host.bin_tiles_bounded(order, starts, rects, images, width, height, capacity,
                                   intersections)


def bin_blocks_tiles_bounded(order, starts, rects, images, width, height, capacity, totals):
    """Stage 2 of the block path without reading the totals on the host: a
    point list of `capacity` entries, with M and E read from `totals` (int64
    [3] on the device, bin_blocks_order's). Returns (point_list, ranges,
    overflow) as bin_tiles_bounded does; within the capacity the point list's
    first M entries and the ranges equal bin_blocks_tiles', the rest -1."""
    return _host.bin_blocks_tiles_bounded(order, starts, rects, images, width, height, capacity,
                                          totals)


def bin_depth_first(geometry, radii, image_ids, images, width, height, overlap=None,
                    capacity=None, flags=None, violations=None, near_plane=0.0, far_plane=0.0):
    """Both binning stages with the one host synchronisation for M between
    them (rasterize.cu:466-469): (point_list, ranges).

    M is copied to pinned host memory behind stage 1 and the host waits on
    an event recorded after that copy, not on the stream, so GPU work that
    ``overlap()`` queues (independent of M) runs while the host waits.
    With ``capacity`` there is no synchronisation at all: the point list
    has that many entries, and ``flags(overflow, total)`` receives the
    bounded stage 2's status word (bin_blocks_tiles_bounded's, or
    bin_tiles_bounded's where the block path does not fit or the tile path
    is selected) and the live count M, both device tensors, for the caller
    to fold into its own records. ``violations`` (a device
    int32 word of gs_check_values and a function that raises for a nonzero
    word) is read back with M and reported before M is checked or used.
    ``near_plane``/``far_plane`` (an addition): the planes the pairs with
    tiles lie between, which narrow the block path's depth keys; 0, 0 (the
    default) sorts the raw depth bits."""
    return _host.bin_depth_first(geometry, radii, image_ids, images, width, height, overlap,
                                 capacity, flags, violations, near_plane, far_plane)


def pack_visible(radii: torch.Tensor, with_rows: bool = False, sync: bool = True):
    """Ascending indices of pairs with radii > 0 (int64). Synchronises once.

    With ``with_rows`` also returns row_of_pair (int32, the packed row of
    every pair or -1). With ``sync=False`` nothing is read back: the indices
    keep one entry per pair (those past the visible count V undefined) and
    V, a device int64 tensor of one element, is returned last."""
    return _host.pack_visible(radii, with_rows, sync)


# --------------------------------------------------------------------------
# Input value contracts (rendering.py:88-153).

CHECK_MAX_TENSORS = 16


def check_tensors(tensors: dict, device: torch.device) -> None:
    """Require every ``name: (value, shape)`` entry to be a contiguous float32
    tensor of exactly that shape on ``device``: TypeError for a non-tensor,
    ValueError otherwise, naming the first entry that fails."""
    _host.check_tensors(tensors, device)


def check_values(tensors, quaternions, scales, opacities, view_matrices, intrinsics,
                 weights=None, magnitudes=None) -> int:
    """Violated-contract bits of gs_check_values over the given inputs.

    Bit k < 16: tensors[k] is not finite; the GS_CHECK_* bits above that
    name the value contracts. One launch and one read-back of the word."""
    word = check_values_word(tensors, quaternions, scales, opacities, view_matrices,
                             intrinsics, weights, magnitudes)
    return int(word.item()) & 0xFFFFFFFF


def check_values_word(tensors, quaternions, scales, opacities, view_matrices, intrinsics,
                      weights=None, magnitudes=None) -> torch.Tensor:
    """check_values without the read-back: the int32 [1] device word."""
    return _host.check_values_word(list(tensors), quaternions, scales, opacities, view_matrices,
                                   intrinsics, weights, magnitudes)


# --------------------------------------------------------------------------
# Fused projection + SH + record assembly (the renderer's front end).


def records_forward(means, quaternions, scales, opacities, view_matrices, intrinsics, sh,
                    shared, sh_degree, width, height, near_plane, far_plane, packed,
                    fixed_rows=False):
    """Compositor rows for every visible (packed) or every (dense) pair.

    With ``packed`` and ``fixed_rows`` the visible count is not read back:
    every output keeps one row per pair, the packed rows first; the rows past
    them have radius 0 (so binning skips them), zero projected means and ids
    of -1.

    means/quaternions/scales [S,N,*], view_matrices [S,C,4,4], intrinsics
    [S,C,3,3]; with SH (sh_degree >= 0) also opacities [S,N], sh = (first,
    second) [S,N,K,3] and shared = (weights, magnitudes, phases) [S,N,4].
    Returns a dict of geometry [Q,17], projected_means [Q,2], row_radii [Q],
    primitive_ids [Q], image_ids [Q], the meta ids scene_ids / camera_ids /
    surfel_ids [Q], dense_radii [S,C,N], row_of_pair ([S*C*N] int32 or None)
    and selected (packed pair indices or None), plus appearance [Q,18] and
    opacity_rows [Q] with SH.
    """
    return _host.records_forward(means, quaternions, scales, opacities, view_matrices, intrinsics,
                                 sh, shared, sh_degree, width, height, near_plane, far_plane,
                                 packed, fixed_rows)


def records_backward(means, quaternions, scales, view_matrices, intrinsics, sh, sh_degree,
                     row_of_pair, geometry, grad_geometry, grad_projected_means,
                     grad_appearance, grad_opacity_rows, camera_grads=True):
    """Gradients of (means, quaternions, scales, view_matrices, intrinsics) and,
    with SH, of (first, second, weights, magnitudes, phases, opacities).
    With camera_grads False the camera adjoint is skipped and the view and
    intrinsics gradients are None."""
    return _host.records_backward(means, quaternions, scales, view_matrices, intrinsics, sh,
                                  sh_degree, row_of_pair, geometry, grad_geometry,
                                  grad_projected_means, grad_appearance, grad_opacity_rows,
                                  bool(camera_grads))


# --------------------------------------------------------------------------
# Compositor operators (the reference's _C.rasterize_forward / backward).


# Map channel groups in map order: rgb, alpha, depth, normals, distortion.
MAP_GROUPS = (3, 1, 1, 3, 1)


def split_map_groups(maps: torch.Tensor) -> list:
    """The five channel-group views [..., k] of a [..., 9] map tensor."""
    groups, first = [], 0
    for k in MAP_GROUPS:
        groups.append(maps[..., first:first + k])
        first += k
    return groups


def _flat_pixel_stride(t: torch.Tensor):
    """(pixel stride, channel stride) in elements when every pixel of the
    [I,H,W,k] tensor t sits at p * pixel_stride from t's first element,
    p = (i*H + y)*W + x; None otherwise."""
    *pixel_dims, k = t.shape
    strides = t.stride()
    stride = None
    inner = 1
    for size, step in reversed(list(zip(pixel_dims, strides[:-1]))):
        if size > 1:
            if stride is None:
                stride = step // inner if step % inner == 0 else -1
            if stride < 0 or step != stride * inner:
                return None
        inner *= size
    return (0 if stride is None else stride), (strides[-1] if k > 1 else 0)


def _map_group_args(groups, what: str):
    """ctypes arrays (device pointers, [pixel, channel] strides) of the groups."""
    pointers = (ctypes.c_void_p * len(MAP_GROUPS))()
    strides = (ctypes.c_int64 * (2 * len(MAP_GROUPS)))()
    for g, t in enumerate(groups):
        if t is None:
            continue
        layout = _flat_pixel_stride(t)
        _require(layout is not None, f"{what} must have uniformly strided pixels")
        pointers[g] = t.data_ptr()
        strides[2 * g], strides[2 * g + 1] = layout
    return pointers, strides


def rasterize_forward(
    geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds,
    width, height, neural, near_plane, far_plane, outputs=None, overlap=None, capacity=None,
    flags=None, replay=False, violations=None, split=None,
):
    """Bin, sort and composite: returns [maps, point_list, ranges, state, contributors].

    Mirrors rasterizeForward (rasterize.cu:426-503), including its structural
    checks, its one host synchronisation for the intersection count and its
    output shapes: maps [I,H,W,9], point_list int32 [M], ranges int32
    [I*tw*th, 2], state [I,H,W,3], contributors int32 [I,H,W].


    ``outputs`` (an addition): five float32 tensors [I,H,W,k], k in
    MAP_GROUPS, that receive the map channel groups instead of one maps
    tensor; the first returned item is then that tuple. ``overlap`` (an
    addition): called once while the host waits for M, to queue GPU work
    that does not depend on it. ``capacity`` / ``flags`` (additions): bin
    into a point list of fixed capacity without reading M on the host (see
    bin_depth_first). ``replay`` (an addition): also return, as a sixth item,
    the tiles' replay lists for rasterize_backward - (lists [M, 2] int32,
    counts [I*tw*th] int32, segments): per tile, the point-list entries that
    some pixel took, in list order - or None when the point list is too long
    for them (2^28 entries or more). ``segments`` is None, or (length,
    checkpoint state, checkpoint index) when tiles are split: tiles longer
    than ``length`` records are composited in segments of that many list
    records, merged per pixel, and their backward is replayed in the same
    segments, each from a checkpoint the forward wrote (see
    gs_render_forward). ``split`` (an addition): the segment length, 0 for
    none, or None to choose it (split_length: only images with fewer than
    SPLIT_MAX_TILES tiles are split, whether or not a backward follows). ``violations`` (an addition): a pending value
    check, raised with the read-back of M (see bin_depth_first).
    """
    return _host.rasterize_forward(
        geometry, appearance, opacities, primitive_ids, image_ids, radii, backgrounds, width,
        height, neural, near_plane, far_plane, outputs, overlap, capacity, flags, replay,
        violations, -1 if split is None else int(split), SPLIT_MAX_TILES, SPLIT_LENGTH,
        SPLIT_MAX_SLOTS,
    )


def zero_accumulators(geometry, appearance, opacities, backgrounds, shared=True):
    """Zeroed gradient accumulators for rasterize_backward: with ``shared``,
    contiguous views of one allocation cleared by one fill; else separate
    tensors (for callers that must not return aliased tensors). With
    appearance column groups the appearance accumulator is a tuple of four."""
    return _host.zero_accumulators(geometry, appearance, opacities, backgrounds, shared)


def rasterize_backward(
    geometry, appearance, opacities, primitive_ids, backgrounds, point_list, ranges, state,
    contributors, grad_maps, width, height, neural, near_plane, far_plane, accumulators=None,
    replay=None,
):
    """Reverse compositing: returns [grad_geometry, grad_appearance, grad_opacities,
    grad_backgrounds] (rasterize.cu:506-529).

    ``accumulators`` may hold, for the neural renderer, a tuple of the
    SIREN's four parameter groups' gradients in place of the appearance
    rows' (an addition, zero_accumulators with a tuple): input weights
    [P,30], input biases [P,6], output weights [P,18], output biases [P,3];
    grad_appearance is then that tuple.

    ``grad_maps`` is the reference's [I,H,W,9] tensor or (an addition) a
    sequence of five per-group gradients [I,H,W,k] in MAP_GROUPS order, each
    a tensor of any strides or None (zero); strided views are read in place.
    ``accumulators`` (an addition): zeroed tensors from zero_accumulators,
    cleared ahead of time, that receive and are returned as the gradients.
    ``replay`` (an addition): the replay lists returned by rasterize_forward
    (or None); the gradients are the same, computed from fewer records.
    """
    return _host.rasterize_backward(
        geometry, appearance, opacities, primitive_ids, backgrounds, point_list, ranges, state,
        contributors, grad_maps, width, height, neural, near_plane, far_plane, accumulators,
        replay,
    )


# --------------------------------------------------------------------------
# Spherical harmonics (the reference's _C.evaluate_sh_forward / backward).


def _check_sh(first, second, directions, degree) -> None:
    """Mirror of checkSH (spherical_harmonics.cu:88-103)."""
    _require(0 <= degree <= 3, "SH degree must be 0 through 3")
    for value in (first, second, directions):
        _require(
            value.is_cuda
            and value.dtype == torch.float32
            and value.is_contiguous()
            and value.device == first.device,
            "SH tensors must be contiguous float32 on the same CUDA device",
        )
    _require(
        first.dim() == 4
        and second.shape == first.shape
        and first.size(2) == (degree + 1) ** 2
        and first.size(3) == 3,
        "SH coefficients must have shape [B, N, K, 3]",
    )
    _require(
        directions.dim() == 4
        and directions.size(0) == first.size(0)
        and directions.size(2) == first.size(1)
        and directions.size(3) == 3,
        "SH directions must have shape [B, C, N, 3]",
    )
    _require(directions.numel() // 3 <= INT_MAX, "too many SH pairs")


def evaluate_sh_forward(first, second, directions, degree):
    """Both SH colours per (scene, camera, surfel): [S, C, N, 6]."""
    _check_sh(first, second, directions, degree)
    device = first.device
    scenes, cameras, n = directions.shape[:3]
    with torch.cuda.device(device):
        colors = torch.empty((scenes, cameras, n, 6), dtype=torch.float32, device=device)
        _check(
            lib.gs_sh_forward(
                _ptr(first), _ptr(second), _ptr(directions), _ptr(colors), scenes, cameras, n,
                degree, _stream(device),
            )
        )
    return colors


def evaluate_sh_backward(first, second, directions, grad_colors, degree):
    """Coefficient gradients summed over cameras and per-pair direction gradients."""
    _check_sh(first, second, directions, degree)
    _require(
        grad_colors.device == first.device
        and grad_colors.dtype == torch.float32
        and grad_colors.is_contiguous()
        and grad_colors.shape == (*directions.shape[:3], 6),
        "invalid SH color gradients",
    )
    device = first.device
    scenes, cameras, n = directions.shape[:3]
    with torch.cuda.device(device):
        gf = torch.empty_like(first)
        gs = torch.empty_like(second)
        gd = torch.empty_like(directions)
        _check(
            lib.gs_sh_backward(
                _ptr(first), _ptr(second), _ptr(directions), _ptr(grad_colors), _ptr(gf),
                _ptr(gs), _ptr(gd), scenes, cameras, n, degree, _stream(device),
            )
        )
    return [gf, gs, gd]


# --------------------------------------------------------------------------
# Projection (the reference's PyTorch project_surfaces, rendering.py:176-218).


def project_forward(means, quaternions, scales, view_matrices, intrinsics, width, height,
                    near_plane, far_plane):
    """Returns transform [S,C,N,3,3], xy [S,C,N,2], normals [S,C,N,3],
    directions [S,C,N,3] and radii int32 [S,C,N]."""
    device = means.device
    scenes, n = means.shape[:2]
    cameras = view_matrices.shape[1]
    with torch.cuda.device(device):
        transform = torch.empty((scenes, cameras, n, 3, 3), dtype=torch.float32, device=device)
        xy = torch.empty((scenes, cameras, n, 2), dtype=torch.float32, device=device)
        normals = torch.empty((scenes, cameras, n, 3), dtype=torch.float32, device=device)
        directions = torch.empty((scenes, cameras, n, 3), dtype=torch.float32, device=device)
        radii = torch.empty((scenes, cameras, n), dtype=torch.int32, device=device)
        _check(
            lib.gs_project_forward(
                _ptr(means), _ptr(quaternions), _ptr(scales), _ptr(view_matrices),
                _ptr(intrinsics), scenes, cameras, n, width, height, near_plane, far_plane,
                _ptr(transform), _ptr(xy), _ptr(normals), _ptr(directions), _ptr(radii),
                _stream(device),
            )
        )
    return transform, xy, normals, directions, radii


def project_backward(means, quaternions, scales, view_matrices, intrinsics, grad_transform,
                     grad_xy, grad_normals, grad_directions):
    """Gradients of (means, quaternions, scales, view_matrices, intrinsics)."""
    device = means.device
    scenes, n = means.shape[:2]
    cameras = view_matrices.shape[1]

    def contiguous(value):
        return None if value is None else value.contiguous()

    grad_transform, grad_xy = contiguous(grad_transform), contiguous(grad_xy)
    grad_normals, grad_directions = contiguous(grad_normals), contiguous(grad_directions)
    with torch.cuda.device(device):
        g_means = torch.empty_like(means)
        g_quats = torch.empty_like(quaternions)
        g_scales = torch.empty_like(scales)
        g_views = torch.empty_like(view_matrices)
        g_intrinsics = torch.empty_like(intrinsics)
        workspace = _workspace(lib.gs_project_backward_workspace_size(scenes, cameras, n), device)
        _check(
            lib.gs_project_backward(
                _ptr(means), _ptr(quaternions), _ptr(scales), _ptr(view_matrices),
                _ptr(intrinsics), scenes, cameras, n, _ptr(grad_transform), _ptr(grad_xy),
                _ptr(grad_normals), _ptr(grad_directions), _ptr(g_means), _ptr(g_quats),
                _ptr(g_scales), _ptr(g_views), _ptr(g_intrinsics), _ptr(workspace),
                workspace.numel(), _stream(device),
            )
        )
    return g_means, g_quats, g_scales, g_views, g_intrinsics


# --------------------------------------------------------------------------
# Kernel timing.


def profile_enable(enable: bool) -> None:
    _check(lib.gs_profile_enable(1 if enable else 0))


def profile_read(family: str) -> tuple[float, int]:
    """Total milliseconds and launch count of one kernel family."""
    total = ctypes.c_double()
    launches = _c_i64()
    _check(lib.gs_profile_read(PROFILE_FAMILIES[family], ctypes.byref(total), ctypes.byref(launches)))
    return total.value, launches.value
