"""The C-ABI library loads and exports every entry point include/*.h declares.

Only argument-validation paths are called here: they return before any HIP
call, so no GPU is needed.
"""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        names |= set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(gs_\w+)\s*\(", text, re.M))
    return names


def test_header_declares_the_api():
    names = declared_symbols()
    for required in ("gs_project_forward", "gs_project_backward", "gs_sh_forward",
                     "gs_sh_backward", "gs_pack_visible", "gs_count_tiles", "gs_emit_tiles",
                     "gs_sort_pairs", "gs_find_ranges", "gs_render_forward",
                     "gs_render_backward", "gs_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from diff_gabor_splatting_amd import _native

    library = ctypes.CDLL(str(_native._LIBRARY_PATH))
    for name in sorted(declared_symbols()):
        assert hasattr(library, name), name
    assert set(_native.exported_symbols()) == declared_symbols()
    assert _native.lib.gs_abi_version() == 13


def test_argument_errors_return_status_and_message():
    from diff_gabor_splatting_amd import _native

    lib = _native.lib
    status = lib.gs_sort_pairs(None, None, None, None, 10, 0, 70, None, 0, None)
    assert status == 1 and b"bit range" in lib.gs_last_error()
    status = lib.gs_project_forward(*([None] * 5), 0, 1, 4, 8, 8, 0.2, 100.0, *([None] * 6))
    assert status == 1 and b"scenes" in lib.gs_last_error()
    status = lib.gs_sh_forward(None, None, None, None, 1, 1, 4, 5, None)
    assert status == 1 and b"degree" in lib.gs_last_error()
    status = lib.gs_find_ranges(None, -1, None, 4, None)
    assert status == 2
    status = lib.gs_render_forward(0, *([None] * 7), 1, 16, 16, 1.0, 0.5, *([None] * 5), 0,
                                   None, 0, None, None, 0, None, 0, None)
    assert status == 1 and b"clipping" in lib.gs_last_error()
    # Split-tile arguments are checked before any launch.
    dummy = ctypes.c_void_p(16)
    maps = (ctypes.c_void_p * 5)(*([16] * 5))
    strides = (ctypes.c_int64 * 10)()
    forward = [0, *([dummy] * 7), 1, 16, 16, 0.5, 1.0, maps, strides, dummy, dummy]
    status = lib.gs_render_forward(*forward, None, 0, None, 100, dummy, dummy, 4, dummy, 1 << 20,
                                   None)
    assert status == 1 and b"multiple of 64" in lib.gs_last_error()
    backward = [0, *([dummy] * 7), dummy, dummy, None, None]
    # (..., grad_geometry, grad_appearance, grad_appearance_columns (null:
    # rows), grad_opacities, grad_backgrounds, workspace, bytes, stream)
    status = lib.gs_render_backward(*backward, 64, dummy, dummy, 4, maps, strides, 1, 16, 16,
                                    0.5, 1.0, dummy, dummy, None, dummy, dummy, dummy, 1 << 20,
                                    None)
    assert status == 1 and b"replay lists" in lib.gs_last_error()
    status = lib.gs_render_forward(*forward, dummy, 10, dummy, 64, dummy, dummy, 0, dummy,
                                   1 << 20, None)
    assert status == 2 and b"segment capacity" in lib.gs_last_error()
    assert (lib.gs_render_backward_workspace_size(1, 64, 64, 100)
            >= lib.gs_render_workspace_size(1, 64, 64) + 8 * (16 + 100))
    # Workspace smaller than required is rejected before any launch.
    need = lib.gs_scan_workspace_size(1000)
    dummy = ctypes.c_void_p(16)
    status = lib.gs_count_tiles(dummy, dummy, 1000, 16, 16, dummy, dummy, need - 1, None)
    assert status == 4 and b"workspace" in lib.gs_last_error()
    # Zero-sized work is a successful no-op.
    assert lib.gs_sort_pairs(None, None, None, None, 0, 0, 64, None, 0, None) == 0
    assert lib.gs_last_error() == b""


def test_static_forward_rejects_more_tiles_than_its_scratch():
    """gs_render_forward_static refuses more image tiles than its static
    scratch holds (GS_RENDER_STATIC_MAX_TILES) before any HIP call, so the
    placeholder pointers below are never dereferenced."""
    from diff_gabor_splatting_amd import _native

    lib = _native.lib
    static_max_tiles = 1 << 20
    side = 16 * 1025  # 1025 x 1025 tiles
    dummy = ctypes.c_void_p(256)
    groups = (ctypes.c_void_p * 5)(*([256] * 5))
    strides = (ctypes.c_int64 * 10)()
    status = lib.gs_render_forward_static(0, *([dummy] * 7), 1, side, side, 0.2, 100.0, groups,
                                          strides, dummy, dummy, None, 0, None, None)
    assert status == 4
    message = lib.gs_last_error().decode()
    assert f"at most {static_max_tiles} image tiles" in message and "1050625" in message


@pytest.mark.parametrize("m", [0, 1, 4096, 4097, 10**6])
def test_workspace_sizes_grow_with_input(m):
    from diff_gabor_splatting_amd import _native

    lib = _native.lib
    assert lib.gs_sort_workspace_size(m) >= 12 * m
    assert lib.gs_scan_workspace_size(m) >= 8 * ((m + 4095) // 4096)


def _declarations():
    """Parameter type lists of every gs_* prototype in include/*.h."""
    out = {}
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        for match in re.finditer(r"\b(gs_\w+)\s*\(([^)]*)\)\s*;", text):
            params = [p.strip() for p in match.group(2).split(",") if p.strip() not in ("", "void")]
            out[match.group(1)] = params
    return out


def _ctype_class(param):
    if "*" in param:
        return "pointer"
    kind = param.rsplit(" ", 1)[0].replace("const ", "").strip()
    return {"int32_t": "int32", "int": "int32", "int64_t": "int64", "size_t": "size",
            "float": "float", "double": "double"}[kind]


def test_ctypes_signatures_match_the_header():
    from diff_gabor_splatting_amd import _native

    classes = {ctypes.c_void_p: "pointer", ctypes.c_int32: "int32", ctypes.c_int64: "int64",
               ctypes.c_size_t: "size", ctypes.c_float: "float", ctypes.c_double: "double"}
    declared = _declarations()
    for name, (_, argtypes) in _native._SIGNATURES.items():
        params = declared[name]
        assert len(params) == len(argtypes), (name, len(params), len(argtypes))
        for index, (param, argtype) in enumerate(zip(params, argtypes)):
            expected = _ctype_class(param)
            actual = classes.get(argtype, "pointer")
            assert expected == actual, (name, index, param, argtype)


def test_split_policy():
    """Split tiles: a fixed 64-record segment below 2048 image tiles, slots
    enough for every tile longer than that (floor(M / 64) + min(tiles,
    floor(M / 65)) + 1) up to the cap, and an index buffer whose work list
    starts at an even offset."""
    from diff_gabor_splatting_amd import _native

    assert _native.split_length(16, 1000) == 64
    assert _native.split_length(2047, 10**7) == 64  # independent of the count
    assert _native.split_length(2048, 1000) == 0 and _native.split_length(16, 0) == 0
    assert _native.split_slots(89_449, 64, 1024) == 1_397 + 1_024 + 1
    assert _native.split_slots(89_449, 64, 4096) == 1_397 + 1_376 + 1
    assert _native.split_slots(10**8, 64, 1024) == _native.SPLIT_MAX_SLOTS
    assert _native.split_slots(1000, 0, 16) == 0
    # Brute force: every way of cutting M records into tiles (here, random
    # tile lengths) needs at most split_slots slots for its tiles longer
    # than 64 records.
    import random

    rng = random.Random(5)
    for _ in range(2000):
        tiles = rng.randint(1, 64)
        lengths = [rng.choice((0, 1, 63, 64, 65, 128, 129, rng.randint(0, 3000)))
                   for _ in range(tiles)]
        m = sum(lengths)
        need = sum(-(-n // 64) for n in lengths if n > 64)
        assert need <= _native.split_slots(m, 64, tiles) < _native.SPLIT_MAX_SLOTS
    assert _native.split_index_length(7, 10) == 18 + 34
    assert _native.split_index_length(8, 10) == 18 + 36


def test_host_extension_binds_exported_entry_points():
    """The C++ host functions call the library through addresses handed
    over at import; every name they need is an exported, declared symbol,
    and a table that lacks one is refused without unbinding the module."""
    from diff_gabor_splatting_amd import _host, _native

    names = _host.entry_points()
    assert set(names) <= set(_native.exported_symbols())
    with pytest.raises(RuntimeError, match="lacks gs_last_error"):
        _host.bind({})
    _native._bind_host(_native.lib)


def test_host_checks_raise_before_any_launch():
    """Structural checks of the C++ host functions run on the host: CPU
    tensors are refused with the reference's messages before anything is
    launched."""
    import torch

    from diff_gabor_splatting_amd import _native

    q = 3
    geometry = torch.zeros(q, 17)
    args = (geometry, torch.zeros(q, 18), torch.zeros(q), torch.zeros(q, dtype=torch.int64),
            torch.zeros(q, dtype=torch.int64), torch.zeros(q, dtype=torch.int32),
            torch.zeros(1, 3), 16, 16, False, 0.1, 10.0)
    with pytest.raises(RuntimeError, match="native rendering requires CUDA float32 tensors"):
        _native.rasterize_forward(*args)
    with pytest.raises(RuntimeError, match="native rendering requires CUDA float32 tensors"):
        _native.rasterize_backward(geometry, torch.zeros(q, 18), torch.zeros(q),
                                   torch.zeros(q, dtype=torch.int64), torch.zeros(1, 3),
                                   torch.zeros(0, dtype=torch.int32),
                                   torch.zeros(1, 2, dtype=torch.int32), torch.zeros(1, 16, 16, 3),
                                   torch.zeros(1, 16, 16, dtype=torch.int32),
                                   torch.zeros(1, 16, 16, 9), 16, 16, False, 0.1, 10.0)
    with pytest.raises(RuntimeError, match="too many tensors to check"):
        _native.check_values_word([geometry] * 17, *(torch.zeros(1),) * 5)


def test_block_path_limit():
    """gs_bin_blocks_fit (host arithmetic only): at most 65536 tile blocks of
    4 x 4 tiles (16-bit block ids); past that the synchronised binning keeps
    the tile sort."""
    from diff_gabor_splatting_amd import _native

    lib = _native.lib
    assert lib.gs_bin_blocks_fit(1, 1920, 1080) == 1       # 30 x 17 = 510 blocks
    assert lib.gs_bin_blocks_fit(128, 1920, 1080) == 1     # 65,280 blocks
    assert lib.gs_bin_blocks_fit(129, 1920, 1080) == 0     # 65,790 blocks
    assert lib.gs_bin_blocks_fit(1, 16 * 1024, 16 * 1024) == 1  # 256 x 256 blocks
    assert lib.gs_bin_blocks_fit(1, 16 * 1024 + 1, 16 * 1024) == 0
    assert lib.gs_bin_blocks_fit(1, 0, 16) == 0
