"""Shape contract and routing of the kernel API (CPU only).

The same truth tables the reference pins in its ``tests/test_dims.py``
(reference ``tests/test_dims.py:25-248``): which (D, G, DV) the single-tile
ops serve, which go to the blocked ops, which are refused and with what
message; the mode switches and their errors; the blocked tile-size function;
the tile-table switch. Nothing here needs a GPU.
"""

import pytest
import torch

from flashslice_amd.kernels import (set_dot_mode, set_kernel_mode, set_stats_mode,
                                    set_tile_table, single_tile_dims, stats_mode, tile_table,
                                    unsupported_dims)
from flashslice_amd.kernels import blocked as fb
from flashslice_amd.kernels import slice_ops as fs
from flashslice_amd.kernels.blocked import set_block_g, tiles
from flashslice_amd.kernels.slice_ops import _use_blocked


@pytest.mark.parametrize("d,g", [(16, 16), (32, 32), (32, 64), (32, 128), (128, 32)])
def test_single_tile_dims(d, g):
    assert unsupported_dims(d, g) is None
    assert single_tile_dims(d, g)
    assert not _use_blocked(d, g)


@pytest.mark.parametrize("d,g", [(32, 8), (32, 256), (32, 48), (8, 32), (256, 32), (24, 40),
                                 (32, 1), (32, 1024)])
def test_blocked_dims(d, g):
    assert unsupported_dims(d, g) is None
    assert not single_tile_dims(d, g)
    assert _use_blocked(d, g)


@pytest.mark.parametrize("d,g", [(512, 32), (0, 32), (32, 0)])
def test_unsupported_dims(d, g):
    why = unsupported_dims(d, g)
    assert why and ("dim_head" in why or "slice_num" in why)


def test_kernel_mode_switch():
    try:
        set_kernel_mode("blocked")
        assert _use_blocked(32, 32)
        set_kernel_mode("single-tile")
        assert not _use_blocked(32, 32)
        with pytest.raises(ValueError, match="single-tile"):
            _use_blocked(32, 256)
        with pytest.raises(ValueError):
            set_kernel_mode("fast")
    finally:
        set_kernel_mode("auto")
    assert not _use_blocked(32, 32) and _use_blocked(32, 256)


@pytest.mark.parametrize("d,g,dt,gb", [(32, 256, 32, 64), (32, 48, 32, 64), (32, 8, 32, 16),
                                       (24, 40, 32, 64), (64, 256, 64, 32), (256, 32, 256, 16)])
def test_blocked_tiles(d, g, dt, gb):
    assert tiles(d, g) == (dt, gb)


@pytest.mark.parametrize("d,g,dot,gb", [(56, 1024, 3, 64), (56, 1024, 0, 32), (56, 1024, 4, 64),
                                        (128, 256, 3, 32), (32, 256, 3, 64)])
def test_blocked_tiles_by_dot(d, g, dot, gb):
    assert tiles(d, g, dot)[1] == gb


def test_set_block_g():
    try:
        set_block_g(32)
        assert tiles(32, 256) == (32, 32)
        for bad in (8, 48, 0):
            with pytest.raises(ValueError):
                set_block_g(bad)
    finally:
        set_block_g(None)
    assert tiles(32, 256) == (32, 64)


@pytest.mark.parametrize("d,g,dv", [(32, 32, 24), (56, 1024, 32), (64, 64, 32)])
def test_value_width_routes_to_blocked(d, g, dv):
    assert unsupported_dims(d, g, dv) is None
    assert not single_tile_dims(d, g, dv)
    assert _use_blocked(d, g, dv)


def test_equal_value_width_keeps_single_tile():
    assert single_tile_dims(32, 32, 32)
    assert not _use_blocked(32, 32, 32)


def test_value_width_bounds():
    assert "value width" in unsupported_dims(32, 32, 512)
    assert "value width" in unsupported_dims(32, 32, 0)


def test_stats_mode_switch():
    assert stats_mode() in ("online", "two-pass")
    try:
        set_stats_mode("two-pass")
        assert stats_mode() == "two-pass"
        with pytest.raises(ValueError):
            set_stats_mode("streaming")
    finally:
        set_stats_mode("online")
    assert stats_mode() == "online"


def test_tile_table_selection():
    try:
        set_tile_table("ada")
        assert tile_table() == "ada"
        set_tile_table("hopper")
        assert tile_table() == "hopper"
        with pytest.raises(ValueError):
            set_tile_table("ampere")
    finally:
        set_tile_table("auto")
    assert tile_table() == "cdna4"


def test_dot_modes():
    x32 = torch.empty(1, 1, 1, 1)
    x16 = torch.empty(1, 1, 1, 1, dtype=torch.bfloat16)
    try:
        for mode, lvl32, lvl16 in (("ieee", 0, 0), ("tf32", 1, 1), ("bf16v", 1, 2),
                                   ("bf16", 1, 3), ("tf32x3", 4, 4), ("", 0, 0)):
            set_dot_mode(mode)
            assert fs._dot_mode(x32) == lvl32 and fs._dot_mode(x16) == lvl16
        with pytest.raises(ValueError):
            set_dot_mode("fp8")
    finally:
        set_dot_mode("")


def test_prep_wb_layouts_and_errors():
    x = torch.empty(2, 5, 3, 8)
    for wshape, bshape in (((4, 8), (4,)), ((3, 4, 8), (3, 4)), ((2, 3, 4, 8), (2, 3, 4)),
                           ((1, 3, 4, 8), (1, 4))):
        w, b, G = fs._prep_wb(x, torch.empty(wshape), torch.empty(bshape))
        assert G == 4
    w, b, G = fs._prep_wb(x, torch.empty(4, 8), None)
    assert b.shape == (4,) and torch.equal(b, torch.zeros(4))
    with pytest.raises(ValueError, match="last dim"):
        fs._prep_wb(x, torch.empty(4, 7), None)
    with pytest.raises(ValueError, match="weight must be"):
        fs._prep_wb(x, torch.empty(8), None)
    with pytest.raises(ValueError, match="bias must be"):
        fs._prep_wb(x, torch.empty(4, 8), torch.empty(5))
    with pytest.raises(ValueError, match="along heads"):
        fs._prep_wb(x, torch.empty(2, 4, 8), None)
    with pytest.raises(ValueError, match="along batch"):
        fs._prep_wb(x, torch.empty(3, 3, 4, 8), None)


def test_wb_layout_strides():
    # zero strides where shared; reference slice_ops.py:461-478
    assert fs._wb_layout(torch.empty(4, 8), torch.empty(4), 2, 3) == (0, 0, 0, 0)
    assert fs._wb_layout(torch.empty(3, 4, 8), torch.empty(3, 4), 2, 3) == (0, 32, 0, 4)
    assert fs._wb_layout(torch.empty(2, 3, 4, 8), torch.empty(2, 3, 4), 2, 3) == (96, 32, 12, 4)
    with pytest.raises(ValueError, match="bias has 5 slices"):
        fs._wb_layout(torch.empty(4, 8), torch.empty(5), 2, 3)


def test_public_api_names():
    import flashslice_amd.kernels as K
    assert set(K.__all__) == {"fused_slice", "fused_deslice", "unsupported_dims",
                              "single_tile_dims", "set_dot_mode", "set_kernel_mode",
                              "set_block_g", "set_stats_mode", "stats_mode", "set_tile_table",
                              "tile_table", "fused_deslice_slice", "fused_coupling", "fused_slice_varlen",
                              "fused_deslice_varlen"}
    assert set(fb.__all__) == {"tiles", "set_block_g", "compute_stats", "set_stats_mode",
                               "stats_mode"}
