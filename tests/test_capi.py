"""The C ABI on the CPU: the library loads, exports what include/moe355.h
declares, plans are consistent, and bad arguments are rejected before any
GPU work (no compute runs here)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from reframework_amd import _capi


def test_library_exports_every_declared_symbol():
    lib = _capi.lib()
    declared = _capi.header_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_capi._SIGNATURES)


def test_version_and_constants():
    assert _capi.version() == 101
    text = open(_capi.HEADER_PATH).read()
    assert "#define MOE355_MAX_EXPERTS 256" in text
    assert ctypes.sizeof(_capi.Plan) == 12 * 4 + 9 * 8


@pytest.mark.parametrize("T,H,I,E,K,dtype,path", [
    (4096, 4096, 14336, 8, 2, _capi.BF16, _capi.PATH_MFMA_TILED),
    (512, 4096, 14336, 8, 2, _capi.BF16, _capi.PATH_MFMA_TILED),
    (256, 4096, 14336, 8, 2, _capi.BF16, _capi.PATH_MFMA_TILED128),
    (128, 4096, 14336, 8, 2, _capi.BF16, _capi.PATH_MFMA_TILED128),
    (16, 4096, 14336, 8, 2, _capi.BF16, _capi.PATH_MFMA_SKINNY),
    (1, 4096, 14336, 8, 2, _capi.BF16, _capi.PATH_MFMA_SKINNY),
    (2048, 4096, 6400, 16, 2, _capi.BF16, _capi.PATH_MFMA_TILED),
    (8, 2048, 1408, 64, 6, _capi.BF16, _capi.PATH_MFMA_SKINNY),
    (4096, 2048, 1408, 64, 6, _capi.BF16, _capi.PATH_MFMA_TILED),
    (512, 1024, 2816, 8, 2, _capi.F32, _capi.PATH_SIMT),
    (128, 1024, 2816, 8, 2, _capi.F16, _capi.PATH_MFMA_TILED128),
    (512, 1024, 2816, 8, 2, _capi.F16, _capi.PATH_MFMA_TILED),
])
def test_plan_paths_and_layout(T, H, I, E, K, dtype, path):
    p = _capi.make_plan(T, H, I, E, K, dtype)
    assert p.path == path and p.rows == T * K
    offs = [p.off_block_counts, p.off_offsets, p.off_slot_to_row, p.off_row_src, p.off_tile_map,
            p.off_inter, p.off_y, p.off_part, p.workspace_bytes]
    assert all(o % 256 == 0 for o in offs) and offs == sorted(offs)
    esz = 4 if dtype == _capi.F32 else 2
    assert p.off_y - p.off_inter >= T * K * I * esz
    assert p.off_part - p.off_y >= p.down_splits * T * K * H * 4
    if p.path in (_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128):
        # one 256x256 fp32 partial tile per CU (256 without a GPU) for the tail splits
        assert p.workspace_bytes - p.off_part >= 256 * 256 * 256 * 4
    else:
        assert p.workspace_bytes == p.off_part
    assert p.off_tile_map - p.off_row_src >= 4 * T * K
    if p.path == _capi.PATH_MFMA_SKINNY:
        assert (I // 128) % p.down_splits == 0


def test_tiled_path_keeps_token_offsets_below_2gb():
    # token-row byte offsets are 32-bit with bit 31 marking padding rows
    assert _capi.make_plan(262143, 4096, 14336, 8, 2, _capi.BF16).path == _capi.PATH_MFMA_TILED
    assert _capi.make_plan(262144, 4096, 14336, 8, 2, _capi.BF16).path != _capi.PATH_MFMA_TILED
    plan = _capi.Plan()
    assert _capi.lib().moe355_make_plan_path(262144, 4096, 14336, 8, 2, _capi.BF16,
                                             _capi.PATH_MFMA_TILED, ctypes.byref(plan)) == -2


@pytest.mark.parametrize("T,K,E,tile,path", [(4096, 2, 8, 256, -1), (16, 2, 8, 16, -1),
                                             (8, 6, 64, 16, -1), (333, 3, 7, 64, -1),
                                             (128, 2, 8, 128, -1), (777, 2, 5, 128, 4)])
def test_tile_map_capacity_bounds_every_routing(T, K, E, tile, path):
    dtype = _capi.F32 if (tile == 64 and path < 0 and T == 333) else _capi.BF16
    H, I = (256, 256) if tile != 16 else (256, 128)
    p = _capi.make_plan(T, H, I, E, K, dtype, path)
    assert p.tile_rows == tile
    rng = np.random.default_rng(0)
    R = T * K
    for _ in range(200):
        # random split of R rows over E experts, including extreme ones
        cuts = np.sort(rng.integers(0, R + 1, size=E - 1))
        m = np.diff(np.concatenate([[0], cuts, [R]]))
        assert int(np.sum(-(-m // tile))) <= p.max_tiles
    m = np.full(E, R // E)
    m[: R % E] += 1
    assert int(np.sum(-(-m // tile))) <= p.max_tiles


@pytest.mark.parametrize("args,code,msg", [
    ((4, 64, 64, 8, 9, _capi.BF16), -1, "top-k"),
    ((4, 64, 64, 300, 2, _capi.BF16), -2, "E=300"),
    ((4, 60, 64, 8, 2, _capi.BF16), -2, "multiples"),
    ((4, 64, 64, 8, 2, 7), -1, "dtype"),
    ((-1, 64, 64, 8, 2, _capi.BF16), -1, "bad sizes"),
])
def test_plan_rejects_bad_shapes(args, code, msg):
    plan = _capi.Plan()
    rc = _capi.lib().moe355_make_plan(*args, ctypes.byref(plan))
    assert rc == code
    assert msg in _capi.lib().moe355_last_error().decode()


def test_entry_points_reject_null_arguments_without_launching():
    lib = _capi.lib()
    rc = lib.moe355_router_topk(None, None, None, 2, 64, 8, 2, _capi.BF16, 1, 0, 0, None, None,
                                None, None)
    assert rc == -1 and "NULL" in lib.moe355_last_error().decode()
    rc = lib.moe355_topk_from_logits(None, 3, 8, 2, 1, None, None, None)
    assert rc == -1
    rc = lib.moe355_router_topk_ld(None, None, None, 2, 64, 8, 2, _capi.BF16, 1, 0, 0, None, None,
                                   None, 1, None)
    assert rc == -1 and "stride" in lib.moe355_last_error().decode()
    p = _capi.make_plan(4, 256, 256, 8, 2, _capi.BF16)
    assert lib.moe355_permute(ctypes.byref(p), None, 0, None, 0, None, None) == -1
    assert lib.moe355_gate_up(ctypes.byref(p), None, None, 0, None, None) == -1
    assert lib.moe355_gate_up(ctypes.byref(p), None, None, 9, None, None) == -1
    assert "activation" in lib.moe355_last_error().decode()
    assert lib.moe355_h2d_async(None, None, 0, None) == 0
    assert lib.moe355_h2d_async(None, None, 16, None) == -1
    bad = _capi.Plan()
    assert lib.moe355_down(ctypes.byref(bad), None, None, None) == -1
    assert "moe355_make_plan" in lib.moe355_last_error().decode()
    assert lib.moe355_fused_experts(None, None, None, None, None, 0, None, 0, 4, 256, 256, 8, 2,
                                    _capi.BF16, 0, None, 0, None, 0, None) == -3


def test_staging_entry_points_reject_bad_arguments_before_any_hip_call():
    lib = _capi.lib()
    assert lib.moe355_copy_to_host(None, None, 0, None) == 0
    assert lib.moe355_copy_to_host(None, None, 64, None) == -1
    assert lib.moe355_copy_to_host(0x1008, 0x2000, 64, None) == -1  # host_dst not 16-byte aligned
    assert "aligned" in lib.moe355_last_error().decode()
    assert lib.moe355_merge_host_f32(0x1000, 0x2000, 6, _capi.BF16, 0x3000, None) == -1
    assert "multiple of 4" in lib.moe355_last_error().decode()
    assert lib.moe355_merge_host_f32(0x1000, 0x2000, 8, 7, 0x3000, None) == -1
    assert lib.moe355_host_staging_alloc(16, None) == -1
    assert lib.moe355_host_staging_free(None) == 0
    # the multi-region copy: region count, NULL arrays, alignment, all before any HIP call
    srcs = (ctypes.c_void_p * 5)(0x2000, 0x3000, 0x4000, 0x5000, 0x6000)
    offs = (ctypes.c_size_t * 5)(0, 16, 32, 48, 64)
    sizes = (ctypes.c_size_t * 5)(16, 16, 16, 16, 16)
    assert lib.moe355_copy_to_host_multi(0x1000, 0, srcs, offs, sizes, None) == 0
    assert lib.moe355_copy_to_host_multi(0x1000, 5, srcs, offs, sizes, None) == -1
    assert "regions" in lib.moe355_last_error().decode()
    assert lib.moe355_copy_to_host_multi(None, 2, srcs, offs, sizes, None) == -1
    assert lib.moe355_copy_to_host_multi(0x1000, 2, None, offs, sizes, None) == -1


def test_zero_tokens_is_a_no_op():
    lib = _capi.lib()
    assert lib.moe355_router_topk(None, None, None, 0, 64, 8, 2, _capi.BF16, 1, 0, 0, None, None,
                                  None, None) == 0
    assert lib.moe355_fused_experts(None, None, None, None, None, 0, None, 0, 0, 256, 256, 8, 2,
                                    _capi.BF16, 0, None, 0, None, 0, None) == 0


@pytest.mark.parametrize("path,tile", [(_capi.PATH_MFMA_TILED, 256), (_capi.PATH_MFMA_TILED128, 128),
                                       (_capi.PATH_MFMA_SKINNY, 16),
                                       (_capi.PATH_SIMT, 64)])
def test_forced_path_plans(path, tile):
    p = _capi.make_plan(300, 512, 384, 8, 2, _capi.BF16, path)
    assert p.path == path and p.tile_rows == tile
    assert p.max_tiles >= -(-600 // tile)
    if path in (_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128):
        assert (384 // 32) % p.down_splits == 0


def test_forced_path_rejects_shapes_it_cannot_run():
    lib = _capi.lib()
    plan = _capi.Plan()
    # fp32 has no MFMA family; H=384 is not a multiple of the 256-row weight tile
    assert lib.moe355_make_plan_path(4, 256, 256, 8, 2, _capi.F32, _capi.PATH_MFMA_TILED,
                                     ctypes.byref(plan)) == -2
    assert lib.moe355_make_plan_path(4, 384, 256, 8, 2, _capi.BF16, _capi.PATH_MFMA_TILED,
                                     ctypes.byref(plan)) == -2
    assert lib.moe355_make_plan_path(4, 384, 256, 8, 2, _capi.BF16, _capi.PATH_MFMA_TILED128,
                                     ctypes.byref(plan)) == -2
    assert lib.moe355_make_plan_path(4, 256, 256, 8, 2, _capi.BF16, 7, ctypes.byref(plan)) == -1
    # 3 was a removed family's number
    assert lib.moe355_make_plan_path(4, 256, 256, 8, 2, _capi.BF16, 3, ctypes.byref(plan)) == -1
    assert "unknown path" in lib.moe355_last_error().decode()


def test_activation_codes():
    assert _capi.act_code("silu") == 0 and _capi.act_code("gelu_tanh") == 2
    with pytest.raises(ValueError, match="unknown gated activation"):
        _capi.act_code("relu")
