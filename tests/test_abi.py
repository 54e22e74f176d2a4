"""The C ABI library (no GPU needed): it loads, exports every function that
include/gsplat_hip.h declares, and its host-only entry points (version,
error plumbing, workspace sizes, argument validation) behave as declared.
No kernel is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gsplat_hip.h")
LIB = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gsplat_hip_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libgsplat_hip.so is not built (run __graft_entry__.build())")
    return ctypes.CDLL(LIB)


def test_header_declares_the_chain():
    names = declared_functions()
    for op in ("quat_scale_to_covar_preci_fwd", "quat_scale_to_covar_preci_bwd", "projection_fwd", "projection_bwd",
               "spherical_harmonics_fwd", "spherical_harmonics_bwd", "isect_count_scan", "isect_encode",
               "isect_sort", "isect_tile_sorted", "isect_offset", "rasterize_fwd", "rasterize_bwd"):
        assert "gsplat_hip_" + op in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_error_plumbing(lib):
    lib.gsplat_hip_abi_version.restype = ctypes.c_int
    assert lib.gsplat_hip_abi_version() >= 200  # the SH camera forward takes radii
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_isect_sort.restype = ctypes.c_int
    lib.gsplat_hip_isect_sort.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p]
    # invalid key width: rejected on the host before any device work
    rc = lib.gsplat_hip_isect_sort(None, None, 10, 65, None, None, None, 0, None)
    assert rc == 1
    assert b"invalid" in lib.gsplat_hip_last_error()
    # empty input: nothing to do
    assert lib.gsplat_hip_isect_sort(None, None, 0, 40, None, None, None, 0, None) == 0


def test_workspace_sizes(lib):
    for name, args in (("gsplat_hip_isect_sort_workspace_size", (ctypes.c_int64,)),
                       ("gsplat_hip_isect_count_scan_workspace_size", (ctypes.c_int64,)),
                       ("gsplat_hip_exclusive_scan_i32_workspace_size", (ctypes.c_int64,)),
                       ("gsplat_hip_isect_tile_sorted_workspace_size", (ctypes.c_int64, ctypes.c_int64)),
                       ("gsplat_hip_rasterize_bwd_workspace_size",
                        (ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32))):
        f = getattr(lib, name)
        f.restype = ctypes.c_size_t
        f.argtypes = list(args)
    assert lib.gsplat_hip_isect_sort_workspace_size(0) == 0
    small = lib.gsplat_hip_isect_sort_workspace_size(1000)
    big = lib.gsplat_hip_isect_sort_workspace_size(5_000_000)
    assert 0 < small < big
    # the alternate key + value buffers alone take 12 bytes per key
    assert big >= 12 * 5_000_000
    assert lib.gsplat_hip_isect_tile_sorted_workspace_size(1_000_000, 5_400_000) > 12 * 5_400_000
    assert lib.gsplat_hip_isect_tile_sorted_workspace_size(0, 10) == 0
    # cost + order per tile, one background partial per tile and channel
    assert lib.gsplat_hip_rasterize_bwd_workspace_size(1, 3, 82, 53) >= (2 + 3) * 4 * 82 * 53
    assert lib.gsplat_hip_rasterize_bwd_workspace_size(2, 64, 82, 53) >= 2 * (2 + 64) * 4 * 82 * 53
    assert lib.gsplat_hip_rasterize_bwd_workspace_size(0, 3, 82, 53) == 0
    assert lib.gsplat_hip_exclusive_scan_i32_workspace_size(1 << 20) > 0


def test_rasterize_rejects_bad_sizes(lib):
    f = lib.gsplat_hip_rasterize_fwd
    f.restype = ctypes.c_int
    i64, i32, p = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
    f.argtypes = [p, p, p, p, p, p, p, p, i64, i64, i32, i32, i32, i32, i32, i32, i64, p, p, p, p]
    # 65 channels exceed the supported maximum
    rc = f(None, None, None, None, None, None, None, None, 1, 10, 65, 16, 16, 16, 1, 1, 0, None, None, None, None)
    assert rc == 1
    # a tile grid that does not cover the image
    rc = f(None, None, None, None, None, None, None, None, 1, 10, 3, 64, 64, 16, 2, 2, 0, None, None, None, None)
    assert rc == 1


def test_image_loss_sizes_and_validation(lib):
    i64, p = ctypes.c_int64, ctypes.c_void_p
    lib.gsplat_hip_image_loss_map_size.restype = i64
    lib.gsplat_hip_image_loss_map_size.argtypes = [i64, i64, i64, i64, ctypes.c_int]
    lib.gsplat_hip_image_loss_workspace_size.restype = ctypes.c_size_t
    lib.gsplat_hip_image_loss_workspace_size.argtypes = [i64, i64, i64, i64, ctypes.c_int]
    # the conv2d map: H + 2 (ws // 2) - ws + 1 rows (one more for even windows)
    assert lib.gsplat_hip_image_loss_map_size(2, 840, 1297, 3, 11) == 2 * 840 * 1297 * 3
    assert lib.gsplat_hip_image_loss_map_size(1, 10, 20, 3, 8) == 11 * 21 * 3
    assert lib.gsplat_hip_image_loss_map_size(1, 10, 20, 3, 0) == -1
    # two float partials per block of 16 map rows x (256 - (ws - 1) C) map
    # values: ceil(840 / 16) x ceil(3891 / 226) blocks
    assert lib.gsplat_hip_image_loss_workspace_size(1, 840, 1297, 3, 11) == 2 * 4 * 53 * 18
    # (ws - 1) C > 128: row-segment blocks of 16 rows x 256 values
    assert lib.gsplat_hip_image_loss_workspace_size(1, 40, 30, 16, 11) == 2 * 4 * 3 * 2
    assert lib.gsplat_hip_image_loss_workspace_size(0, 840, 1297, 3, 11) == 0
    f = lib.gsplat_hip_image_loss_fwd
    f.restype = ctypes.c_int
    f.argtypes = [p, p, i64, i64, i64, i64, ctypes.c_int, p, p, p, ctypes.c_size_t, p]
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    # rejected on the host before any device work: window 0, a staged row
    # segment beyond 1024 values ((11 - 1) * 80 > 768)
    assert f(None, None, 1, 8, 8, 3, 0, None, None, None, 0, None) == 1
    assert f(None, None, 1, 8, 8, 80, 11, None, None, None, 0, None) == 1
    assert b"768" in lib.gsplat_hip_last_error()
