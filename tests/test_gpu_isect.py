"""GPU parity for tile intersection: counts, offsets, keys, sorted order and
tile offsets must be bit-exact with the oracle (gsplat_core/test/test.cpp:
653-1065 known answers; random scenes with many equal keys). Also calls the
C ABI directly (ctypes) for the sort and offsets, and checks size-independent
properties at a large size."""
import ctypes
import os

import numpy as np
import pytest

from _helpers import dev, gsplat, host

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")


def _key(tile, bits):
    return (tile << 32) | bits


def test_known_answers():
    g = gsplat()
    m = np.array([[[20, 20], [50, 50], [8, 8]]], np.float32)
    r = np.array([[[10, 10], [5, 5], [0, 0]]], np.int32)
    d = np.array([[1.0, 0.5, 2.0]], np.float32)
    out = g.intersect_tile_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(d)}, 1, 16, 4, 4)
    assert host(out["tiles_per_gauss"]).tolist() == [[4, 4, 0]]
    ids = host(out["isect_ids"])
    assert ((ids >> 32) & 0x1F).tolist() == [0, 1, 4, 5, 10, 11, 14, 15]
    assert host(out["flatten_ids"]).tolist() == [0, 0, 0, 0, 1, 1, 1, 1]
    offs = host(g.intersect_offset_forward(out["isect_ids"], 1, 4, 4))
    assert offs.ravel().tolist() == [0, 1, 2, 2, 2, 3, 4, 4, 4, 4, 4, 5, 6, 6, 6, 7]
    # swapped order: sort reorders (test.cpp:857-954)
    m2 = np.array([[[50, 50], [20, 20], [8, 8]]], np.float32)
    r2 = np.array([[[5, 5], [10, 10], [0, 0]]], np.int32)
    d2 = np.array([[0.5, 1.0, 2.0]], np.float32)
    uns = g.intersect_tile_forward({"means2d": dev(m2), "radii": dev(r2), "depths": dev(d2)}, 1, 16, 4, 4, sort=False)
    assert host(uns["isect_ids"]).tolist() == ([_key(t, 0x3F000000) for t in (10, 11, 14, 15)] +
                                               [_key(t, 0x3F800000) for t in (0, 1, 4, 5)])
    srt = g.intersect_tile_forward({"means2d": dev(m2), "radii": dev(r2), "depths": dev(d2)}, 1, 16, 4, 4)
    assert host(srt["isect_ids"]).tolist() == ([_key(t, 0x3F800000) for t in (0, 1, 4, 5)] +
                                               [_key(t, 0x3F000000) for t in (10, 11, 14, 15)])
    assert host(srt["flatten_ids"]).tolist() == [1, 1, 1, 1, 0, 0, 0, 0]


def random_projected(rng, I, N, W, H, ties, signed=False):
    means2d = np.stack([rng.uniform(-30, W + 30, (I, N)), rng.uniform(-30, H + 30, (I, N))], -1).astype(np.float32)
    radii = rng.integers(0, 60, size=(I, N, 2)).astype(np.int32)
    radii[rng.random((I, N)) < 0.2] = 0
    depths = rng.uniform(0.1, 50, (I, N)).astype(np.float32)
    if ties:
        depths = np.round(depths * 2).astype(np.float32) / 2
    if signed:
        # negative, -0.0 and +0.0 depths: the key holds the raw float bits, so
        # negative depths sort after every positive one
        pick = rng.random((I, N))
        depths[pick < 0.1] *= -1
        depths[(pick >= 0.1) & (pick < 0.15)] = -0.0
        depths[(pick >= 0.15) & (pick < 0.2)] = 0.0
    return means2d, radii, depths


@pytest.mark.parametrize("I,N,W,H,ts,ties,signed", [(1, 20000, 640, 480, 16, False, False),
                                                    (3, 7000, 300, 200, 16, True, False),
                                                    (2, 5000, 130, 70, 8, True, False),
                                                    (1, 3000, 1297, 840, 16, True, False),
                                                    (2, 4000, 200, 150, 16, True, True)])
def test_random_bit_exact(oracle, I, N, W, H, ts, ties, signed):
    g = gsplat()
    rng = np.random.default_rng(I * 100 + N)
    m, r, d = random_projected(rng, I, N, W, H, ties, signed)
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    got = g.intersect_tile_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(d)}, I, ts, tw, th)
    exp = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
    np.testing.assert_array_equal(host(got["tiles_per_gauss"]), exp["tiles_per_gauss"])
    np.testing.assert_array_equal(host(got["isect_ids"]), exp["isect_ids"])
    np.testing.assert_array_equal(host(got["flatten_ids"]), exp["flatten_ids"])
    np.testing.assert_array_equal(host(g.intersect_offset_forward(got["isect_ids"], I, tw, th)),
                                  oracle.isect_offset(exp["isect_ids"], I, tw, th))
    # unsorted encode order and the standalone scan
    uns = g.intersect_tile_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(d)}, I, ts, tw, th, sort=False)
    counts = oracle.isect_count(m, r, ts, tw, th)
    offs, total = oracle.exclusive_scan(counts)
    ek, ef = oracle.isect_encode(m, r, d, offs, I, ts, tw, th, total)
    np.testing.assert_array_equal(host(uns["isect_ids"]), ek)
    np.testing.assert_array_equal(host(uns["flatten_ids"]), ef)


def test_empty_and_all_culled():
    g = gsplat()
    m = np.zeros((1, 50, 2), np.float32)
    r = np.zeros((1, 50, 2), np.int32)
    d = np.ones((1, 50), np.float32)
    out = g.intersect_tile_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(d)}, 1, 16, 3, 2)
    assert out["isect_ids"].numel() == 0 and out["flatten_ids"].numel() == 0
    assert host(g.intersect_offset_forward(out["isect_ids"], 1, 3, 2)).ravel().tolist() == [0] * 6


def _c_sort(keys_t, vals_t, key_bits):
    import torch

    lib = ctypes.CDLL(LIB)
    lib.gsplat_hip_isect_sort_workspace_size.restype = ctypes.c_size_t
    lib.gsplat_hip_isect_sort_workspace_size.argtypes = [ctypes.c_int64]
    lib.gsplat_hip_isect_sort.restype = ctypes.c_int
    lib.gsplat_hip_isect_sort.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p]
    n = keys_t.numel()
    ws_bytes = lib.gsplat_hip_isect_sort_workspace_size(n)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=keys_t.device)
    ko = torch.empty_like(keys_t)
    vo = torch.empty_like(vals_t)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.gsplat_hip_isect_sort(keys_t.data_ptr(), vals_t.data_ptr(), n, key_bits, ko.data_ptr(), vo.data_ptr(),
                                   ws.data_ptr(), ws_bytes, stream)
    assert rc == 0
    torch.cuda.synchronize()
    return ko, vo


@pytest.mark.parametrize("n,bits", [(1, 40), (4095, 20), (4097, 33), (100003, 45), (262144, 64)])
def test_c_abi_sort_stable(n, bits):
    import torch

    rng = np.random.default_rng(n)
    hi = (1 << bits) if bits < 63 else (1 << 62)
    keys = rng.integers(0, min(hi, 1 << 62), size=n, dtype=np.int64)
    keys[rng.random(n) < 0.3] = keys[0]  # many duplicates
    vals = np.arange(n, dtype=np.int32)
    ko, vo = _c_sort(dev(keys), dev(vals), bits)
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(host(ko), keys[order])
    np.testing.assert_array_equal(host(vo), vals[order])
    del torch


def test_large_properties():
    """Size-independent checks at ~5M intersections: keys non-decreasing,
    each flatten id appears tiles_per_gauss times, offsets = lower bound."""
    g = gsplat()
    import torch

    rng = np.random.default_rng(11)
    I, N, W, H, ts = 1, 600_000, 1297, 840, 16
    m, r, d = random_projected(rng, I, N, W, H, ties=True)
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    out = g.intersect_tile_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(d)}, I, ts, tw, th)
    keys = out["isect_ids"]
    assert keys.numel() > 3_000_000
    assert bool(torch.all(keys[1:] >= keys[:-1]))
    counts = torch.bincount(out["flatten_ids"].long(), minlength=I * N)
    assert torch.equal(counts.to(torch.int32), out["tiles_per_gauss"].reshape(-1))
    offs = g.intersect_offset_forward(keys, I, tw, th).reshape(-1).long()
    want = torch.arange(tw * th, device=keys.device, dtype=torch.int64)
    lb = torch.searchsorted(keys >> 32, want, right=False)
    assert torch.equal(offs, lb)


def test_c_abi_tile_sorted_one_call(oracle):
    """gsplat_hip_isect_tile_sorted (both steps in one call, shared
    workspace) gives the oracle's sorted keys and ids."""
    import torch

    rng = np.random.default_rng(11)
    I, N, W, H, ts = 2, 6000, 300, 200, 16
    m, r, d = random_projected(rng, I, N, W, H, True, True)
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    exp = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
    counts = oracle.isect_count(m, r, ts, tw, th).astype(np.int32)
    n_isects = int(counts.sum())
    lib = ctypes.CDLL(LIB)
    p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.gsplat_hip_isect_tile_sorted_workspace_size.restype = ctypes.c_size_t
    lib.gsplat_hip_isect_tile_sorted_workspace_size.argtypes = [i64, i64]
    lib.gsplat_hip_isect_tile_sorted.restype = ctypes.c_int
    lib.gsplat_hip_isect_tile_sorted.argtypes = [p, p, p, p, i64, i64, i32, i32, i32, i64, p, p, p, ctypes.c_size_t, p]
    ws_bytes = lib.gsplat_hip_isect_tile_sorted_workspace_size(I * N, n_isects)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    md, rd, dd, cd = dev(m), dev(r), dev(d), dev(counts)
    ids = torch.empty(n_isects, dtype=torch.int64, device="cuda")
    flat = torch.empty(n_isects, dtype=torch.int32, device="cuda")
    rc = lib.gsplat_hip_isect_tile_sorted(md.data_ptr(), rd.data_ptr(), dd.data_ptr(), cd.data_ptr(), I, I * N, ts,
                                          tw, th, n_isects, ids.data_ptr(), flat.data_ptr(), ws.data_ptr(), ws_bytes,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(ids), exp["isect_ids"])
    np.testing.assert_array_equal(host(flat), exp["flatten_ids"])


@pytest.mark.parametrize("n", [1, 1023, 4097, 16383, 16384, 16385, 65536, 65537, 1 << 20])
def test_c_abi_exclusive_scan(n):
    """gsplat_hip_exclusive_scan_i32 against numpy, in place, on both sides of
    the single-block / three-kernel switch (16384 values)."""
    import torch

    lib = ctypes.CDLL(LIB)
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_exclusive_scan_i32_workspace_size.restype = ctypes.c_size_t
    lib.gsplat_hip_exclusive_scan_i32_workspace_size.argtypes = [ctypes.c_int64]
    lib.gsplat_hip_exclusive_scan_i32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    v = np.random.default_rng(n).integers(0, 100, n).astype(np.int32)
    x = torch.from_numpy(v).cuda()
    total = torch.zeros(1, dtype=torch.int64, device="cuda")
    ws = torch.empty(max(lib.gsplat_hip_exclusive_scan_i32_workspace_size(n), 1), dtype=torch.uint8, device="cuda")
    rc = lib.gsplat_hip_exclusive_scan_i32(x.data_ptr(), x.data_ptr(), n, total.data_ptr(), ws.data_ptr(),
                                           ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    expect = np.concatenate([[0], np.cumsum(v.astype(np.int64))[:-1]])
    np.testing.assert_array_equal(host(x), expect)
    assert int(total.item()) == int(v.astype(np.int64).sum())
