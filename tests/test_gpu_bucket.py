"""The tile-bucketed intersection (gsplat_hip_isect_bucket_count / _sort)
against the oracle, bit for bit: tiles_per_gauss, the sorted isect_ids and
flatten_ids, the tile offsets, the count M and the longest tile list. Scenes
cover several images, 8x8 tiles, depth ties (the tile sort's (depth, id)
re-sort), negative and signed-zero depths, empty input, every capacity of
the per-tile LDS sort (lists up to 2560, 4096, 8192 and 16384 entries, one
class at a time and all in one call), and lists longer than 16384 (split by
their leading depth bits into LDS-sorted runs, or sorted in global memory
when one digit is too crowded) beside short ones in one frame."""
import ctypes
import os

import numpy as np
import pytest

from _helpers import dev, gsplat, host

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")
P, I64, I32, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_isect_bucket_supported.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_supported.argtypes = [I64, I32, I32]
    lib.gsplat_hip_isect_bucket_max_list.restype = I64
    lib.gsplat_hip_isect_bucket_count_workspace_size.restype = SZ
    lib.gsplat_hip_isect_bucket_count_workspace_size.argtypes = [I64, I64, I32, I32, I32]
    lib.gsplat_hip_isect_bucket_count.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_count.argtypes = [P, P, I64, I64, I32, I32, I32, P, P, P, SZ, P]
    lib.gsplat_hip_isect_bucket_sort_workspace_size.restype = SZ
    lib.gsplat_hip_isect_bucket_sort_workspace_size.argtypes = [I64]
    lib.gsplat_hip_isect_bucket_sort.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_sort.argtypes = [P, P, P, I64, I64, I32, I32, I32, I64, I64, P, P, P, P, SZ, P, SZ, P]
    return lib


def bucket(lib, m, r, d, I, ts, tw, th):
    """count, read back (M, longest), sort: as the C++ layer does."""
    import torch

    numel = d.size
    md, rd, dd = dev(m), dev(r), dev(d)
    stream = torch.cuda.current_stream().cuda_stream
    tpg = torch.empty(numel, dtype=torch.int32, device="cuda")
    totals = torch.zeros(2, dtype=torch.int64, device="cuda")
    ws1b = lib.gsplat_hip_isect_bucket_count_workspace_size(I, numel, ts, tw, th)
    ws1 = torch.empty(max(ws1b, 1), dtype=torch.uint8, device="cuda")
    rc = lib.gsplat_hip_isect_bucket_count(md.data_ptr(), rd.data_ptr(), I, numel, ts, tw, th, tpg.data_ptr(),
                                           totals.data_ptr(), ws1.data_ptr(), ws1b, stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    M, longest = (int(v) for v in totals.cpu())
    ids = torch.empty(M, dtype=torch.int64, device="cuda")
    flat = torch.empty(M, dtype=torch.int32, device="cuda")
    offs = torch.empty(I * th * tw, dtype=torch.int32, device="cuda")
    ws2b = lib.gsplat_hip_isect_bucket_sort_workspace_size(M)
    ws2 = torch.empty(max(ws2b, 1), dtype=torch.uint8, device="cuda")
    rc = lib.gsplat_hip_isect_bucket_sort(md.data_ptr(), rd.data_ptr(), dd.data_ptr(), I, numel, ts, tw, th, M,
                                          longest, ids.data_ptr(), flat.data_ptr(), offs.data_ptr(), ws1.data_ptr(),
                                          ws1b, ws2.data_ptr(), ws2b, stream)
    torch.cuda.synchronize()
    return rc, M, longest, host(tpg), host(ids), host(flat), host(offs).reshape(I, th, tw)


def _check(oracle, lib, m, r, d, I, ts, tw, th):
    exp = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
    eoffs = oracle.isect_offset(exp["isect_ids"], I, tw, th)
    rc, M, longest, tpg, ids, flat, offs = bucket(lib, m, r, d, I, ts, tw, th)
    assert rc == 0, lib.gsplat_hip_last_error()
    assert M == exp["isect_ids"].size
    lens = np.diff(np.append(eoffs.ravel(), M))
    assert longest == (lens.max() if lens.size else 0)
    np.testing.assert_array_equal(tpg, exp["tiles_per_gauss"].ravel())
    np.testing.assert_array_equal(ids, exp["isect_ids"])
    np.testing.assert_array_equal(flat, exp["flatten_ids"])
    np.testing.assert_array_equal(offs, eoffs)
    return M, longest


@pytest.mark.parametrize("I,N,W,H,ts,ties,signed", [(1, 20000, 640, 480, 16, False, False),
                                                    (3, 7000, 300, 200, 16, True, False),
                                                    (2, 5000, 130, 70, 8, True, False),
                                                    (1, 3000, 1297, 840, 16, True, False),
                                                    (2, 4000, 200, 150, 16, True, True),
                                                    (1, 9000, 64, 48, 16, False, False)])
def test_bucket_bit_exact(oracle, I, N, W, H, ts, ties, signed):
    from test_gpu_isect import random_projected

    lib = _lib()
    rng = np.random.default_rng(I * 1000 + N)
    m, r, d = random_projected(rng, I, N, W, H, ties, signed)
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    print(f"bucket I={I} N={N} {W}x{H} ts={ts} ties={ties} signed={signed}", flush=True)
    _check(oracle, lib, m, r, d, I, ts, tw, th)


@pytest.mark.parametrize("crowd", [2000, 3500, 6000, 12000])
def test_bucket_every_tile_sort_capacity(oracle, crowd):
    """`crowd` Gaussians cover tile (2, 1) (and their neighbours), so the
    longest list selects each LDS capacity of the tile sort in turn; a third
    of them share depths (the id re-sort)."""
    from test_gpu_isect import random_projected

    lib = _lib()
    rng = np.random.default_rng(crowd)
    W, H, ts = 256, 160, 16
    tw, th = W // ts, H // ts
    m, r, d = random_projected(rng, 1, 6000, W, H, ties=False)
    cm = np.stack([rng.uniform(36, 44, crowd), rng.uniform(20, 28, crowd)], -1).astype(np.float32)[None]
    cr = rng.integers(1, 12, (1, crowd, 2)).astype(np.int32)
    cd = rng.uniform(0.5, 20, (1, crowd)).astype(np.float32)
    cd[:, : crowd // 3] = np.round(cd[:, : crowd // 3])
    m, r, d = np.concatenate([m, cm], 1), np.concatenate([r, cr], 1), np.concatenate([d, cd], 1)
    print(f"bucket crowd={crowd}", flush=True)
    M, longest = _check(oracle, lib, m, r, d, 1, ts, tw, th)
    assert crowd <= longest <= lib.gsplat_hip_isect_bucket_max_list()


def test_bucket_all_sort_classes_in_one_call(oracle):
    """Crowds of 2000, 3500, 6000 and 12000 Gaussians on four different
    tiles of two images: lists of every tile-sort class (up to 2560, 4096,
    8192 and 16384 entries) in one intersection, so the short-list launch
    and the three class launches all run; a third of each crowd shares
    depths."""
    from test_gpu_isect import random_projected

    lib = _lib()
    rng = np.random.default_rng(2024)
    I, W, H, ts = 2, 320, 192, 16
    tw, th = W // ts, H // ts
    m, r, d = random_projected(rng, I, 4000, W, H, ties=False)
    crowds = []
    for k, (n, cx, cy) in enumerate([(2000, 40, 24), (3500, 200, 40), (6000, 104, 136), (12000, 264, 152)]):
        cm = np.stack([rng.uniform(cx - 4, cx + 4, (I, n)), rng.uniform(cy - 4, cy + 4, (I, n))], -1)
        cr = rng.integers(1, 10, (I, n, 2))
        cd = rng.uniform(0.5, 20, (I, n))
        cd[:, : n // 3] = np.round(cd[:, : n // 3])
        crowds.append((cm.astype(np.float32), cr.astype(np.int32), cd.astype(np.float32)))
    m = np.concatenate([m] + [c[0] for c in crowds], 1)
    r = np.concatenate([r] + [c[1] for c in crowds], 1)
    d = np.concatenate([d] + [c[2] for c in crowds], 1)
    print("bucket all sort classes", flush=True)
    M, longest = _check(oracle, lib, m, r, d, I, ts, tw, th)
    lens = np.diff(np.append(oracle.isect_offset(oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)["isect_ids"],
                                                 I, tw, th).ravel(), M))
    for lo, hi in [(0, 2560), (2560, 4096), (4096, 8192), (8192, 16384)]:
        assert ((lens > lo) & (lens <= hi)).any(), (lo, hi)


def test_bucket_empty_and_limits(oracle):
    lib = _lib()
    assert lib.gsplat_hip_isect_bucket_max_list() == 16384
    assert lib.gsplat_hip_isect_bucket_supported(1, 240, 135)      # 3840x2160 at 16 px
    assert not lib.gsplat_hip_isect_bucket_supported(1, 480, 270)  # 7680x4320 at 16 px
    m = np.zeros((1, 50, 2), np.float32)
    r = np.zeros((1, 50, 2), np.int32)
    d = np.ones((1, 50), np.float32)
    rc, M, longest, tpg, ids, flat, offs = bucket(lib, m, r, d, 1, 16, 3, 2)
    assert rc == 0 and M == 0 and longest == 0 and not tpg.any() and not offs.any()


def test_list_longer_than_the_tile_sort(oracle):
    """20000 Gaussians on one tile, a quarter of them at one depth: the
    bucketed sort splits the list by its leading depth bits and sorts the
    runs in LDS (the quarter at one depth exceeds no run: the (id, depth)
    re-sort of a run); the same list with every depth equal goes to the
    global-memory radix sort (ids only). Both through the C ABI and
    intersect_tile_forward, against the oracle."""
    lib = _lib()
    g = gsplat()
    rng = np.random.default_rng(4)
    n = 20000
    m = np.stack([rng.uniform(17, 31, n), rng.uniform(17, 31, n)], -1).astype(np.float32)[None]
    r = np.full((1, n, 2), 2, np.int32)
    d = rng.uniform(1, 9, (1, n)).astype(np.float32)
    d[:, ::4] = 3.0
    for depths in (d, np.full_like(d, 5.0)):
        print(f"bucket long list, {np.unique(depths).size} distinct depths", flush=True)
        M, longest = _check(oracle, lib, m, r, depths, 1, 16, 4, 4)
        assert longest > 16384
        out = g.intersect_tile_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(depths)}, 1, 16, 4, 4)
        exp = oracle.isect_tile(m, r, depths, 1, 16, 4, 4, sort=True)
        np.testing.assert_array_equal(host(out["isect_ids"]), exp["isect_ids"])
        np.testing.assert_array_equal(host(out["flatten_ids"]), exp["flatten_ids"])
        np.testing.assert_array_equal(host(out["tiles_per_gauss"]), exp["tiles_per_gauss"])


def test_short_and_long_lists_in_one_frame(oracle):
    """Lists longer than the LDS tile sorts hold beside short lists and lists
    of every LDS class in one frame of two images: 20000 Gaussians on one
    tile (a quarter at one depth: split into LDS-sorted runs), 40000 on
    another (half of them at one depth, so one digit of the leading bits
    holds more than a run: the global-memory radix sort with its id
    re-sort), crowds of 3500 and 12000, and a random background; bit for bit
    against the oracle."""
    from test_gpu_isect import random_projected

    lib = _lib()
    rng = np.random.default_rng(40)
    I, W, H, ts = 2, 256, 192, 16
    tw, th = W // ts, H // ts
    m, r, d = random_projected(rng, I, 5000, W, H, ties=False)
    parts = [(m, r, d)]
    for n, cx, cy, kind in [(20000, 24, 24, "tie"), (40000, 200, 120, "crowded"), (3500, 120, 40, "flat"),
                            (12000, 72, 168, "tie")]:
        cm = np.stack([rng.uniform(cx - 6, cx + 6, (I, n)), rng.uniform(cy - 6, cy + 6, (I, n))], -1)
        cr = rng.integers(1, 3, (I, n, 2))
        cd = rng.uniform(1, 90, (I, n)) if kind == "crowded" else rng.uniform(1, 9, (I, n))
        if kind == "tie":
            cd[:, ::4] = 3.0
        if kind == "crowded":
            cd[:, ::2] = 30.0
        parts.append((cm.astype(np.float32), cr.astype(np.int32), cd.astype(np.float32)))
    m = np.concatenate([p[0] for p in parts], 1)
    r = np.concatenate([p[1] for p in parts], 1)
    d = np.concatenate([p[2] for p in parts], 1)
    print(f"bucket short and long lists N={d.shape[1]}", flush=True)
    M, longest = _check(oracle, lib, m, r, d, I, ts, tw, th)
    assert longest > 2 * 16384


@pytest.mark.parametrize("step", [0.25, 2.0])
def test_bucket_short_and_long_depth_runs(oracle, step):
    """Depths on a grid of `step`: equal-depth runs inside one tile list are a
    few entries long (step 0.25: the insertion sort of short runs) or
    hundreds long (step 2.0: the (id, depth) re-sort of the whole list)."""
    lib = _lib()
    rng = np.random.default_rng(int(step * 100))
    I, N, W, H, ts = 2, 9000, 320, 240, 16
    m = np.stack([rng.uniform(0, W, (I, N)), rng.uniform(0, H, (I, N))], -1).astype(np.float32)
    r = rng.integers(2, 24, size=(I, N, 2)).astype(np.int32)
    d = (np.round(rng.uniform(1, 10, (I, N)) / step) * step).astype(np.float32)
    print(f"bucket runs step={step}", flush=True)
    _check(oracle, lib, m, r, d, I, ts, W // ts, H // ts)


def test_fused_offsets_op(oracle):
    """intersect_tile_offsets_forward: the sorted intersection and its tile
    offsets from one call, against the oracle's isect_tile + isect_offset."""
    from test_gpu_isect import random_projected

    g = gsplat()
    rng = np.random.default_rng(77)
    I, N, W, H, ts = 2, 12000, 500, 380, 16
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    m, r, d = random_projected(rng, I, N, W, H, ties=True)
    got = g.intersect_tile_offsets_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(d)}, I, ts, tw, th)
    exp = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
    np.testing.assert_array_equal(host(got["tiles_per_gauss"]), exp["tiles_per_gauss"])
    np.testing.assert_array_equal(host(got["isect_ids"]), exp["isect_ids"])
    np.testing.assert_array_equal(host(got["flatten_ids"]), exp["flatten_ids"])
    np.testing.assert_array_equal(host(got["tile_offsets"]), oracle.isect_offset(exp["isect_ids"], I, tw, th))


def test_split_begin_end(oracle):
    """intersect_tile_offsets_begin / _end: the oracle's lists with other work
    queued between the halves (another intersection that reads its own count
    back), two pending calls finished in reverse order, and a pending call
    dropped unfinished (its read-back slot is reused afterwards)."""
    import torch
    from test_gpu_isect import random_projected

    g = gsplat()
    rng = np.random.default_rng(91)
    I, W, H, ts = 1, 400, 300, 16
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    scenes = [random_projected(rng, I, n, W, H, ties=True) for n in (6000, 9000)]
    inputs = [{"means2d": dev(m), "radii": dev(r), "depths": dev(d)} for m, r, d in scenes]
    pa = g.intersect_tile_offsets_begin(inputs[0], I, ts, tw, th)
    pb = g.intersect_tile_offsets_begin(inputs[1], I, ts, tw, th)
    mid = g.intersect_tile_forward(inputs[1], I, ts, tw, th)  # its own count read-back in between
    torch.cuda.current_stream().synchronize()
    dropped = g.intersect_tile_offsets_begin(inputs[0], I, ts, tw, th)
    del dropped
    outs = {1: g.intersect_tile_offsets_end(pb), 0: g.intersect_tile_offsets_end(pa)}
    assert g.intersect_tile_offsets_end(pa)["isect_ids"].data_ptr() == outs[0]["isect_ids"].data_ptr()
    for k, (m, r, d) in enumerate(scenes):
        exp = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
        got = outs[k]
        np.testing.assert_array_equal(host(got["tiles_per_gauss"]), exp["tiles_per_gauss"])
        np.testing.assert_array_equal(host(got["isect_ids"]), exp["isect_ids"])
        np.testing.assert_array_equal(host(got["flatten_ids"]), exp["flatten_ids"])
        np.testing.assert_array_equal(host(got["tile_offsets"]), oracle.isect_offset(exp["isect_ids"], I, tw, th))
    np.testing.assert_array_equal(host(mid["isect_ids"]), host(outs[1]["isect_ids"]))
