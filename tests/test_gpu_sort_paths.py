"""The radix sort's less-travelled paths, forced at small sizes through the
library's test hooks and checked bit for bit against numpy's stable sort and
the oracle's intersection lists:

- the look-back recount: a partition whose predecessor has not published
  within the spin limit recounts its digit prefix from the pass input. A
  negative limit recounts in every partition, a zero limit whenever the first
  poll finds an unpublished predecessor (a run-dependent mix of both ways);
- the reduce-then-scan path that sorts of 2^30 keys or more take (histogram,
  scan, scatter per pass), forced by lowering the onesweep key limit;
- the signed sort that skips constant digits on the device (every key shape
  of digits constant and varying, all keys equal), on all three paths;
- in the depth-presorted intersection, the tile-key sort carrying each
  entry's depth bits (taken above 2^21 pairs) and the encode blocks' rank
  ranges from the up-front split kernel (taken from 65536 blocks), forced on
  at small sizes for the AABB, ellipse and packed encodes;
- the carrying AABB sort's generated first pass (keys formed inside the pass
  from the depth ranks' rects instead of encoded; taken with at least four
  entries per Gaussian) against the encoded one, with one, two and three
  passes, several images, partitions spanning more ranks than one LDS chunk
  holds, and the recount of its look-back prefix from the rects.

Every kernel runs to completion in these tests: the hooks only change which
of two correct ways a partition obtains its prefix, or which sort runs."""
import ctypes
import os

import numpy as np
import pytest

from _helpers import dev, gsplat, host

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")
PART = 4096  # keys per onesweep partition


def _lib():
    lib = ctypes.CDLL(LIB)
    p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_sort_debug_set.restype = None
    lib.gsplat_hip_sort_debug_set.argtypes = [i32, i64]
    lib.gsplat_hip_sort_debug_reset.restype = None
    lib.gsplat_hip_sort_lookback_recounts.restype = ctypes.c_int
    lib.gsplat_hip_sort_lookback_recounts.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    lib.gsplat_hip_isect_sort_workspace_size.restype = ctypes.c_size_t
    lib.gsplat_hip_isect_sort_workspace_size.argtypes = [i64]
    lib.gsplat_hip_isect_sort.restype = ctypes.c_int
    lib.gsplat_hip_isect_sort.argtypes = [p, p, i64, i32, p, p, p, ctypes.c_size_t, p]
    lib.gsplat_hip_isect_sort_i64.restype = ctypes.c_int
    lib.gsplat_hip_isect_sort_i64.argtypes = [p, p, i64, p, p, p, ctypes.c_size_t, p]
    lib.gsplat_hip_isect_debug_set.restype = None
    lib.gsplat_hip_isect_debug_set.argtypes = [i64, i64]
    lib.gsplat_hip_isect_debug_reset.restype = None
    lib.gsplat_hip_isect_debug_generated.restype = None
    lib.gsplat_hip_isect_debug_generated.argtypes = [i32]
    lib.gsplat_hip_isect_tile_sorted_workspace_size.restype = ctypes.c_size_t
    lib.gsplat_hip_isect_tile_sorted_workspace_size.argtypes = [i64, i64]
    lib.gsplat_hip_isect_tile_sorted.restype = ctypes.c_int
    lib.gsplat_hip_isect_tile_sorted.argtypes = [p, p, p, p, i64, i64, i32, i32, i32, i64, p, p, p, ctypes.c_size_t, p]
    return lib


@pytest.fixture
def lib():
    lib = _lib()
    lib.gsplat_hip_sort_debug_reset()
    lib.gsplat_hip_isect_debug_reset()
    yield lib
    lib.gsplat_hip_sort_debug_reset()
    lib.gsplat_hip_isect_debug_reset()


def _recounts(lib):
    v = ctypes.c_uint64(0)
    assert lib.gsplat_hip_sort_lookback_recounts(ctypes.byref(v)) == 0, lib.gsplat_hip_last_error()
    return int(v.value)


def _sort(lib, keys, vals, bits):
    import torch

    n = keys.size
    kd, vd = dev(keys), dev(vals)
    ws_bytes = lib.gsplat_hip_isect_sort_workspace_size(n)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    ko, vo = torch.empty_like(kd), torch.empty_like(vd)
    rc = lib.gsplat_hip_isect_sort(kd.data_ptr(), vd.data_ptr(), n, bits, ko.data_ptr(), vo.data_ptr(),
                                   ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    torch.cuda.synchronize()
    return host(ko), host(vo)


def _sort_i64(lib, keys, vals):
    """The device-planned signed sort (all 64 bits, constant digits skipped
    on the device)."""
    import torch

    n = keys.size
    kd, vd = dev(keys), dev(vals)
    ws_bytes = lib.gsplat_hip_isect_sort_workspace_size(n)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    ko, vo = torch.empty_like(kd), torch.empty_like(vd)
    rc = lib.gsplat_hip_isect_sort_i64(kd.data_ptr(), vd.data_ptr(), n, ko.data_ptr(), vo.data_ptr(),
                                       ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(kd), keys)  # inputs unchanged
    return host(ko), host(vo)


def _signed_keys(kind, n, seed):
    rng = np.random.default_rng(seed)
    if kind == "full":  # every digit varies, both signs, extremes
        keys = rng.integers(np.iinfo(np.int64).min, np.iinfo(np.int64).max, size=n, dtype=np.int64)
        keys[: min(n, 4)] = np.array([np.iinfo(np.int64).min, -1, 0, np.iinfo(np.int64).max])[: min(n, 4)]
    elif kind == "ids":  # intersection-shaped: image | tile | depth bits, high digits constant
        keys = (rng.integers(0, 3, n) << 46) | (rng.integers(0, 4346, n) << 32) | rng.integers(0, 1 << 32, n)
    elif kind == "middle":  # digits 2, 3 and 5 constant (0xAB, 0x00, 0x7F), the rest varying, some negative
        keys = rng.integers(0, 1 << 62, size=n, dtype=np.int64)
        keys &= ~np.int64((0xFF << 16) | (0xFF << 24) | (0xFF << 40))
        keys |= np.int64((0xAB << 16) | (0x7F << 40))
        keys[rng.random(n) < 0.5] *= -1
    elif kind == "negative":  # all negative, one varying digit in the middle
        keys = -(np.int64(1) << 50) + (rng.integers(0, 256, n).astype(np.int64) << 24)
    else:  # "equal": no pass runs, the output is the input
        keys = np.full(n, -12345678901, np.int64)
    keys = keys.astype(np.int64)
    keys[rng.random(n) < 0.3] = keys[0]  # ties: stability matters
    return keys, rng.permutation(n).astype(np.int32)


@pytest.mark.parametrize("kind", ["full", "ids", "middle", "negative", "equal"])
@pytest.mark.parametrize("n", [1, 4096, 100_003])
@pytest.mark.parametrize("path", ["onesweep", "recount", "reduce_then_scan"])
def test_signed_planned_sort(lib, kind, n, path):
    """gsplat_hip_isect_sort_i64 against numpy's stable argsort of the int64
    keys: signed order, all 64 bits, on each sort path."""
    keys, vals = _signed_keys(kind, n, n + len(kind))
    order = np.argsort(keys, kind="stable")
    print(f"signed planned sort kind={kind} n={n} path={path}", flush=True)
    if path == "recount":
        lib.gsplat_hip_sort_debug_set(-1, 0)
    elif path == "reduce_then_scan":
        lib.gsplat_hip_sort_debug_set(1 << 18, 1)
    for _ in range(2):  # the second run reuses the plan words of the first
        ko, vo = _sort_i64(lib, keys, vals)
        np.testing.assert_array_equal(ko, keys[order])
        np.testing.assert_array_equal(vo, vals[order])


def _keys(n, bits, seed):
    rng = np.random.default_rng(seed)
    keys = rng.integers(0, 1 << min(bits, 62), size=n, dtype=np.int64)
    keys[rng.random(n) < 0.3] = keys[0]  # many equal keys: stability matters
    return keys, np.arange(n, dtype=np.int32)


@pytest.mark.parametrize("n,bits", [(4097, 20), (100_003, 45), (262_144, 64)])
def test_forced_recount_is_exact(lib, n, bits):
    keys, vals = _keys(n, bits, n)
    order = np.argsort(keys, kind="stable")
    print(f"forced recount n={n} bits={bits}", flush=True)
    before = _recounts(lib)
    lib.gsplat_hip_sort_debug_set(-1, 0)
    ko, vo = _sort(lib, keys, vals, bits)
    np.testing.assert_array_equal(ko, keys[order])
    np.testing.assert_array_equal(vo, vals[order])
    # every partition but the first of every pass took the recount
    passes, parts = (bits + 7) // 8, (n + PART - 1) // PART
    assert _recounts(lib) - before == passes * (parts - 1)


@pytest.mark.parametrize("n,bits", [(50_000, 33), (300_001, 64)])
def test_zero_spin_limit_is_exact(lib, n, bits):
    keys, vals = _keys(n, bits, n + 1)
    order = np.argsort(keys, kind="stable")
    print(f"zero spin limit n={n} bits={bits}", flush=True)
    lib.gsplat_hip_sort_debug_set(0, 0)
    for _ in range(3):
        ko, vo = _sort(lib, keys, vals, bits)
        np.testing.assert_array_equal(ko, keys[order])
        np.testing.assert_array_equal(vo, vals[order])


def test_default_path_does_not_recount(lib):
    keys, vals = _keys(1 << 20, 48, 3)
    before = _recounts(lib)
    ko, _ = _sort(lib, keys, vals, 48)
    np.testing.assert_array_equal(ko, np.sort(keys, kind="stable"))
    assert _recounts(lib) == before


@pytest.mark.parametrize("n,bits", [(1, 40), (4095, 20), (4097, 33), (100_003, 45), (262_144, 64)])
def test_reduce_then_scan_path_is_exact(lib, n, bits):
    keys, vals = _keys(n, bits, n + 2)
    order = np.argsort(keys, kind="stable")
    print(f"reduce-then-scan n={n} bits={bits}", flush=True)
    lib.gsplat_hip_sort_debug_set(1 << 18, 1)  # every sort of >= 1 key takes the fallback
    ko, vo = _sort(lib, keys, vals, bits)
    np.testing.assert_array_equal(ko, keys[order])
    np.testing.assert_array_equal(vo, vals[order])


@pytest.mark.parametrize("carry,splits,generated", [(False, False, False), (False, True, False),
                                                     (True, False, False), (True, True, False),
                                                     (True, False, True)])
@pytest.mark.parametrize("mode", ["onesweep", "recount", "reduce_then_scan"])
def test_intersection_pipeline_on_forced_paths(lib, oracle, mode, carry, splits, generated):
    """The two sorts of the depth-presorted intersection pipeline (32-bit
    depth keys gathering the counts; 32-bit tile keys assembling the 64-bit
    ids, with the depth bits gathered or carried), through the C ABI's one-call
    entry point, on the forced sort paths give the oracle's sorted lists bit
    for bit."""
    import torch

    from test_gpu_isect import random_projected

    rng = np.random.default_rng(5)
    I, N, W, H, ts = 2, 30_000, 640, 480, 16
    m, r, d = random_projected(rng, I, N, W, H, ties=True, signed=True)
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    exp = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
    counts = oracle.isect_count(m, r, ts, tw, th).astype(np.int32)
    n_isects = int(counts.sum())
    print(f"intersection pipeline, {mode} carry={carry} splits={splits} generated={generated}, "
          f"{n_isects} intersections", flush=True)
    assert n_isects >= 4 * I * N  # the generated pass's condition
    if mode == "recount":
        lib.gsplat_hip_sort_debug_set(-1, 0)
    elif mode == "reduce_then_scan":
        lib.gsplat_hip_sort_debug_set(1 << 18, 1)
    lib.gsplat_hip_isect_debug_set(0 if carry else 1 << 40, 1 if splits else 1 << 40)
    lib.gsplat_hip_isect_debug_generated(1 if generated else 0)
    ws_bytes = lib.gsplat_hip_isect_tile_sorted_workspace_size(I * N, n_isects)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    md, rd, dd, cd = dev(m), dev(r), dev(d), dev(counts)
    ids = torch.empty(n_isects, dtype=torch.int64, device="cuda")
    flat = torch.empty(n_isects, dtype=torch.int32, device="cuda")
    rc = lib.gsplat_hip_isect_tile_sorted(md.data_ptr(), rd.data_ptr(), dd.data_ptr(), cd.data_ptr(), I, I * N, ts,
                                          tw, th, n_isects, ids.data_ptr(), flat.data_ptr(), ws.data_ptr(), ws_bytes,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(ids), exp["isect_ids"])
    np.testing.assert_array_equal(host(flat), exp["flatten_ids"])


@pytest.mark.parametrize("layout", ["accutile", "packed", "packed_accutile"])
def test_sorted_encodes_with_carried_bits_and_splits(lib, oracle, layout):
    """The ellipse and packed sorted encodes (which take the depth-presorted
    path) with the depth bits carried and the split kernel forced on give the
    oracle's sorted lists bit for bit."""
    from test_gpu_accutile import TS, _inputs
    from _helpers import projected_scene

    g = gsplat()
    rng = np.random.default_rng(23)
    lib.gsplat_hip_isect_debug_set(0, 1)
    W, H = 640, 480
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    print(f"sorted encode {layout} with carried bits and splits", flush=True)
    if layout == "accutile":
        I, N = 2, 20_000
        means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
        out = g._gsplat_core.intersect_tile_forward(_inputs(means, radii, depths, conics, opac), I, TS, tw, th)
        ref = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=True, conics=conics, opacities=opac)
    else:
        I, nnz = 4, 30_000
        means, radii, conics, opac, depths = (a[0] for a in projected_scene(rng, 1, nnz, W, H))
        img = np.sort(rng.integers(0, I, nnz)).astype(np.int32)
        inp = {"means2d": dev(means), "radii": dev(radii), "depths": dev(depths), "image_ids": dev(img)}
        kw = {}
        if layout == "packed_accutile":
            inp["conics"], inp["opacities"] = dev(conics), dev(opac)
            kw = {"conics": conics, "opacities": opac}
        out = g.intersect_tile_forward(inp, I, TS, tw, th)
        ref = oracle.isect_tile_packed(means, radii, depths, img, I, TS, tw, th, sort=True, **kw)
    np.testing.assert_array_equal(host(out["isect_ids"]), ref["isect_ids"])
    np.testing.assert_array_equal(host(out["flatten_ids"]), ref["flatten_ids"])


@pytest.mark.parametrize("case", ["mixed", "three_passes", "one_pass", "images"])
@pytest.mark.parametrize("recount", [False, True])
def test_generated_first_pass(lib, oracle, case, recount):
    """The generated first pass (carried bits, keys formed in the pass) gives
    the oracle's sorted lists bit for bit: mixed has a depth range of
    one-tile and invisible Gaussians before large ones, so partitions there
    hold more ranks than one LDS chunk (1535); three_passes a 65536-tile grid
    (17 key bits); one_pass an 8 x 8 tile grid (7 bits: the generated pass is
    also the last); images four images. recount: every partition recounts its
    look-back prefix from the rects."""
    import torch

    from test_gpu_isect import random_projected

    rng = np.random.default_rng({"mixed": 1, "three_passes": 2, "one_pass": 3, "images": 4}[case])
    I, ts = 1, 16
    if case == "mixed":
        N, W, H = 40_000, 640, 480
        m = np.stack([rng.uniform(0, W, (I, N)), rng.uniform(0, H, (I, N))], -1).astype(np.float32)
        d = rng.uniform(0.1, 50, (I, N)).astype(np.float32)
        near = d < 25  # the near half: one-tile Gaussians, a third of them invisible
        r = np.where(near[..., None], 3, rng.integers(40, 120, (I, N, 2))).astype(np.int32)
        r[near & (rng.random((I, N)) < 0.33)] = 0
    elif case == "three_passes":
        N, W, H = 30_000, 4096, 4096
        m, r, d = random_projected(rng, I, N, W, H, ties=True)
    elif case == "one_pass":
        N, W, H = 5_000, 128, 128
        m, r, d = random_projected(rng, I, N, W, H, ties=True, signed=True)
    else:
        I, N, W, H = 4, 8_000, 320, 240
        m, r, d = random_projected(rng, I, N, W, H, ties=True)
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    exp = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
    counts = oracle.isect_count(m, r, ts, tw, th).astype(np.int32)
    n_isects = int(counts.sum())
    print(f"generated first pass {case} recount={recount}: {I}x{N} Gaussians, {tw}x{th} tiles, "
          f"{n_isects} intersections", flush=True)
    assert n_isects >= 4 * I * N
    if recount:
        lib.gsplat_hip_sort_debug_set(-1, 0)
    lib.gsplat_hip_isect_debug_set(0, 1 << 40)  # carry the depth bits
    before = _recounts(lib)
    ws_bytes = lib.gsplat_hip_isect_tile_sorted_workspace_size(I * N, n_isects)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    md, rd, dd, cd = dev(m), dev(r), dev(d), dev(counts)
    ids = torch.empty(n_isects, dtype=torch.int64, device="cuda")
    flat = torch.empty(n_isects, dtype=torch.int32, device="cuda")
    rc = lib.gsplat_hip_isect_tile_sorted(md.data_ptr(), rd.data_ptr(), dd.data_ptr(), cd.data_ptr(), I, I * N, ts,
                                          tw, th, n_isects, ids.data_ptr(), flat.data_ptr(), ws.data_ptr(), ws_bytes,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(ids), exp["isect_ids"])
    np.testing.assert_array_equal(host(flat), exp["flatten_ids"])
    if recount:  # every partition after the first of every pass (the depth sort's too) recounted
        assert _recounts(lib) - before > (n_isects + PART - 1) // PART - 1
