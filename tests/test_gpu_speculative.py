"""The speculative second step of the tile-bucket intersection: the scatter
and tile sort launched before M is on the host, into outputs sized by the
previous call's M, reading the new M on the device.

- C ABI (gsplat_hip_isect_bucket_sort_speculative): with a capacity at or
  above M and the longest list covered by the launched tile sort classes,
  the outputs equal the exact step's bit for bit; with a capacity below M,
  nothing is written past the capacity (guard words after the outputs and
  the workspace keep their values) -- the result is then discarded by the
  caller. gsplat_hip_isect_bucket_sort_covers against the class caps.
- C++ layer (intersect_tile_offsets_forward and the begin / end pair): the
  same inputs twice (the second call speculates and keeps its result), then
  inputs of the same shape with more entries (speculation discarded: M over
  the capacity) and with a list longer than any before (discarded: class not
  launched), each against the oracle."""
import ctypes
import os

import numpy as np
import pytest

from _helpers import dev, host, projected_scene

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")
P, I64, I32, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
GUARD = 4096


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_isect_bucket_count_workspace_size.restype = SZ
    lib.gsplat_hip_isect_bucket_count_workspace_size.argtypes = [I64, I64, I32, I32, I32]
    lib.gsplat_hip_isect_bucket_count.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_count.argtypes = [P, P, I64, I64, I32, I32, I32, P, P, P, SZ, P]
    lib.gsplat_hip_isect_bucket_sort_workspace_size.restype = SZ
    lib.gsplat_hip_isect_bucket_sort_workspace_size.argtypes = [I64]
    lib.gsplat_hip_isect_bucket_sort_covers.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_sort_covers.argtypes = [I64, I64]
    lib.gsplat_hip_isect_bucket_sort_speculative.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_sort_speculative.argtypes = [P, P, P, P, P, I32, P, I64, I64, I32, I32, I32, I64, I64,
                                                             P, P, P, P, P, SZ, P, SZ, P]
    return lib


def test_covers():
    lib = _lib()
    caps = [2560, 4096, 8192, 16384]
    for launched in [0, 100, 2560, 2561, 4096, 5000, 8192, 9000, 16384, 20000, 100000]:
        for longest in [0, 1, 2560, 2561, 4096, 4097, 8192, 8193, 16384, 16385, 99999]:
            cls = lambda x: sum(x > c for c in caps)
            assert lib.gsplat_hip_isect_bucket_sort_covers(launched, longest) == int(cls(longest) <= cls(launched))


def _scene(seed, n, W, H, crowd=0):
    rng = np.random.default_rng(seed)
    m, r, _, _, d = (a[0] for a in projected_scene(rng, 1, n, W, H))
    if crowd:  # one crowded tile: a long list
        m[:crowd] = [40.0, 24.0]
        r[:crowd] = [2, 2]
    return m, r, d


@pytest.mark.parametrize("cap_kind", ["exact", "larger", "smaller"])
@pytest.mark.parametrize("crowd", [0, 5000])
def test_c_abi_speculative(oracle, cap_kind, crowd):
    import torch

    lib = _lib()
    I, W, H, ts = 1, 400, 300, 16
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    m, r, d = _scene(7 + crowd, 20000, W, H, crowd)
    exp = oracle.isect_tile(m[None], r[None], d[None], I, ts, tw, th, sort=True)
    M = exp["isect_ids"].size
    eoffs = oracle.isect_offset(exp["isect_ids"], I, tw, th)
    longest = int(np.diff(np.append(eoffs.ravel(), M)).max())
    cap = {"exact": M, "larger": M + 1000, "smaller": M // 2}[cap_kind]
    print(f"speculative C ABI cap={cap_kind} crowd={crowd} M={M} longest={longest}", flush=True)
    stream = torch.cuda.current_stream().cuda_stream
    md, rd, dd = dev(m), dev(r), dev(d)
    numel = d.size
    tpg = torch.empty(numel, dtype=torch.int32, device="cuda")
    totals = torch.zeros(2, dtype=torch.int64, device="cuda")
    ws1b = lib.gsplat_hip_isect_bucket_count_workspace_size(I, numel, ts, tw, th)
    ws1 = torch.empty(ws1b, dtype=torch.uint8, device="cuda")
    assert lib.gsplat_hip_isect_bucket_count(md.data_ptr(), rd.data_ptr(), I, numel, ts, tw, th, tpg.data_ptr(),
                                             totals.data_ptr(), ws1.data_ptr(), ws1b, stream) == 0
    # outputs and workspace with guard words after the capacity
    ids = torch.full((cap + GUARD,), -7, dtype=torch.int64, device="cuda")
    flat = torch.full((cap + GUARD,), -7, dtype=torch.int32, device="cuda")
    offs = torch.empty(I * th * tw, dtype=torch.int32, device="cuda")
    ws2b = lib.gsplat_hip_isect_bucket_sort_workspace_size(cap)
    ws2 = torch.full((ws2b + 8 * GUARD,), 0x5A, dtype=torch.uint8, device="cuda")
    rc = lib.gsplat_hip_isect_bucket_sort_speculative(
        md.data_ptr(), rd.data_ptr(), None, None, dd.data_ptr(), 0, None, I, numel, ts, tw, th, cap, longest,
        totals.data_ptr(), ids.data_ptr(), flat.data_ptr(), offs.data_ptr(), ws1.data_ptr(), ws1b, ws2.data_ptr(),
        ws2b, stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    torch.cuda.synchronize()
    assert int(totals[0]) == M
    assert (host(ids[cap:]) == -7).all() and (host(flat[cap:]) == -7).all()
    assert (host(ws2[ws2b:]) == 0x5A).all()
    if cap >= M:
        np.testing.assert_array_equal(host(ids[:M]), exp["isect_ids"])
        np.testing.assert_array_equal(host(flat[:M]), exp["flatten_ids"])
        np.testing.assert_array_equal(host(offs).reshape(I, th, tw), eoffs)


@pytest.mark.parametrize("split", [False, True])
def test_layer_speculation_kept_and_discarded(oracle, split):
    from gsplat_core import _gsplat_core as _C

    I, W, H, ts = 1, 320, 240, 16
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts

    def run(m, r, d):
        inp = {"means2d": dev(m[None]), "radii": dev(r[None]), "depths": dev(d[None])}
        if split:
            return _C.intersect_tile_offsets_end(_C.intersect_tile_offsets_begin(inp, I, ts, tw, th))
        return _C.intersect_tile_offsets_forward(inp, I, ts, tw, th)

    n = 12345 + int(split)  # a shape of its own, so the first call has no hint
    cases = [("first", _scene(1, n, W, H)), ("same", _scene(1, n, W, H)),
             ("more entries", _scene(2, n, W, H)), ("long list", _scene(3, n, W, H, crowd=9000)),
             ("fewer", _scene(4, n, W, H))]
    # more entries: larger radii for the same count
    cases[2][1][1][:] = cases[2][1][1] * 2 + 1
    for name, (m, r, d) in cases:
        print(f"speculation split={split}: {name}", flush=True)
        exp = oracle.isect_tile(m[None], r[None], d[None], I, ts, tw, th, sort=True)
        o = run(m, r, d)
        np.testing.assert_array_equal(host(o["isect_ids"]), exp["isect_ids"], err_msg=name)
        np.testing.assert_array_equal(host(o["flatten_ids"]), exp["flatten_ids"], err_msg=name)
        np.testing.assert_array_equal(host(o["tiles_per_gauss"]), exp["tiles_per_gauss"], err_msg=name)
        np.testing.assert_array_equal(host(o["tile_offsets"]), oracle.isect_offset(exp["isect_ids"], I, tw, th),
                                      err_msg=name)
