"""gsplat_hip_rasterize_bwd_noalloc (the allocation-free rasterize backward,
schedule scratch in a static device array) against gsplat_hip_rasterize_bwd
(caller workspace), both called through the C ABI: gradients within 1e-4
relative of each other (the float atomics may add in a different order; the
parity bar is 1e-3), on two calls in a row, the second with a smaller input,
so stale scratch contents from the first call would show. Also: sizes beyond
the scratch are rejected on the host."""
import ctypes
import os

import numpy as np
import pytest

from _helpers import assert_close_rel, dev, gsplat, host

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")
P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
BWD_ARGS = [P, P, P, P, P, P, P, P, I64, I64, I32, I32, I32, I32, I32, I32, I64, P, P, P, P, P, P, P, P, P, P]


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_rasterize_bwd.restype = ctypes.c_int
    lib.gsplat_hip_rasterize_bwd.argtypes = BWD_ARGS + [P, ctypes.c_size_t, P]
    lib.gsplat_hip_rasterize_bwd_noalloc.restype = ctypes.c_int
    lib.gsplat_hip_rasterize_bwd_noalloc.argtypes = BWD_ARGS + [P]
    lib.gsplat_hip_rasterize_bwd_workspace_size.restype = ctypes.c_size_t
    lib.gsplat_hip_rasterize_bwd_workspace_size.argtypes = [I64, I32, I32, I32]
    lib.gsplat_hip_rasterize_bwd_noalloc_max_scratch.restype = ctypes.c_size_t
    return lib


def _scene(oracle, seed, I, N, W, H, ts, C):
    from test_gpu_raster import make_scene

    rng = np.random.default_rng(seed)
    s = make_scene(oracle, rng, I, N, W, H, ts, C)
    g = gsplat()
    inp = {k: dev(s[k]) for k in ("means2d", "conics", "colors", "opacities", "backgrounds", "tile_offsets",
                                  "flatten_ids")}
    fwd = g.rasterize_to_pixels_3dgs_forward(inp, W, H, ts)
    v_rc = dev(rng.normal(size=(I, H, W, C)).astype(np.float32))
    v_ra = dev(rng.normal(size=(I, H, W, 1)).astype(np.float32))
    return s, inp, fwd, v_rc, v_ra


def _call(lib, noalloc, inp, fwd, v_rc, v_ra, I, N, C, W, H, ts):
    import torch

    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    G = I * N
    outs = {"v_means2d_abs": torch.full((G * 2,), 7.0, device="cuda"),
            "v_means2d": torch.full((G * 2,), 7.0, device="cuda"),
            "v_conics": torch.full((G * 3,), 7.0, device="cuda"),
            "v_colors": torch.full((G * C,), 7.0, device="cuda"),
            "v_opacities": torch.full((G,), 7.0, device="cuda"),
            "v_backgrounds": torch.full((I * C,), 7.0, device="cuda")}
    args = [inp["means2d"].data_ptr(), inp["conics"].data_ptr(), inp["colors"].data_ptr(),
            inp["opacities"].data_ptr(), inp["backgrounds"].data_ptr(), None, inp["tile_offsets"].data_ptr(),
            inp["flatten_ids"].data_ptr(), I, N, C, W, H, ts, tw, th, inp["flatten_ids"].numel(),
            fwd["render_alphas"].data_ptr(), fwd["last_ids"].data_ptr(), v_rc.data_ptr(), v_ra.data_ptr(),
            outs["v_means2d_abs"].data_ptr(), outs["v_means2d"].data_ptr(), outs["v_conics"].data_ptr(),
            outs["v_colors"].data_ptr(), outs["v_opacities"].data_ptr(), outs["v_backgrounds"].data_ptr()]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.gsplat_hip_rasterize_bwd_noalloc(*args, stream)
    else:
        ws_bytes = lib.gsplat_hip_rasterize_bwd_workspace_size(I, C, tw, th)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        rc = lib.gsplat_hip_rasterize_bwd(*args, ws.data_ptr(), ws_bytes, stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    torch.cuda.synchronize()
    return {k: host(v) for k, v in outs.items()}


def test_noalloc_backward_matches_workspace_backward(oracle):
    lib = _lib()
    # the second call is smaller (fewer images, tiles, Gaussians and channels)
    for seed, (I, N, W, H, ts, C) in enumerate([(2, 3000, 320, 200, 16, 3), (1, 900, 96, 80, 16, 2)]):
        print(f"noalloc backward call {seed}: I={I} N={N} {W}x{H} C={C}", flush=True)
        s, inp, fwd, v_rc, v_ra = _scene(oracle, 40 + seed, I, N, W, H, ts, C)
        want = _call(lib, False, inp, fwd, v_rc, v_ra, I, N, C, W, H, ts)
        got = _call(lib, True, inp, fwd, v_rc, v_ra, I, N, C, W, H, ts)
        # the two calls run the same kernels and differ only in the order of
        # their float atomic additions (sums that cancel lose a few more
        # digits); stale scratch from the first call would be off by O(1)
        for k in want:
            assert np.isfinite(want[k]).all(), k
            assert_close_rel(got[k], want[k], 1e-4, k)
        assert np.abs(want["v_colors"]).max() > 0 and np.abs(want["v_backgrounds"]).max() > 0


def test_noalloc_rejects_sizes_beyond_the_scratch():
    lib = _lib()
    cap = lib.gsplat_hip_rasterize_bwd_noalloc_max_scratch()
    assert cap == 8 << 20
    # 16 images of 3840x2160 at 64 channels: far more schedule than the scratch
    # holds; rejected on the host before any pointer is touched
    dummy = ctypes.c_void_p(16)
    args = [dummy] * 8 + [16, 10, 64, 3840, 2160, 16, 240, 135, 100, dummy, dummy, dummy, None, None,
                          dummy, dummy, dummy, dummy, dummy, None]
    rc = lib.gsplat_hip_rasterize_bwd_noalloc(*args)
    assert rc == 1
    assert b"static scratch" in lib.gsplat_hip_last_error()
    assert lib.gsplat_hip_rasterize_bwd_workspace_size(16, 64, 240, 135) > cap
