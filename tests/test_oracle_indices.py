"""Pins the oracle's rasterize_to_indices (upstream gsplat's
rasterize_to_indices_in_range; the reference's planned
rasterize_to_indices_3dgs_forward, note/gsplat_cuda_source_map.md:494-545)
against the oracle forward rasterizer, which its own tests pin: the listed
Gaussians of a pixel are exactly the ones the forward composites -- the last
one is flatten_ids[last_ids], their float32 recomposition reproduces the
forward image bit for bit and their alpha product its transmittance -- and
chunked ranges with carried transmittances extend the full list."""
import ctypes
import ctypes.util

import numpy as np

from test_oracle_raster import make_scene

# the C library's expf, which the oracle's float32 loop calls (numpy's float32
# exp may differ from it in the last bit)
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]


def _expf(x):
    return np.float32(_libm.expf(float(x)))


def _pixel_lists(gids, idx, n_pix):
    order = np.argsort(idx, kind="stable")
    assert (order == np.arange(idx.size)).all()  # pixel-major already
    bounds = np.searchsorted(idx, np.arange(n_pix + 1))
    return [gids[bounds[p]:bounds[p + 1]] for p in range(n_pix)]


def test_indices_are_the_composited_entries(oracle):
    rng = np.random.default_rng(4)
    s = make_scene(oracle, rng, I=2, N=120, W=40, H=28, ts=8, C=3, dtype=np.float32, mean_opac=(0.3, 0.95))
    W, H, ts = s["W"], s["H"], s["ts"]
    f = oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                              s["flatten_ids"], W, H, ts)
    gids, idx = oracle.raster_indices(s["means2d"], s["conics"], s["opacities"], s["tile_offsets"], s["flatten_ids"],
                                      W, H, ts)
    I = s["tile_offsets"].shape[0]
    lists = _pixel_lists(gids, idx, I * H * W)
    m2 = s["means2d"].reshape(-1, 2)
    co = s["conics"].reshape(-1, 3)
    cl = s["colors"].reshape(-1, 3)
    op = s["opacities"].ravel()
    rc = f["render_colors"].reshape(-1, 3)
    ra = f["render_alphas"].ravel()
    li = f["last_ids"].ravel()
    n_multi = 0
    for p, lst in enumerate(lists):
        img, rem = divmod(p, H * W)
        y, x = divmod(rem, W)
        px, py = np.float32(x + 0.5), np.float32(y + 0.5)
        T = np.float32(1.0)
        out = np.zeros(3, np.float32)
        for g in lst:
            dx, dy = m2[g, 0] - px, m2[g, 1] - py
            sig = np.float32(0.5) * (co[g, 0] * dx * dx + co[g, 2] * dy * dy) + co[g, 1] * dx * dy
            a = min(np.float32(0.99), op[g] * _expf(-sig))
            out = out + cl[g] * (a * T)
            T = T * (np.float32(1) - a)
        np.testing.assert_array_equal(out, rc[p], err_msg=f"pixel {p}")
        np.testing.assert_allclose(1 - T, ra[p], rtol=0, atol=1e-6)
        if len(lst):
            assert lst[-1] == s["flatten_ids"][li[p]]
        n_multi += len(lst) > 1
    assert n_multi > 100


def test_chunked_ranges_concatenate(oracle):
    rng = np.random.default_rng(8)
    s = make_scene(oracle, rng, I=1, N=150, W=32, H=24, ts=8, C=3, dtype=np.float32, mean_opac=(0.5, 0.99))
    W, H, ts = s["W"], s["H"], s["ts"]
    args = (s["means2d"], s["conics"], s["opacities"], s["tile_offsets"], s["flatten_ids"], W, H, ts)
    full_g, full_i = oracle.raster_indices(*args)
    n_pix = H * W
    full = _pixel_lists(full_g, full_i, n_pix)
    m2 = s["means2d"].reshape(-1, 2)
    co = s["conics"].reshape(-1, 3)
    op = s["opacities"].ravel()
    T = np.ones((1, H, W), np.float32)
    got = [[] for _ in range(n_pix)]
    k = 7
    for r0 in range(0, 200, k):
        g, i = oracle.raster_indices(*args, range_start=r0, range_end=r0 + k, transmittances=T)
        for gg, ii in zip(g, i):
            got[ii].append(gg)
            y, x = divmod(int(ii), W)
            dx, dy = m2[gg, 0] - np.float32(x + 0.5), m2[gg, 1] - np.float32(y + 0.5)
            sig = np.float32(0.5) * (co[gg, 0] * dx * dx + co[gg, 2] * dy * dy) + co[gg, 1] * dx * dy
            T[0, y, x] = T[0, y, x] * (np.float32(1) - min(np.float32(0.99), op[gg] * _expf(-sig)))
    # a pixel whose list ended because the transmittance would have fallen to
    # 1e-4 is not marked done across calls: a later range starts again from
    # the carried transmittance, so the full list is a prefix of the chunked
    # one (equal wherever the list ended by running out of entries)
    for p in range(n_pix):
        assert list(full[p]) == got[p][:len(full[p])], p
