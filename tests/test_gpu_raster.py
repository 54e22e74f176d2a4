"""GPU parity for rasterization against the oracle: images within 1e-4
max-abs, alphas within 1e-5 relative, last_ids exact, gradients within 1e-3
relative; plus the reference's closed forms and tile masks
(gsplat_core/test/test.cpp:1067-1386)."""
import numpy as np
import pytest

from _helpers import assert_close_rel, dev, gsplat, host

pytestmark = pytest.mark.gpu

IMG_ATOL = 1e-4
GRAD_RTOL = 1e-3


def _raster_inputs(s):
    inp = {"means2d": dev(s["means2d"]), "conics": dev(s["conics"]), "colors": dev(s["colors"]),
           "opacities": dev(s["opacities"]), "tile_offsets": dev(s["tile_offsets"]),
           "flatten_ids": dev(s["flatten_ids"])}
    if s.get("backgrounds") is not None:
        inp["backgrounds"] = dev(s["backgrounds"])
    if s.get("masks") is not None:
        inp["masks"] = dev(s["masks"])
    return inp


def test_single_gaussian_closed_form():
    g = gsplat()
    s = dict(means2d=np.array([[[1.0, 1.0]]], np.float32), conics=np.array([[[1.0, 0.0, 1.0]]], np.float32),
             colors=np.array([[[1.0, 0.0, 0.0]]], np.float32), opacities=np.array([[0.5]], np.float32),
             backgrounds=np.array([[0.1, 0.2, 0.3]], np.float32), tile_offsets=np.zeros((1, 1, 1), np.int32),
             flatten_ids=np.zeros(1, np.int32))
    out = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s), 2, 2, 2)
    a = 0.5 * np.exp(-0.25)
    np.testing.assert_allclose(host(out["render_alphas"]).ravel(), a, atol=1e-5)
    np.testing.assert_allclose(host(out["render_colors"]).reshape(4, 3),
                               [[a + (1 - a) * 0.1, (1 - a) * 0.2, (1 - a) * 0.3]] * 4, atol=1e-5)
    assert np.all(host(out["last_ids"]) == 0)
    # masks: right tile masked -> background, alpha 0 (test.cpp:1199-1271)
    s["tile_offsets"] = np.array([[[0, 1]]], np.int32)
    s["masks"] = np.array([[[True, False]]])
    out = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s), 4, 2, 2)
    ra = host(out["render_alphas"])[0, :, :, 0]
    np.testing.assert_allclose(ra[:, :2], a, atol=1e-5)
    np.testing.assert_allclose(ra[:, 2:], 0, atol=1e-7)
    np.testing.assert_allclose(host(out["render_colors"])[0, :, 2:], np.broadcast_to([0.1, 0.2, 0.3], (2, 2, 3)),
                               atol=1e-6)


def test_backward_reference_case(oracle):
    # test.cpp:1273-1386 inputs (CPU vs GPU at 1e-4 in the reference)
    g = gsplat()
    s = dict(means2d=np.array([[[0.75, 0.75], [1.35, 1.15]]], np.float32),
             conics=np.array([[[0.35, 0.02, 0.45], [0.25, -0.03, 0.3]]], np.float32),
             colors=np.array([[[0.8, 0.2, 0.1], [0.1, 0.7, 0.4]]], np.float32),
             opacities=np.array([[0.6, 0.45]], np.float32), backgrounds=np.array([[0.05, 0.1, 0.2]], np.float32),
             tile_offsets=np.zeros((1, 1, 1), np.int32), flatten_ids=np.array([0, 1], np.int32))
    v_rc = np.array([0.2, -0.1, 0.3, 0.4, 0.05, -0.2, -0.3, 0.25, 0.15, 0.1, -0.4, 0.35], np.float32).reshape(1, 2, 2, 3)
    v_ra = np.array([0.2, -0.1, 0.05, 0.3], np.float32).reshape(1, 2, 2, 1)
    fwd = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s), 2, 2, 2)
    bwd = g.rasterize_to_pixels_3dgs_backward(_raster_inputs(s), fwd, {"v_render_colors": dev(v_rc),
                                                                        "v_render_alphas": dev(v_ra)}, 2, 2, 2,
                                              absgrad=True)
    ef = oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                               s["flatten_ids"], 2, 2, 2, backgrounds=s["backgrounds"])
    eb = oracle.raster_backward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                s["flatten_ids"], 2, 2, 2, ef["render_alphas"], ef["last_ids"], v_rc, v_ra,
                                backgrounds=s["backgrounds"], absgrad=True)
    for k in eb:
        np.testing.assert_allclose(host(bwd[k]), eb[k], atol=1e-4, err_msg=k)


def make_scene(oracle, rng, I, N, W, H, ts, C, opac=(0.05, 0.95), scale=(2.0, 6.0), masks=False):
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    means2d = np.stack([rng.uniform(-10, W + 10, (I, N)), rng.uniform(-10, H + 10, (I, N))], -1).astype(np.float32)
    A = rng.normal(size=(I, N, 2, 2)) * rng.uniform(*scale, (I, N, 1, 1))
    cov = A @ np.swapaxes(A, -1, -2) + 0.3 * np.eye(2)
    inv = np.linalg.inv(cov)
    conics = np.stack([inv[..., 0, 0], inv[..., 0, 1], inv[..., 1, 1]], -1).astype(np.float32)
    radii = np.ceil(3.33 * np.sqrt(np.stack([cov[..., 0, 0], cov[..., 1, 1]], -1))).astype(np.int32)
    depths = rng.uniform(1, 10, (I, N)).astype(np.float32)
    isect = oracle.isect_tile(means2d, radii, depths, I, ts, tw, th)
    offs = oracle.isect_offset(isect["isect_ids"], I, tw, th)
    s = dict(means2d=means2d, conics=conics, colors=rng.uniform(0, 1, (I, N, C)).astype(np.float32),
             opacities=rng.uniform(*opac, (I, N)).astype(np.float32),
             backgrounds=rng.uniform(0, 0.3, (I, C)).astype(np.float32), tile_offsets=offs,
             flatten_ids=isect["flatten_ids"])
    if masks:
        s["masks"] = rng.random((I, th, tw)) < 0.8
    return s


def _oracle_fwd(oracle, s, W, H, ts):
    return oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                 s["flatten_ids"], W, H, ts, backgrounds=s.get("backgrounds"), masks=s.get("masks"))


@pytest.mark.parametrize("I,N,W,H,ts,C,masks,opac", [
    (1, 3000, 256, 256, 16, 3, False, (0.05, 0.95)),
    (2, 1500, 200, 120, 16, 3, True, (0.05, 0.95)),
    (1, 2000, 100, 90, 8, 1, False, (0.5, 0.99)),
    (1, 1500, 96, 64, 16, 4, False, (0.05, 0.95)),
    (1, 1200, 90, 70, 16, 2, True, (0.05, 0.95)),   # two channels, ragged last tile strip, masked tiles
    (1, 800, 64, 48, 16, 5, False, (0.05, 0.95)),
    (2, 700, 80, 64, 16, 32, True, (0.05, 0.95)),  # any channel count, masked tiles, two images
    (1, 4000, 128, 128, 16, 3, False, (0.9, 0.99)),  # saturating: early termination
])
def test_forward_backward_vs_oracle(oracle, I, N, W, H, ts, C, masks, opac):
    g = gsplat()
    rng = np.random.default_rng(N + C)
    s = make_scene(oracle, rng, I, N, W, H, ts, C, opac=opac, masks=masks)
    got = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s), W, H, ts)
    exp = _oracle_fwd(oracle, s, W, H, ts)
    img_err = np.abs(host(got["render_colors"]) - exp["render_colors"]).max()
    assert img_err <= IMG_ATOL, f"image max-abs {img_err}"
    assert np.abs(host(got["render_alphas"]) - exp["render_alphas"]).max() <= IMG_ATOL
    li_mismatch = np.mean(host(got["last_ids"]) != exp["last_ids"])
    assert li_mismatch == 0.0, f"last_ids mismatch fraction {li_mismatch}"
    v_rc = rng.normal(size=exp["render_colors"].shape).astype(np.float32)
    v_ra = rng.normal(size=exp["render_alphas"].shape).astype(np.float32)
    bwd = g.rasterize_to_pixels_3dgs_backward(
        _raster_inputs(s), {"render_alphas": got["render_alphas"], "last_ids": got["last_ids"]},
        {"v_render_colors": dev(v_rc), "v_render_alphas": dev(v_ra)}, W, H, ts, absgrad=True)
    eb = oracle.raster_backward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                s["flatten_ids"], W, H, ts, exp["render_alphas"], exp["last_ids"], v_rc, v_ra,
                                backgrounds=s["backgrounds"], masks=s.get("masks"), absgrad=True)
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities", "v_backgrounds", "v_means2d_abs"):
        assert_close_rel(host(bwd[k]), eb[k], GRAD_RTOL, k)
    if I == 1 and C == 3 and not masks:
        # an absent v_render_alphas means zeros
        fo = {"render_alphas": got["render_alphas"], "last_ids": got["last_ids"]}
        z = g.rasterize_to_pixels_3dgs_backward(_raster_inputs(s), fo, {"v_render_colors": dev(v_rc),
                                                                        "v_render_alphas": dev(0 * v_ra)}, W, H, ts)
        n = g.rasterize_to_pixels_3dgs_backward(_raster_inputs(s), fo, {"v_render_colors": dev(v_rc)}, W, H, ts)
        for k in ("v_means2d", "v_conics", "v_colors", "v_opacities", "v_backgrounds"):
            assert_close_rel(host(n[k]), host(z[k]), 1e-5, k)


def test_empty_lists_and_no_background(oracle):
    g = gsplat()
    rng = np.random.default_rng(5)
    s = make_scene(oracle, rng, 1, 50, 64, 64, 16, 3)
    s["means2d"][...] = -1000.0  # nothing lands on screen in the raster (lists still reference them)
    s.pop("backgrounds")
    got = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s), 64, 64, 16)
    exp = _oracle_fwd(oracle, s, 64, 64, 16)
    np.testing.assert_allclose(host(got["render_colors"]), exp["render_colors"], atol=IMG_ATOL)
    empty = dict(s, flatten_ids=np.zeros(0, np.int32), tile_offsets=np.zeros((1, 4, 4), np.int32))
    got = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(empty), 64, 64, 16)
    assert np.all(host(got["render_colors"]) == 0) and np.all(host(got["render_alphas"]) == 0)


def test_non_finite_values_stay_local(oracle):
    """A non-finite colour reaches only the pixels that take its Gaussian, and
    a non-finite cotangent only the Gaussians that its pixel takes (the
    reference skips a record a pixel does not take): NaN / inf patterns equal
    the oracle's, and the finite values agree to the usual tolerances."""
    g = gsplat()
    rng = np.random.default_rng(77)
    W = H = 96
    s = make_scene(oracle, rng, 1, 1200, W, H, 16, 3)
    s["colors"][0, 5] = [np.inf, 0.5, 0.5]
    s["colors"][0, 17] = [0.2, np.nan, 0.1]
    got = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s), W, H, 16)
    exp = _oracle_fwd(oracle, s, W, H, 16)
    rc, erc = host(got["render_colors"]), exp["render_colors"]
    np.testing.assert_array_equal(np.isnan(rc), np.isnan(erc))
    np.testing.assert_array_equal(np.isinf(rc), np.isinf(erc))
    fin = np.isfinite(erc)
    assert fin.mean() > 0.5 and (~fin).any()
    assert np.abs(rc[fin] - erc[fin]).max() <= IMG_ATOL
    np.testing.assert_array_equal(host(got["last_ids"]), exp["last_ids"])

    s["colors"][0, 5] = [0.9, 0.5, 0.5]
    s["colors"][0, 17] = [0.2, 0.3, 0.1]
    got = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s), W, H, 16)
    exp = _oracle_fwd(oracle, s, W, H, 16)
    v_rc = rng.normal(size=exp["render_colors"].shape).astype(np.float32)
    v_rc[0, 40, 41, 0] = np.nan
    v_rc[0, 70, 12, 2] = np.inf
    v_ra = rng.normal(size=exp["render_alphas"].shape).astype(np.float32)
    bwd = g.rasterize_to_pixels_3dgs_backward(
        _raster_inputs(s), {"render_alphas": got["render_alphas"], "last_ids": got["last_ids"]},
        {"v_render_colors": dev(v_rc), "v_render_alphas": dev(v_ra)}, W, H, 16)
    eb = oracle.raster_backward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                s["flatten_ids"], W, H, 16, exp["render_alphas"], exp["last_ids"], v_rc, v_ra,
                                backgrounds=s["backgrounds"])
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities"):
        a, e = host(bwd[k]), eb[k]
        np.testing.assert_array_equal(np.isfinite(a), np.isfinite(e), err_msg=k)
        bad = ~np.isfinite(e)
        assert bad.any() and (~bad).mean() > 0.9, k
        assert_close_rel(np.where(bad, 0, a), np.where(bad, 0, e), GRAD_RTOL, k)


@pytest.mark.parametrize("I,N,W,H,ts,chunk", [(1, 2000, 200, 150, 16, None), (2, 3000, 131, 97, 16, 37),
                                               (1, 1500, 96, 64, 8, None)])
def test_rasterize_to_indices_vs_oracle(oracle, I, N, W, H, ts, chunk):
    """rasterize_to_indices_3dgs: the (gaussian, pixel) lists bit-exact with
    the oracle, for the full range and for a range chunk from carried
    transmittances."""
    rng = np.random.default_rng(N)
    s = make_scene(oracle, rng, I, N, W, H, ts, 3)
    g = gsplat()
    inp = {"means2d": dev(s["means2d"]), "conics": dev(s["conics"]), "opacities": dev(s["opacities"]),
           "tile_offsets": dev(s["tile_offsets"]), "flatten_ids": dev(s["flatten_ids"])}
    r0, r1 = (0, 2**40) if chunk is None else (chunk, 2 * chunk)
    trans = None
    if chunk is not None:
        trans = rng.uniform(0.2, 1.0, (I, H, W)).astype(np.float32)
        inp["transmittances"] = dev(trans)
    print(f"raster indices I={I} N={N} {W}x{H} ts={ts} chunk={chunk}", flush=True)
    out = g.rasterize_to_indices_3dgs_forward(inp, r0, r1, W, H, ts)
    eg, ei = oracle.raster_indices(s["means2d"], s["conics"], s["opacities"], s["tile_offsets"], s["flatten_ids"],
                                   W, H, ts, range_start=r0, range_end=r1, transmittances=trans)
    assert ei.size > 1000
    np.testing.assert_array_equal(host(out["indices"]), ei)
    np.testing.assert_array_equal(host(out["gaussian_ids"]), eg)


def test_exp_alpha_extremes():
    """The rasterizer's exp (C ABI probe): within 2 ulp of exp in float64 from
    -103 to 88, at most 2^-149 from -104 down (including the arguments where
    an unclamped float32 Cody-Waite reduction overflows: -3e9, -1e10,
    -FLT_MAX, -inf), and NaN for NaN."""
    import ctypes

    import torch

    from test_gpu_isect import LIB

    lib = ctypes.CDLL(LIB)
    lib.gsplat_hip_exp_alpha_eval.restype = ctypes.c_int
    lib.gsplat_hip_exp_alpha_eval.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    rng = np.random.default_rng(3)
    normal = np.concatenate([rng.uniform(-103, 88, 100_000), np.linspace(-103, 0, 4097)]).astype(np.float32)
    tiny = np.array([-104, -150, -1e3, -2.9e9, -3e9, -1e10, -3.4028235e38, -np.inf], np.float32)
    tiny = np.concatenate([tiny, -np.exp(rng.uniform(np.log(104), np.log(3e38), 10_000)).astype(np.float32)])
    y = np.concatenate([normal, tiny, np.array([np.nan], np.float32)])
    yd = dev(y)
    out = torch.empty_like(yd)
    assert lib.gsplat_hip_exp_alpha_eval(yd.data_ptr(), y.size, out.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    got = host(out)
    a, b = normal.size, normal.size + tiny.size
    want = np.exp(normal.astype(np.float64))
    assert np.all(np.abs(got[:a] - want) <= 2 * np.spacing(want.astype(np.float32)).astype(np.float64))
    t = got[a:b]
    assert np.all((t >= 0) & (t <= 2.0 ** -149)), t[~((t >= 0) & (t <= 2.0 ** -149))][:5]
    assert np.isnan(got[b])


def test_ill_conditioned_records_far_from_the_mean(oracle):
    """Records the per-wave cull never drops (conics with det <= 1e-4 c0 c2)
    reach pixels where sigma is about 5e9 and where it is +inf; the
    reference's exp gives 0 there and skips them. A NaN conic gives the
    reference's std::min(0.99, NaN) = 0.99 alpha with no geometry gradient.
    Images, last_ids and gradients equal the oracle's."""
    g = gsplat()
    rng = np.random.default_rng(9)
    W = H = 48
    ts = 16
    s = make_scene(oracle, rng, 1, 300, W, H, ts, 3)
    n0 = s["means2d"].shape[1]
    special_m = np.array([[8.5, 9.0], [24.5, 30.0], [40.0, 40.0], [8.5, 40.0]], np.float32)
    b1 = np.float32(np.sqrt(1e8 * (1 - 5e-5)))
    b2 = np.float32(np.sqrt(3e38 * (1 - 5e-5)))
    special_c = np.array([[1e8, b1, 1.0],        # sigma ~ 5e9 ten pixels off its column
                          [3e38, b2, 1.0],       # sigma = +inf two pixels off its column
                          [np.nan, 0.0, 0.5],    # NaN conic: alpha 0.99
                          [1e8, -b1, 1.0]], np.float32)
    special_r = np.array([[40, 40], [40, 40], [4, 4], [40, 40]], np.int32)
    means2d = np.concatenate([s["means2d"], special_m[None]], 1)
    conics = np.concatenate([s["conics"], special_c[None]], 1)
    colors = np.concatenate([s["colors"], rng.uniform(0, 1, (1, 4, 3)).astype(np.float32)], 1)
    opac = np.concatenate([s["opacities"], np.array([[0.9, 0.8, 0.7, 0.95]], np.float32)], 1)
    # radii and depths: the scene's lists plus the special records (deepest)
    A_cov = np.linalg.inv(np.stack([np.stack([s["conics"][..., 0], s["conics"][..., 1]], -1),
                                    np.stack([s["conics"][..., 1], s["conics"][..., 2]], -1)], -2))
    radii = np.ceil(3.33 * np.sqrt(np.stack([A_cov[..., 0, 0], A_cov[..., 1, 1]], -1))).astype(np.int32)
    radii = np.concatenate([radii, special_r[None]], 1)
    depths = np.concatenate([rng.uniform(1, 10, (1, n0)), np.array([[11.0, 12.0, 13.0, 14.0]])], 1).astype(np.float32)
    tw = th = W // ts
    isect = oracle.isect_tile(means2d, radii, depths, 1, ts, tw, th)
    offs = oracle.isect_offset(isect["isect_ids"], 1, tw, th)
    s2 = dict(means2d=means2d, conics=conics, colors=colors, opacities=opac, backgrounds=s["backgrounds"],
              tile_offsets=offs, flatten_ids=isect["flatten_ids"])
    got = g.rasterize_to_pixels_3dgs_forward(_raster_inputs(s2), W, H, ts)
    exp = _oracle_fwd(oracle, s2, W, H, ts)
    assert np.abs(host(got["render_colors"]) - exp["render_colors"]).max() <= IMG_ATOL
    assert np.abs(host(got["render_alphas"]) - exp["render_alphas"]).max() <= IMG_ATOL
    np.testing.assert_array_equal(host(got["last_ids"]), exp["last_ids"])
    # the special records do take some pixels (their own columns / the NaN tile)
    fid = isect["flatten_ids"]
    assert all(np.isin(np.flatnonzero(fid == n0 + k), exp["last_ids"].ravel()).any() for k in (0, 2, 3))
    v_rc = rng.normal(size=exp["render_colors"].shape).astype(np.float32)
    v_ra = rng.normal(size=exp["render_alphas"].shape).astype(np.float32)
    bwd = g.rasterize_to_pixels_3dgs_backward(
        _raster_inputs(s2), {"render_alphas": got["render_alphas"], "last_ids": got["last_ids"]},
        {"v_render_colors": dev(v_rc), "v_render_alphas": dev(v_ra)}, W, H, ts, absgrad=True)
    eb = oracle.raster_backward(means2d, conics, colors, opac, offs, isect["flatten_ids"], W, H, ts,
                                exp["render_alphas"], exp["last_ids"], v_rc, v_ra, backgrounds=s["backgrounds"],
                                absgrad=True)
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities", "v_backgrounds", "v_means2d_abs"):
        a, e = host(bwd[k]), eb[k]
        np.testing.assert_array_equal(np.isfinite(a), np.isfinite(e), err_msg=k)
        assert_close_rel(np.where(np.isfinite(e), a, 0), np.where(np.isfinite(e), e, 0), GRAD_RTOL, k)


@pytest.mark.parametrize("I,N,W,H,ts,masks,opac", [(1, 3000, 256, 256, 16, False, (0.05, 0.95)),
                                                   (2, 1500, 200, 120, 16, True, (0.05, 0.95)),
                                                   (1, 4000, 128, 128, 16, False, (0.9, 0.99)),
                                                   (1, 2000, 100, 90, 8, False, (0.5, 0.99))])
def test_count_evals_vs_oracle(oracle, I, N, W, H, ts, masks, opac):
    """gsplat_hip_rasterize_count_evals (E_f, the forward loop's evaluations up
    to each pixel's termination, per tile) equals the oracle's count of its
    own forward loop, tile for tile, with masks, several images, saturating
    scenes and 8-pixel tiles."""
    import ctypes
    import os

    import torch

    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gsplat-mlx_amd",
                                   "gsplat_core", "libgsplat_hip.so"))
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.gsplat_hip_rasterize_count_evals.argtypes = [P, P, P, P, P, P, I64, I64, I32, I32, I32, I32, I32, I64, P, P]
    rng = np.random.default_rng(N + 7)
    s = make_scene(oracle, rng, I, N, W, H, ts, 3, opac=opac, masks=masks)
    exp = _oracle_fwd(oracle, s, W, H, ts)
    th, tw = s["tile_offsets"].shape[-2:]
    t = {k: dev(v) for k, v in s.items() if k in ("means2d", "conics", "opacities", "tile_offsets", "flatten_ids")}
    mk = dev(s["masks"].astype(np.uint8)) if masks else None
    out = torch.zeros(I * th * tw, dtype=torch.int64, device="cuda")
    print(f"count evals I={I} N={N} {W}x{H} ts={ts}", flush=True)
    rc = lib.gsplat_hip_rasterize_count_evals(
        t["means2d"].data_ptr(), t["conics"].data_ptr(), t["opacities"].data_ptr(), mk.data_ptr() if masks else None,
        t["tile_offsets"].data_ptr(), t["flatten_ids"].data_ptr(), I, I * N, W, H, ts, tw, th,
        s["flatten_ids"].size, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(out).reshape(I, th, tw), exp["tile_evals"])
    assert exp["tile_evals"].sum() > 0
