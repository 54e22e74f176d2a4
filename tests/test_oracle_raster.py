"""Pins the oracle's rasterizer: the reference's closed forms and mask cases
(gsplat_core/test/test.cpp:1067-1386), a brute-force float64 compositing
restatement written with numpy, float64 finite differences for every backward
output, and the closed-form background gradient sum_p T_final * v_rc
(scripts/export_ref/export_rasterize_to_pixels_3dgs_backward.py:91)."""
import numpy as np
import pytest

ALPHA_T = 1 / 255


def single_gaussian_inputs():
    return dict(means2d=np.array([[[1.0, 1.0]]], np.float32), conics=np.array([[[1.0, 0.0, 1.0]]], np.float32),
                colors=np.array([[[1.0, 0.0, 0.0]]], np.float32), opacities=np.array([[0.5]], np.float32),
                backgrounds=np.array([[0.1, 0.2, 0.3]], np.float32))


def test_single_gaussian_closed_form(oracle):
    # test.cpp:1067-1131
    inp = single_gaussian_inputs()
    out = oracle.raster_forward(inp["means2d"], inp["conics"], inp["colors"], inp["opacities"],
                                np.zeros((1, 1, 1), np.int32), np.zeros(1, np.int32), 2, 2, 2,
                                backgrounds=inp["backgrounds"])
    a = 0.5 * np.exp(-0.25)
    assert out["render_colors"].shape == (1, 2, 2, 3) and out["last_ids"].shape == (1, 2, 2)
    np.testing.assert_allclose(out["render_alphas"].ravel(), a, atol=1e-5)
    np.testing.assert_allclose(out["render_colors"].reshape(4, 3), [[a + (1 - a) * 0.1, (1 - a) * 0.2, (1 - a) * 0.3]] * 4, atol=1e-5)
    assert np.all(out["last_ids"] == 0)


def test_tile_masks(oracle):
    # test.cpp:1199-1271
    inp = single_gaussian_inputs()
    out = oracle.raster_forward(inp["means2d"], inp["conics"], inp["colors"], inp["opacities"],
                                np.array([[[0, 1]]], np.int32), np.zeros(1, np.int32), 4, 2, 2,
                                backgrounds=inp["backgrounds"], masks=np.array([[[True, False]]]))
    a = 0.5 * np.exp(-0.25)
    rc = out["render_colors"][0]
    ra = out["render_alphas"][0, :, :, 0]
    np.testing.assert_allclose(ra[:, :2], a, atol=1e-5)
    np.testing.assert_allclose(ra[:, 2:], 0, atol=1e-7)
    np.testing.assert_allclose(rc[:, 2:], np.broadcast_to([0.1, 0.2, 0.3], (2, 2, 3)), atol=1e-6)
    assert np.all(out["last_ids"] == 0)


def make_scene(oracle, rng, I=2, N=60, W=40, H=28, ts=8, C=3, dtype=np.float64, mean_opac=(0.3, 0.9)):
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    means2d = np.stack([rng.uniform(0, W, (I, N)), rng.uniform(0, H, (I, N))], -1)
    A = rng.normal(size=(I, N, 2, 2)) * 3
    cov = A @ np.swapaxes(A, -1, -2) + 2 * np.eye(2)
    inv = np.linalg.inv(cov)
    conics = np.stack([inv[..., 0, 0], inv[..., 0, 1], inv[..., 1, 1]], -1)
    colors = rng.uniform(0, 1, (I, N, C))
    opac = rng.uniform(*mean_opac, (I, N))
    radii = np.ceil(3.33 * np.sqrt(np.stack([cov[..., 0, 0], cov[..., 1, 1]], -1))).astype(np.int32)
    depths = rng.uniform(1, 10, (I, N)).astype(np.float32)
    isect = oracle.isect_tile(means2d.astype(np.float32), radii, depths, I, ts, tw, th)
    offs = oracle.isect_offset(isect["isect_ids"], I, tw, th)
    bg = rng.uniform(0, 0.3, (I, C))
    return dict(means2d=means2d.astype(dtype), conics=conics.astype(dtype), colors=colors.astype(dtype),
                opacities=opac.astype(dtype), backgrounds=bg.astype(dtype), tile_offsets=offs,
                flatten_ids=isect["flatten_ids"], W=W, H=H, ts=ts)


def brute_force_render(s):
    """Per-pixel front-to-back compositing over the pixel's tile list (numpy)."""
    I, H, W = s["tile_offsets"].shape[0], s["H"], s["W"]
    C = s["colors"].shape[-1]
    ts = s["ts"]
    th, tw = s["tile_offsets"].shape[1:]
    offs = s["tile_offsets"].ravel()
    fl = s["flatten_ids"]
    m2 = s["means2d"].reshape(-1, 2)
    co = s["conics"].reshape(-1, 3)
    cl = s["colors"].reshape(-1, C)
    op = s["opacities"].ravel()
    img = np.zeros((I, H, W, C))
    alp = np.zeros((I, H, W))
    for i in range(I):
        for y in range(H):
            for x in range(W):
                t = i * tw * th + (y // ts) * tw + x // ts
                end = offs[t + 1] if t + 1 < offs.size else fl.size
                g = fl[offs[t]:end]
                dx = m2[g, 0] - (x + 0.5)
                dy = m2[g, 1] - (y + 0.5)
                sig = 0.5 * (co[g, 0] * dx * dx + co[g, 2] * dy * dy) + co[g, 1] * dx * dy
                a = np.minimum(0.99, op[g] * np.exp(-sig))
                T = 1.0
                for k in np.nonzero((sig >= 0) & (a >= ALPHA_T))[0]:
                    if T * (1 - a[k]) <= 1e-4:
                        break
                    img[i, y, x] += cl[g[k]] * a[k] * T
                    T *= 1 - a[k]
                alp[i, y, x] = 1 - T
                img[i, y, x] += T * s["backgrounds"][i]
    return img, alp


def test_brute_force_compositing(oracle):
    rng = np.random.default_rng(0)
    s = make_scene(oracle, rng)
    out = oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                s["flatten_ids"], s["W"], s["H"], s["ts"], backgrounds=s["backgrounds"])
    img, alp = brute_force_render(s)
    np.testing.assert_allclose(out["render_colors"], img, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(out["render_alphas"][..., 0], alp, rtol=1e-12, atol=1e-13)


def test_early_termination_matches_brute_force(oracle):
    rng = np.random.default_rng(1)
    s = make_scene(oracle, rng, N=300, mean_opac=(0.95, 0.99))
    out = oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                s["flatten_ids"], s["W"], s["H"], s["ts"], backgrounds=s["backgrounds"])
    img, alp = brute_force_render(s)
    assert np.mean(out["render_alphas"] > 0.999) > 0.2  # termination is exercised
    np.testing.assert_allclose(out["render_colors"], img, rtol=1e-12, atol=1e-13)


def _loss(oracle, s, v_rc, v_ra, **over):
    t = dict(s, **over)
    out = oracle.raster_forward(t["means2d"], t["conics"], t["colors"], t["opacities"], t["tile_offsets"],
                                t["flatten_ids"], t["W"], t["H"], t["ts"], backgrounds=t["backgrounds"])
    return np.sum(out["render_colors"] * v_rc) + np.sum(out["render_alphas"] * v_ra), out["last_ids"]


@pytest.mark.parametrize("seed", [2, 3])
def test_backward_finite_differences(oracle, seed):
    rng = np.random.default_rng(seed)
    s = make_scene(oracle, rng, I=1, N=12, W=24, H=16, mean_opac=(0.3, 0.8))
    fwd = oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                s["flatten_ids"], s["W"], s["H"], s["ts"], backgrounds=s["backgrounds"])
    v_rc = rng.normal(size=fwd["render_colors"].shape)
    v_ra = rng.normal(size=fwd["render_alphas"].shape)
    bwd = oracle.raster_backward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                 s["flatten_ids"], s["W"], s["H"], s["ts"], fwd["render_alphas"], fwd["last_ids"],
                                 v_rc, v_ra, backgrounds=s["backgrounds"], absgrad=True)
    h = 1e-7
    for name in ("means2d", "conics", "colors", "opacities", "backgrounds"):
        arr = s[name]
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            a0 = arr[idx]
            arr[idx] = a0 + h
            lp, li_p = _loss(oracle, s, v_rc, v_ra)
            arr[idx] = a0 - h
            lm, li_m = _loss(oracle, s, v_rc, v_ra)
            arr[idx] = a0
            assert np.array_equal(li_p, li_m)  # no discrete change under the perturbation
            num[idx] = (lp - lm) / (2 * h)
        np.testing.assert_allclose(bwd["v_" + name], num, rtol=1e-5, atol=1e-7 * max(1, np.abs(num).max()),
                                   err_msg=name)
    # closed-form background gradient and absgrad >= |grad|
    T_final = 1 - fwd["render_alphas"]
    np.testing.assert_allclose(bwd["v_backgrounds"], np.sum(T_final * v_rc, axis=(1, 2)), rtol=1e-12)
    assert np.all(bwd["v_means2d_abs"] >= np.abs(bwd["v_means2d"]) - 1e-12)


def test_tile_evals_pins(oracle):
    """The oracle's per-tile E_f (the forward loop's iterations up to each
    pixel's termination) on known answers: a lone Gaussian never saturates a
    pixel, so every pixel evaluates the whole list; two opaque flat Gaussians
    saturate every pixel at the second entry (T = (1 - 0.99)^2 < 1e-4), so
    each pixel evaluates 2 of 4; a masked tile evaluates nothing. On a random
    scene: a tile whose pixels all end with transmittance above 1e-2 (none can
    have stopped: alpha <= 0.99) evaluates pixels x list length, and every
    tile lies between its pixels' replayed prefixes (last_id - start + 1) and
    pixels x list length."""
    flat = np.array([[[1.0e-6, 0.0, 1.0e-6]]], np.float32)
    for n, per_pixel in ((1, 1), (4, 2)):
        s = dict(means2d=np.full((1, n, 2), 8.0, np.float32), conics=np.repeat(flat, n, 1),
                 colors=np.ones((1, n, 3), np.float32), opacities=np.ones((1, n), np.float32))
        offs = np.array([[[0, n]]], np.int32)
        out = oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], offs,
                                    np.arange(n, dtype=np.int32), 32, 16, 16,
                                    masks=np.array([[[True, False]]]))
        assert out["tile_evals"].tolist() == [[[256 * per_pixel, 0]]]
    rng = np.random.default_rng(3)
    from test_gpu_raster import make_scene

    I, W, H, ts = 1, 160, 96, 16
    s = make_scene(oracle, rng, I, 300, W, H, ts, 3, opac=(0.3, 0.99))
    out = oracle.raster_forward(s["means2d"], s["conics"], s["colors"], s["opacities"], s["tile_offsets"],
                                s["flatten_ids"], W, H, ts)
    th, tw = s["tile_offsets"].shape[-2:]
    offs = s["tile_offsets"].ravel().astype(np.int64)
    ends = np.append(offs[1:], s["flatten_ids"].size)
    alphas = out["render_alphas"][0, :, :, 0]
    last = out["last_ids"][0]
    saturated = unsaturated = 0
    for ty in range(th):
        for tx in range(tw):
            k = ty * tw + tx
            n = ends[k] - offs[k]
            a = alphas[ty * ts:(ty + 1) * ts, tx * ts:(tx + 1) * ts]
            li = last[ty * ts:(ty + 1) * ts, tx * ts:(tx + 1) * ts]
            ev = out["tile_evals"][0, ty, tx]
            replayed = np.where(a > 0, li - offs[k] + 1, 0).sum()
            assert replayed <= ev <= a.size * n
            # a pixel that stops at an entry of alpha <= 0.99 ends with T <= 1e-4 / 0.01
            if (1.0 - a).min() > 0.0101:
                assert ev == a.size * n
                unsaturated += 1
            else:
                saturated += 1
    assert saturated > 0 and unsaturated > 0
