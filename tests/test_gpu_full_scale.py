"""Full-size parity for the three SH-degree-3 workloads:
- sh3_1m: 1M Gaussians, one 1297x840 camera, about 5.4M intersections;
- multiview_3m: 3M Gaussians, 8 cameras on a ring at 1920x1080 (one
  projection call with C = 8, eight images, gradients summed over cameras);
- heavy_6m: 6M Gaussians at 3840x2160, large splats, about 250M
  intersections.

The oracle cannot replay these frames whole in test time, so each stage is
checked where exact parity is cheap, on the GPU's full-size run:
- projection and the fused SH colours, forward and backward, on a random
  subset of Gaussians (these VJPs are per Gaussian) against the oracle;
- intersection: keys non-decreasing, each Gaussian listed tiles_per_gauss
  times, offsets equal to the lower bounds of the keys, and the complete
  lists of sampled tiles (the heaviest and random ones) against the
  reference's tile rectangle (gsplat_intersect.cpp:67-99, restated in numpy
  and pinned here against the oracle's counts) in stable depth order;
- rasterization forward and backward on the sampled tiles: the GPU runs the
  full frame with every other tile masked; the oracle runs the same tiles'
  lists as one compacted problem. Images within 1e-4 max-abs, last
  contributors exact, gradients within 1e-3 relative, every Gaussian outside
  the sampled lists with zero gradient.
"""
import numpy as np
import pytest

from _helpers import FLOOR_ORDERED, MAX_RADIUS_FLIPS, assert_close_rel, dev, gsplat, host
from test_gpu_sh_camera import _oracle_backward as sh_oracle_backward
from test_gpu_sh_camera import _oracle_forward as sh_oracle_forward

pytestmark = pytest.mark.gpu

FWD_RTOL = 1e-5
GRAD_RTOL = 1e-3
IMG_ATOL = 1e-4
EPS2D, NEAR = 0.3, 0.01


def _campos(vm):
    """-R^T t with the kernels' float32 operation order."""
    R, t = vm[..., :3, :3], vm[..., :3, 3]
    c = np.empty(vm.shape[:-2] + (3,), np.float32)
    for i in range(3):
        c[..., i] = -((R[..., 0, i] * t[..., 0] + R[..., 1, i] * t[..., 1]) + R[..., 2, i] * t[..., 2])
    return c


def _tile_rects(means2d, radii, ts, tw, th):
    """gsplat_intersect.cpp:67-99 in float32: [min_x, min_y, max_x, max_y)."""
    f = np.float32
    trx = radii[..., 0].astype(f) / f(ts)
    try_ = radii[..., 1].astype(f) / f(ts)
    tx = means2d[..., 0] / f(ts)
    ty = means2d[..., 1] / f(ts)
    ok = (radii[..., 0] > 0) & (radii[..., 1] > 0)
    r = [np.clip(np.floor(tx - trx), 0, tw), np.clip(np.floor(ty - try_), 0, th),
         np.clip(np.ceil(tx + trx), 0, tw), np.clip(np.ceil(ty + try_), 0, th)]
    return [np.where(ok, v, 0).astype(np.int64) for v in r]


def _run(name, oracle, n_sub=3000, n_heavy=3, n_random=3):
    import torch

    from gsplat_core.scenes import make_scene

    g = gsplat()
    torch.manual_seed(0)
    sc = make_scene(name, seed=0, with_target=False)
    W, H, ts = sc.width, sc.height, sc.tile_size
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    N, C = sc.n, sc.n_cameras
    rng = np.random.default_rng(123)
    print(f"[full-scale] {name}: N={N} C={C} {W}x{H}", flush=True)

    quats = (sc.quats / np.linalg.norm(sc.quats, axis=-1, keepdims=True)).astype(np.float32)
    scales = np.exp(sc.log_scales).astype(np.float32)
    opac = (1.0 / (1.0 + np.exp(-sc.opacity_logits.astype(np.float64)))).astype(np.float32)  # [1, N]
    vm, Ks = sc.viewmats, sc.Ks
    sub = np.sort(rng.choice(N, n_sub, replace=False))

    # ---- projection, forward and backward, on a subset
    inputs = {"means": dev(sc.means), "quats": dev(quats), "scales": dev(scales), "viewmats": dev(vm),
              "Ks": dev(Ks)}
    pk = dict(eps2d=EPS2D, near_plane=NEAR, far_plane=sc.far_plane)
    proj = g.projection_ewa_3dgs_fused_forward(inputs, W, H, **pk)
    e = oracle.projection_forward(sc.means[:, sub], vm, Ks, W, H, quats=quats[:, sub], scales=scales[:, sub], **pk)
    r_got = host(proj["radii"][:, :, sub])
    flips = np.sum(np.any(r_got != e["radii"], axis=-1))
    print(f"[full-scale] radius flips on the {n_sub}-Gaussian subset: {flips}", flush=True)
    assert flips <= MAX_RADIUS_FLIPS, f"{flips} radius mismatches"
    both = np.all(r_got > 0, -1) & np.all(e["radii"] > 0, -1)
    assert both.sum() > 100
    for k in ("means2d", "conics", "depths"):
        assert_close_rel(host(proj[k][:, :, sub])[both], e[k][both], FWD_RTOL, k, floor_rel=FLOOR_ORDERED)
    cot = {"v_means2d": torch.randn(proj["means2d"].shape, device="cuda"),
           "v_depths": torch.randn(proj["depths"].shape, device="cuda"),
           "v_conics": torch.randn(proj["conics"].shape, device="cuda")}
    pb = g.projection_ewa_3dgs_fused_backward(inputs, {"radii": proj["radii"], "conics": proj["conics"]}, cot, W, H,
                                              eps2d=EPS2D)
    eb = oracle.projection_backward(sc.means[:, sub], vm, Ks, W, H, r_got, host(proj["conics"][:, :, sub]),
                                    host(cot["v_means2d"][:, :, sub]), host(cot["v_depths"][:, :, sub]),
                                    host(cot["v_conics"][:, :, sub]), quats=quats[:, sub], scales=scales[:, sub],
                                    eps2d=EPS2D)
    for k in ("v_means", "v_quats", "v_scales"):
        assert_close_rel(host(pb[k][:, sub]), eb[k], GRAD_RTOL, k, floor_rel=FLOOR_ORDERED)
    del pb, cot
    print("[full-scale] projection ok", flush=True)

    # ---- fused SH colours (C cameras), forward and backward, on a subset
    shin = {"means": inputs["means"], "viewmats": inputs["viewmats"], "features_dc": dev(sc.features_dc),
            "features_rest": dev(sc.features_rest)}
    colors = g._gsplat_core.sh_camera_colors_forward(sc.sh_degree, shin)  # [1, C, N, 3]
    campos = _campos(vm)
    raw, dirs, norms, coeffs = sh_oracle_forward(oracle, sc.sh_degree, sc.means[:, sub], campos,
                                                 sc.features_dc[:, sub], sc.features_rest[:, sub])
    x = raw + 0.5
    keep = ~np.any((np.abs(x) < 1e-4) | (np.abs(x - 1) < 1e-4), axis=(1, 3))[0]  # away from the clip bounds
    assert keep.mean() > 0.99
    assert_close_rel(host(colors[:, :, sub])[:, :, keep], np.clip(x, 0, 1)[:, :, keep], FWD_RTOL, "colors", floor_rel=FLOOR_ORDERED)
    v_colors = torch.randn(colors.shape, device="cuda")
    sb = g._gsplat_core.sh_camera_colors_backward(sc.sh_degree, shin, {"v_colors": v_colors})
    ev_means, ev_dc, ev_rest = sh_oracle_backward(oracle, sc.sh_degree, sc.means[:, sub], campos, coeffs, raw, dirs,
                                                  norms, host(v_colors[:, :, sub]), sc.features_rest.shape[2])
    assert_close_rel(host(sb["v_features_dc"][:, sub])[:, keep], ev_dc[:, keep], GRAD_RTOL, "v_features_dc", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(sb["v_features_rest"][:, sub])[:, keep], ev_rest[:, keep], GRAD_RTOL, "v_features_rest", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(sb["v_means"][:, sub])[:, keep], ev_means[:, keep], GRAD_RTOL, "v_means", floor_rel=FLOOR_ORDERED)
    del sb, v_colors
    print("[full-scale] SH colours ok", flush=True)

    # ---- intersection (I = C images)
    out = g.intersect_tile_forward({"means2d": proj["means2d"], "radii": proj["radii"], "depths": proj["depths"]},
                                   C, ts, tw, th)
    keys, flat = out["isect_ids"], out["flatten_ids"]
    M = keys.numel()
    tpg = out["tiles_per_gauss"].reshape(-1)
    assert M == int(tpg.long().sum())
    assert bool(torch.all(keys[1:] >= keys[:-1]))
    counts = torch.bincount(flat.long(), minlength=C * N)
    assert torch.equal(counts.to(torch.int32), tpg)
    del counts
    # the same frame again, with the offsets: the second call of a shape
    # speculates the scatter and tile sort from the first's M (or, for a
    # frame whose long lists chose the depth-presorted path, goes there
    # without the bucket count); the lists must not change
    from gsplat_core import _gsplat_core as _C

    again = _C.intersect_tile_offsets_forward({"means2d": proj["means2d"], "radii": proj["radii"],
                                               "depths": proj["depths"]}, C, ts, tw, th)
    assert torch.equal(again["isect_ids"], keys) and torch.equal(again["flatten_ids"], flat)
    assert torch.equal(again["tiles_per_gauss"].reshape(-1), tpg)
    offs_again = again["tile_offsets"]
    del again
    offs_t = g.intersect_offset_forward(keys, C, tw, th)  # [C, th, tw]
    assert torch.equal(offs_again, offs_t)
    del offs_again
    tile_bits = int(np.floor(np.log2(tw * th))) + 1
    img = torch.arange(C, device="cuda", dtype=torch.int64)[:, None]
    tl = torch.arange(tw * th, device="cuda", dtype=torch.int64)[None, :]
    want = (img << tile_bits) | tl
    lb = torch.searchsorted(keys >> 32, want.reshape(-1), right=False)
    assert torch.equal(offs_t.reshape(-1).long(), lb)
    del lb, want
    offs = host(offs_t).reshape(C, th * tw).astype(np.int64)
    ends = np.append(offs.reshape(-1)[1:], M).reshape(C, th * tw)
    lens = ends - offs
    print(f"[full-scale] M={M} max list {lens.max()}", flush=True)

    # sampled tiles: the heaviest and random interior ones per image
    sampled = []
    interior = np.array([t for t in range(tw * th) if 0 < t % tw < tw - 1 and 0 < t // tw < th - 1])
    for i in range(C):
        heavy = np.argsort(-lens[i])[:n_heavy]
        rand = rng.choice(interior, n_random, replace=False)
        sampled += [(i, int(t)) for t in np.unique(np.concatenate([heavy, rand]))]
    m2_h, r_h, d_h = host(proj["means2d"])[0], host(proj["radii"])[0], host(proj["depths"])[0]  # [C, N, ...]
    # the numpy rectangle restatement agrees with the oracle's per-Gaussian counts
    rx0, ry0, rx1, ry1 = _tile_rects(m2_h[0, sub], r_h[0, sub], ts, tw, th)
    np.testing.assert_array_equal((rx1 - rx0) * (ry1 - ry0), oracle.isect_count(m2_h[0, sub], r_h[0, sub], ts, tw, th))
    flat_h = {}
    for i, t in sampled:
        x0, y0, x1, y1 = _tile_rects(m2_h[i], r_h[i], ts, tw, th)
        tx, ty = t % tw, t // tw
        members = np.nonzero((x0 <= tx) & (tx < x1) & (y0 <= ty) & (ty < y1))[0]
        dbits = d_h[i, members].view(np.uint32)
        exp_list = (i * N + members[np.lexsort((members, dbits))]).astype(np.int32)
        got_list = host(flat[offs[i, t]:ends[i, t]])
        np.testing.assert_array_equal(got_list, exp_list, err_msg=f"tile list (image {i}, tile {t})")
        flat_h[(i, t)] = got_list
    print(f"[full-scale] {len(sampled)} tile lists ok", flush=True)

    # ---- rasterization on the sampled tiles
    opac_img = np.broadcast_to(opac[:, None, :], (1, C, N))
    opac_d = dev(np.array(opac_img))  # a writable copy
    bg = np.tile(np.array(sc.background, np.float32), (C, 1))
    masks = np.zeros((C, th, tw), bool)
    for i, t in sampled:
        masks[i, t // tw, t % tw] = True
    rin = {"means2d": proj["means2d"], "conics": proj["conics"], "colors": colors, "opacities": opac_d,
           "backgrounds": dev(bg), "masks": dev(masks), "tile_offsets": offs_t, "flatten_ids": flat}
    fwd = g.rasterize_to_pixels_3dgs_forward(rin, W, H, ts)
    v_rc = torch.randn(fwd["render_colors"].shape, device="cuda")
    v_ra = torch.randn(fwd["render_alphas"].shape, device="cuda")
    bwd = g.rasterize_to_pixels_3dgs_backward(rin, {"render_alphas": fwd["render_alphas"],
                                                    "last_ids": fwd["last_ids"]},
                                              {"v_render_colors": v_rc, "v_render_alphas": v_ra}, W, H, ts)

    # the oracle's compacted problem: the sampled lists with Gaussian ids
    # renumbered over the Gaussians they use, every other tile empty
    uniq = np.unique(np.concatenate(list(flat_h.values())))
    U = uniq.size
    Nc = (U + C - 1) // C
    pad = C * Nc - U

    def compact(t, width):
        a = host(t).reshape(C * N, width)[uniq]
        return np.concatenate([a, np.zeros((pad, width), a.dtype)]).reshape(C, Nc, width)

    m2c, conc, colc = compact(proj["means2d"], 2), compact(proj["conics"], 3), compact(colors, 3)
    opc = compact(opac_d, 1)[..., 0]
    offs_c = np.zeros(C * th * tw, np.int32)
    lists, pos = [], 0
    for idx in range(C * th * tw):
        offs_c[idx] = pos
        i, t = divmod(idx, th * tw)
        if (i, t) in flat_h:
            lists.append(np.searchsorted(uniq, flat_h[(i, t)]).astype(np.int32))
            pos += lists[-1].size
    flat_c = np.concatenate(lists)
    offs_c = offs_c.reshape(C, th, tw)
    ef = oracle.raster_forward(m2c, conc, colc, opc, offs_c, flat_c, W, H, ts, backgrounds=bg)
    rc, ra, li = host(fwd["render_colors"]), host(fwd["render_alphas"]), host(fwd["last_ids"])
    for i, t in sampled:
        ys = slice((t // tw) * ts, min(H, (t // tw + 1) * ts))
        xs = slice((t % tw) * ts, min(W, (t % tw + 1) * ts))
        err = np.abs(rc[i, ys, xs] - ef["render_colors"][i, ys, xs]).max()
        assert err <= IMG_ATOL, f"image (image {i}, tile {t}) max-abs {err}"
        assert np.abs(ra[i, ys, xs] - ef["render_alphas"][i, ys, xs]).max() <= IMG_ATOL
        rel_g = li[i, ys, xs].astype(np.int64) - offs[i, t]
        rel_o = ef["last_ids"][i, ys, xs].astype(np.int64) - offs_c[i, t // tw, t % tw]
        np.testing.assert_array_equal(np.maximum(rel_g, -1), np.maximum(rel_o, -1),
                                      err_msg=f"last contributors (image {i}, tile {t})")
    eb = oracle.raster_backward(m2c, conc, colc, opc, offs_c, flat_c, W, H, ts, ef["render_alphas"], ef["last_ids"],
                                host(v_rc), host(v_ra), backgrounds=bg, masks=masks)
    for k, width in (("v_means2d", 2), ("v_conics", 3), ("v_colors", 3), ("v_opacities", 1)):
        got = bwd[k].reshape(C * N, width)
        assert_close_rel(host(got)[uniq], eb[k].reshape(C * Nc, width)[:U], GRAD_RTOL, k)
        outside = torch.ones(C * N, dtype=torch.bool, device="cuda")
        outside[torch.from_numpy(uniq).cuda()] = False
        assert int(torch.count_nonzero(got[outside])) == 0, f"{k}: gradient outside the sampled lists"
    assert_close_rel(host(bwd["v_backgrounds"]), eb["v_backgrounds"], GRAD_RTOL, "v_backgrounds")
    print(f"[full-scale] raster ok on {len(sampled)} tiles ({U} Gaussians)", flush=True)


def test_sh3_1m_full_size(oracle):
    _run("sh3_1m", oracle)


def test_multiview_3m_full_size(oracle):
    _run("multiview_3m", oracle)


def test_heavy_6m_full_size(oracle):
    _run("heavy_6m", oracle, n_heavy=6, n_random=10)
