"""Pins the oracle's ellipse ("AccuTile") tile intersection.

No fixture of upstream gsplat's AccuTile ids exists in the reference tree, so
the oracle is pinned by what the geometry fixes:
  * a hand-computed known answer (a circle that misses the corner tiles of
    its AABB rect);
  * conservativeness: every pixel whose float32 alpha passes the rasterizer's
    test (gsplat_rasterize.cpp:304-313: sigma >= 0 and alpha >= 1/255) lies in
    a listed tile of its Gaussian, by brute force over all pixels;
  * tightness: a listed tile's pixel-centre rectangle comes within the slack
    ellipse sigma <= 1.05 ln(255 o) + 1e-4, and every rect tile that comes
    within it by a margin is listed -- the minimum of sigma over the
    rectangle is computed in float64 by a different formulation (interior,
    then the four edges) than the oracle's per-row x-extent;
  * structure: a subset of the AABB lists in the same row-major order;
  * rendering identity: the oracle rasterizer gives the same images and
    gradients from the AccuTile lists as from the AABB lists.
"""
import numpy as np
import pytest

from _helpers import projected_scene

TS = 16


def _rect(oracle, means, radii, W, H):
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    m = means.reshape(-1, 2)
    r = radii.reshape(-1, 2)
    rects = []
    for i in range(m.shape[0]):
        if r[i, 0] <= 0 or r[i, 1] <= 0:
            rects.append((0, 0, 0, 0))
            continue
        fts = np.float32(TS)
        tx, ty = np.float32(m[i, 0]) / fts, np.float32(m[i, 1]) / fts
        rx, ry = np.float32(r[i, 0]) / fts, np.float32(r[i, 1]) / fts
        rects.append((min(max(0, int(np.floor(tx - rx))), tw), min(max(0, int(np.floor(ty - ry))), th),
                      min(max(0, int(np.ceil(tx + rx))), tw), min(max(0, int(np.ceil(ty + ry))), th)))
    return rects


def _tiles_by_gauss(ids, flat, tw):
    out = {}
    for k, g in zip((ids >> 32).tolist(), flat.tolist()):
        out.setdefault(g, []).append(k)
    return out


def _rect_min_sigma(mx, my, a, b, c, x0, x1, y0, y1):
    """min over [x0,x1]x[y0,y1] of sigma(p) = 0.5 (a dx^2 + c dy^2) + b dx dy,
    d = p - m, in float64: zero if the mean is inside, else the least of the
    four edge minima (each a 1D convex quadratic)."""
    if x0 <= mx <= x1 and y0 <= my <= y1:
        return 0.0
    best = np.inf
    for x in (x0, x1):  # vertical edges: dx fixed, dy* = -b dx / c
        dx = x - mx
        dy = min(max(-b * dx / c, y0 - my), y1 - my)
        best = min(best, 0.5 * (a * dx * dx + c * dy * dy) + b * dx * dy)
    for y in (y0, y1):
        dy = y - my
        dx = min(max(-b * dy / a, x0 - mx), x1 - mx)
        best = min(best, 0.5 * (a * dx * dx + c * dy * dy) + b * dx * dy)
    return best


def test_known_answer_circle(oracle):
    # circle of sigma 3 px at the centre of tile (1, 1), opacity 1: slack
    # radius sqrt(2 (1.05 ln 255 + 1e-4)) * 3 = 10.23 px; the AABB rect
    # (radius ceil(3.33 * 3) = 10) is tiles 0..2 x 0..2, and the nearest pixel
    # centre of a corner tile, (15.5, 15.5), is 12.02 px away: the corners drop.
    m = np.array([[[24.0, 24.0]]], np.float32)
    r = np.array([[[10, 10]]], np.int32)
    co = np.array([[[1 / 9, 0.0, 1 / 9]]], np.float32)
    op = np.array([[1.0]], np.float32)
    d = np.array([[2.0]], np.float32)
    aabb = oracle.isect_tile(m, r, d, 1, TS, 4, 4, sort=True)
    acc = oracle.isect_tile(m, r, d, 1, TS, 4, 4, sort=True, conics=co, opacities=op)
    assert aabb["tiles_per_gauss"].tolist() == [[9]]
    assert acc["tiles_per_gauss"].tolist() == [[5]]
    assert ((acc["isect_ids"] >> 32) & 0xFF).tolist() == [1, 4, 5, 6, 9]
    # half the opacity shrinks the slack radius to sqrt(2 (1.05 ln 127.5 + 1e-4)) * 3
    # = 9.55 px: still no corner, still the cross
    acc2 = oracle.isect_tile(m, r, d, 1, TS, 4, 4, conics=co, opacities=op * 0.5)
    assert acc2["tiles_per_gauss"].tolist() == [[5]]
    # opacity below 1/255 (ln(255 o) < 0) and opacity 0: no tiles
    for o in (0.003, 0.0, -1.0):
        assert oracle.isect_count_accutile(m, r, co, np.full((1, 1), o, np.float32), TS, 4, 4).tolist() == [[0]]
    # a conic that is not positive-definite, a NaN opacity: the whole rect
    bad = np.array([[[1.0, 2.0, 1.0]]], np.float32)
    assert oracle.isect_count_accutile(m, r, bad, op, TS, 4, 4).tolist() == [[9]]
    assert oracle.isect_count_accutile(m, r, co, np.full((1, 1), np.nan, np.float32), TS, 4, 4).tolist() == [[9]]


def test_elongated_diagonal(oracle):
    # a thin ellipse along the diagonal keeps the diagonal tiles of its rect
    # and drops the off-diagonal corners
    cov = np.array([[400.0, 396.0], [396.0, 400.0]])  # long axis 28 px, short 1.4 px
    q = np.linalg.inv(cov)
    m = np.array([[[64.0, 64.0]]], np.float32)
    r = np.array([[[67, 67]]], np.int32)
    co = np.array([[[q[0, 0], q[0, 1], q[1, 1]]]], np.float32)
    op = np.array([[1.0]], np.float32)
    ids, fl = oracle.isect_encode_accutile(m, r, co, op, np.ones((1, 1), np.float32), np.zeros((1, 1), np.int32), 1,
                                           TS, 8, 8, int(oracle.isect_count_accutile(m, r, co, op, TS, 8, 8)[0, 0]))
    tiles = ((ids >> 32) & 0xFF).tolist()
    rows = {}
    for t in tiles:
        rows.setdefault(t // 8, []).append(t % 8)
    assert tiles == sorted(tiles)
    for ty, cols in rows.items():
        assert cols == list(range(cols[0], cols[-1] + 1))  # contiguous
        assert ty in cols and len(cols) <= 3  # near the diagonal only
    assert (0 * 8 + 7) not in tiles and (7 * 8 + 0) not in tiles


@pytest.mark.parametrize("seed", [0, 1])
def test_brute_force_conservative_and_tight(oracle, seed):
    rng = np.random.default_rng(seed)
    I, N, W, H = 1, 160, 97, 70
    means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    acc = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=False, conics=conics, opacities=opac)
    listed = _tiles_by_gauss(acc["isect_ids"], acc["flatten_ids"], tw)
    rects = _rect(oracle, means, radii, W, H)
    py, px = np.mgrid[0:H, 0:W]
    m = means.reshape(-1, 2)
    co = conics.reshape(-1, 3)
    op = opac.reshape(-1)
    dropped = kept = 0
    for g in range(N):
        x0, y0, x1, y1 = rects[g]
        mine = set(listed.get(g, []))
        assert all(x0 <= t % tw < x1 and y0 <= t // tw < y1 for t in mine)  # inside the AABB rect
        if not mine and (x1 <= x0 or y1 <= y0):
            continue
        # conservative: every pixel that passes the float32 alpha test
        dx = (m[g, 0] - (px.astype(np.float32) + np.float32(0.5))).astype(np.float32)
        dy = (m[g, 1] - (py.astype(np.float32) + np.float32(0.5))).astype(np.float32)
        a, b, c = (np.float32(v) for v in co[g])
        sig = np.float32(0.5) * (a * dx * dx + c * dy * dy) + b * dx * dy
        alpha = np.minimum(np.float32(0.99), op[g] * np.exp(-sig))
        ok = (sig >= 0) & (alpha >= np.float32(1.0 / 255.0))
        tyy, txx = py[ok] // TS, px[ok] // TS
        inrect = (txx >= x0) & (txx < x1) & (tyy >= y0) & (tyy < y1)
        need = set((tyy[inrect] * tw + txx[inrect]).tolist())
        assert need <= mine, (g, sorted(need - mine))
        # tight in both directions (float64 rectangle minimum)
        lim = 1.05 * np.log(255.0 * float(op[g])) + 1e-4
        for ty in range(y0, y1):
            for tx in range(x0, x1):
                ms = _rect_min_sigma(float(m[g, 0]), float(m[g, 1]), float(a), float(b), float(c),
                                     tx * TS + 0.5, tx * TS + TS - 0.5, ty * TS + 0.5, ty * TS + TS - 0.5)
                t = ty * tw + tx
                if t in mine:
                    assert ms <= lim * (1 + 1e-3) + 1e-5, (g, t, ms, lim)
                    kept += 1
                else:
                    assert ms >= lim * (1 - 1e-3) - 1e-5, (g, t, ms, lim)
                    dropped += 1
    assert dropped > 0.1 * (kept + dropped)  # the test scene does exercise the cull


def test_subset_and_order(oracle):
    rng = np.random.default_rng(5)
    I, N, W, H = 2, 120, 130, 90
    means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    aabb = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=False)
    acc = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=False, conics=conics, opacities=opac)
    assert (acc["tiles_per_gauss"] <= aabb["tiles_per_gauss"]).all()
    assert acc["tiles_per_gauss"].sum() < aabb["tiles_per_gauss"].sum()
    ga = _tiles_by_gauss(aabb["isect_ids"], aabb["flatten_ids"], tw)
    gc = _tiles_by_gauss(acc["isect_ids"], acc["flatten_ids"], tw)
    for g, ks in gc.items():
        assert ks == sorted(ks) and set(ks) <= set(ga[g])
    # flatten ids stay pair-major and the depth bits ride along
    assert (np.diff(acc["flatten_ids"]) >= 0).all()
    d = depths.reshape(-1)
    assert ((acc["isect_ids"] & 0xFFFFFFFF) == d[acc["flatten_ids"]].view(np.uint32)).all()
    # sorted variant is the stable sort of the unsorted one
    srt = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=True, conics=conics, opacities=opac)
    order = np.argsort(acc["isect_ids"], kind="stable")
    assert (srt["isect_ids"] == acc["isect_ids"][order]).all()
    assert (srt["flatten_ids"] == acc["flatten_ids"][order]).all()


def test_rendering_identity(oracle):
    rng = np.random.default_rng(11)
    I, N, W, H, C = 1, 150, 80, 64, 3
    means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
    colors = rng.uniform(0, 1, (I, N, C)).astype(np.float32)
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    outs = []
    for kw in ({}, {"conics": conics, "opacities": opac}):
        it = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=True, **kw)
        offs = oracle.isect_offset(it["isect_ids"], I, tw, th)
        f = oracle.raster_forward(means, conics, colors, opac, offs, it["flatten_ids"], W, H, TS)
        v_rc = np.random.default_rng(3).normal(size=f["render_colors"].shape).astype(np.float32)
        v_ra = np.random.default_rng(4).normal(size=f["render_alphas"].shape).astype(np.float32)
        b = oracle.raster_backward(means, conics, colors, opac, offs, it["flatten_ids"], W, H, TS,
                                   f["render_alphas"], f["last_ids"], v_rc, v_ra)
        outs.append((it, f, b))
    (ia, fa, ba), (ic, fc, bc) = outs
    assert ic["flatten_ids"].size < 0.9 * ia["flatten_ids"].size
    np.testing.assert_array_equal(fa["render_colors"], fc["render_colors"])
    np.testing.assert_array_equal(fa["render_alphas"], fc["render_alphas"])
    hit = fa["render_alphas"][..., 0] > 0
    np.testing.assert_array_equal(ia["flatten_ids"][fa["last_ids"][hit]], ic["flatten_ids"][fc["last_ids"][hit]])
    for k in ba:
        np.testing.assert_array_equal(ba[k], bc[k], err_msg=k)
