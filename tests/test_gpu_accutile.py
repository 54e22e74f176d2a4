"""GPU parity for the ellipse ("AccuTile") tile intersection: counts, keys,
sorted order and tile offsets bit-exact with the oracle, in both encode
orders, through the C ABI of both sorted pipelines (tile buckets, the
default, and the depth-presorted path for large tile grids); rendering through the AccuTile lists equals
rendering through the AABB lists (images bit-exact, gradients to 1e-4: the
per-Gaussian sums run over fewer tiles, in another order)."""
import ctypes
import os

import numpy as np
import pytest

from _helpers import assert_close_rel, assert_close_rel_summation, dev, gsplat, host, projected_scene

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")
TS = 16


def _inputs(means, radii, depths, conics=None, opac=None):
    d = {"means2d": dev(means), "radii": dev(radii), "depths": dev(depths)}
    if conics is not None:
        d["conics"] = dev(conics)
        d["opacities"] = dev(opac)
    return d


def _with_edge_cases(rng, means, radii, conics, opac):
    """NaN / zero / negative / tiny / huge opacities, a non-positive-definite
    and an ill-conditioned conic, zero radii."""
    conics = conics.copy()
    opac = opac.copy()
    radii = radii.copy()
    n = opac.shape[-1]
    pick = rng.choice(n, 8, replace=False)
    opac[..., pick[0]] = np.nan
    opac[..., pick[1]] = 0.0
    opac[..., pick[2]] = -0.5
    opac[..., pick[3]] = 0.003
    opac[..., pick[4]] = 40.0
    conics[..., pick[5], :] = [1.0, 2.0, 1.0]
    conics[..., pick[6], :] = [1.0, 0.99999, 1.0]
    radii[..., pick[7], :] = 0
    return means, radii, conics, opac


@pytest.mark.parametrize("I,N,W,H,sort", [(1, 3000, 331, 217, True), (1, 3000, 331, 217, False),
                                          (3, 2000, 200, 150, True), (2, 40000, 1297, 840, True)])
def test_bit_exact_vs_oracle(oracle, I, N, W, H, sort):
    rng = np.random.default_rng(I * 1000 + N)
    means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
    means, radii, conics, opac = _with_edge_cases(rng, means, radii, conics, opac)
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    print(f"accutile I={I} N={N} {W}x{H} sort={sort}", flush=True)
    g = gsplat()
    out = g._gsplat_core.intersect_tile_forward(_inputs(means, radii, depths, conics, opac), I, TS, tw, th, sort=sort)
    ref = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=sort, conics=conics, opacities=opac)
    np.testing.assert_array_equal(host(out["tiles_per_gauss"]), ref["tiles_per_gauss"])
    np.testing.assert_array_equal(host(out["isect_ids"]), ref["isect_ids"])
    np.testing.assert_array_equal(host(out["flatten_ids"]), ref["flatten_ids"])
    if sort:
        offs = host(g._gsplat_core.intersect_offset_forward(out["isect_ids"], I, tw, th))
        np.testing.assert_array_equal(offs, oracle.isect_offset(ref["isect_ids"], I, tw, th))
    aabb = g._gsplat_core.intersect_tile_forward(_inputs(means, radii, depths), I, TS, tw, th, sort=sort)
    assert out["isect_ids"].numel() < 0.85 * aabb["isect_ids"].numel()


def test_empty_and_all_culled():
    g = gsplat()
    m = np.array([[[24.0, 24.0], [40.0, 8.0]]], np.float32)
    r = np.array([[[10, 10], [6, 6]]], np.int32)
    d = np.array([[1.0, 2.0]], np.float32)
    co = np.array([[[1 / 9, 0.0, 1 / 9]] * 2], np.float32)
    op = np.array([[0.0, 0.002]], np.float32)  # no pixel can reach alpha 1/255
    for sort in (True, False):
        out = g._gsplat_core.intersect_tile_forward(_inputs(m, r, d, co, op), 1, TS, 4, 4, sort=sort)
        assert host(out["tiles_per_gauss"]).tolist() == [[0, 0]]
        assert out["isect_ids"].numel() == 0 and out["flatten_ids"].numel() == 0
    # known answer: the circle drops the four corners of its 3x3 rect
    out = g._gsplat_core.intersect_tile_forward(_inputs(m[:, :1], r[:, :1], d[:, :1], co[:, :1],
                                                        np.ones((1, 1), np.float32)), 1, TS, 4, 4)
    assert ((host(out["isect_ids"]) >> 32) & 0xFF).tolist() == [1, 4, 5, 6, 9]
    with pytest.raises(RuntimeError, match="needs both conics and opacities"):
        g._gsplat_core.intersect_tile_forward({"means2d": dev(m), "radii": dev(r), "depths": dev(d),
                                               "conics": dev(co)}, 1, TS, 4, 4)
    with pytest.raises(RuntimeError, match="conics"):
        g._gsplat_core.intersect_tile_forward(_inputs(m, r, d, co[..., :2].copy(), op), 1, TS, 4, 4)


def _render(g, means, conics, colors, opac, it, I, W, H, v_rc):
    import torch

    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    offs = g._gsplat_core.intersect_offset_forward(it["isect_ids"], I, tw, th)
    inp = {"means2d": dev(means), "conics": dev(conics), "colors": dev(colors), "opacities": dev(opac),
           "tile_offsets": offs, "flatten_ids": it["flatten_ids"]}
    f = g._gsplat_core.rasterize_to_pixels_3dgs_forward(inp, W, H, TS)
    b = g._gsplat_core.rasterize_to_pixels_3dgs_backward(
        inp, f, {"v_render_colors": dev(v_rc), "v_render_alphas": torch.ones_like(f["render_alphas"])}, W, H, TS,
        False)
    return f, b


def test_rendering_identity():
    rng = np.random.default_rng(7)
    I, N, W, H, C = 1, 30000, 640, 480, 3
    means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
    colors = rng.uniform(0, 1, (I, N, C)).astype(np.float32)
    v_rc = rng.normal(size=(I, H, W, C)).astype(np.float32)
    g = gsplat()
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    ia = g._gsplat_core.intersect_tile_forward(_inputs(means, radii, depths), I, TS, tw, th)
    ic = g._gsplat_core.intersect_tile_forward(_inputs(means, radii, depths, conics, opac), I, TS, tw, th)
    print(f"AABB {ia['isect_ids'].numel()} entries, AccuTile {ic['isect_ids'].numel()}", flush=True)
    fa, ba = _render(g, means, conics, colors, opac, ia, I, W, H, v_rc)
    fc, bc = _render(g, means, conics, colors, opac, ic, I, W, H, v_rc)
    np.testing.assert_array_equal(host(fa["render_colors"]), host(fc["render_colors"]))
    np.testing.assert_array_equal(host(fa["render_alphas"]), host(fc["render_alphas"]))
    hit = host(fa["render_alphas"])[..., 0] > 0
    la, lc = host(fa["last_ids"])[hit], host(fc["last_ids"])[hit]
    np.testing.assert_array_equal(host(ia["flatten_ids"])[la], host(ic["flatten_ids"])[lc])
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities"):
        assert_close_rel(host(bc[k]), host(ba[k]), 1e-4, k)  # summation order differs


def _lib():
    lib = ctypes.CDLL(LIB)
    vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_isect_count_scan_workspace_size.restype = sz
    lib.gsplat_hip_isect_count_scan_workspace_size.argtypes = [i64]
    lib.gsplat_hip_isect_count_scan_accutile.argtypes = [vp, vp, vp, vp, i64, i32, i32, i32, vp, vp, vp, vp, sz, vp]
    lib.gsplat_hip_isect_encode_accutile.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i32, i32, i32, i64, vp, vp,
                                                     vp]
    return lib


def test_c_abi_count_encode(oracle):
    import torch

    rng = np.random.default_rng(3)
    I, N, W, H = 2, 5000, 400, 300
    means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    lib = _lib()
    m, r, co, op, d = dev(means), dev(radii), dev(conics), dev(opac), dev(depths)
    n = I * N
    counts = torch.empty(n, dtype=torch.int32, device="cuda")
    offs = torch.empty(n, dtype=torch.int32, device="cuda")
    total = torch.empty(1, dtype=torch.int64, device="cuda")
    ws = torch.empty(lib.gsplat_hip_isect_count_scan_workspace_size(n), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.gsplat_hip_isect_count_scan_accutile(m.data_ptr(), r.data_ptr(), co.data_ptr(), op.data_ptr(), n, TS,
                                                  tw, th, counts.data_ptr(), offs.data_ptr(), total.data_ptr(),
                                                  ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    ref = oracle.isect_count_accutile(means, radii, conics, opac, TS, tw, th).reshape(-1)
    np.testing.assert_array_equal(host(counts), ref)
    ref_offs, ref_total = oracle.exclusive_scan(ref)
    np.testing.assert_array_equal(host(offs), ref_offs)
    assert int(total.item()) == ref_total
    ids = torch.empty(ref_total, dtype=torch.int64, device="cuda")
    fl = torch.empty(ref_total, dtype=torch.int32, device="cuda")
    rc = lib.gsplat_hip_isect_encode_accutile(m.data_ptr(), r.data_ptr(), co.data_ptr(), op.data_ptr(), d.data_ptr(),
                                              offs.data_ptr(), I, n, TS, tw, th, ref_total, ids.data_ptr(),
                                              fl.data_ptr(), stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    rid, rfl = oracle.isect_encode_accutile(means, radii, conics, opac, depths, ref_offs, I, TS, tw, th, ref_total)
    np.testing.assert_array_equal(host(ids), rid)
    np.testing.assert_array_equal(host(fl), rfl)
    # null opacities: an error, not a fault
    rc = lib.gsplat_hip_isect_encode_accutile(m.data_ptr(), r.data_ptr(), co.data_ptr(), None, d.data_ptr(),
                                              offs.data_ptr(), I, n, TS, tw, th, ref_total, ids.data_ptr(),
                                              fl.data_ptr(), stream)
    assert rc != 0 and b"null" in lib.gsplat_hip_last_error()


def _bucket_lib():
    lib = ctypes.CDLL(LIB)
    vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
    lib.gsplat_hip_last_error.restype = ctypes.c_char_p
    lib.gsplat_hip_isect_bucket_accutile_supported.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_accutile_supported.argtypes = [i64, i32, i32]
    lib.gsplat_hip_isect_bucket_count_workspace_size.restype = sz
    lib.gsplat_hip_isect_bucket_count_workspace_size.argtypes = [i64, i64, i32, i32, i32]
    lib.gsplat_hip_isect_bucket_count_accutile.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_count_accutile.argtypes = [vp, vp, vp, vp, i64, i64, i32, i32, i32, vp, vp, vp, sz,
                                                           vp]
    lib.gsplat_hip_isect_bucket_sort_workspace_size.restype = sz
    lib.gsplat_hip_isect_bucket_sort_workspace_size.argtypes = [i64]
    lib.gsplat_hip_isect_bucket_sort_accutile.restype = ctypes.c_int
    lib.gsplat_hip_isect_bucket_sort_accutile.argtypes = [vp, vp, vp, vp, vp, i64, i64, i32, i32, i32, i64, i64, vp,
                                                          vp, vp, vp, sz, vp, sz, vp]
    return lib


def _bucket(lib, means, radii, conics, opac, depths, I, tw, th):
    """count, read back (M, longest), sort: as the C++ layer does."""
    import torch

    numel = depths.size
    m, r, co, op, d = dev(means), dev(radii), dev(conics), dev(opac), dev(depths)
    stream = torch.cuda.current_stream().cuda_stream
    tpg = torch.empty(numel, dtype=torch.int32, device="cuda")
    totals = torch.zeros(2, dtype=torch.int64, device="cuda")
    ws1b = lib.gsplat_hip_isect_bucket_count_workspace_size(I, numel, TS, tw, th)
    ws1 = torch.empty(max(ws1b, 1), dtype=torch.uint8, device="cuda")
    rc = lib.gsplat_hip_isect_bucket_count_accutile(m.data_ptr(), r.data_ptr(), co.data_ptr(), op.data_ptr(), I,
                                                    numel, TS, tw, th, tpg.data_ptr(), totals.data_ptr(),
                                                    ws1.data_ptr(), ws1b, stream)
    assert rc == 0, lib.gsplat_hip_last_error()
    M, longest = (int(v) for v in totals.cpu())
    ids = torch.empty(M, dtype=torch.int64, device="cuda")
    flat = torch.empty(M, dtype=torch.int32, device="cuda")
    offs = torch.empty(I * th * tw, dtype=torch.int32, device="cuda")
    ws2b = lib.gsplat_hip_isect_bucket_sort_workspace_size(M)
    ws2 = torch.empty(max(ws2b, 1), dtype=torch.uint8, device="cuda")
    rc = lib.gsplat_hip_isect_bucket_sort_accutile(m.data_ptr(), r.data_ptr(), co.data_ptr(), op.data_ptr(),
                                                   d.data_ptr(), I, numel, TS, tw, th, M, longest, ids.data_ptr(),
                                                   flat.data_ptr(), offs.data_ptr(), ws1.data_ptr(), ws1b,
                                                   ws2.data_ptr(), ws2b, stream)
    torch.cuda.synchronize()
    return rc, M, longest, host(tpg), host(ids), host(flat), host(offs).reshape(I, th, tw)


@pytest.mark.parametrize("I,N,W,H,ties,culled", [(1, 3000, 331, 217, False, 0.0),
                                                 (3, 2000, 200, 150, True, 0.0),
                                                 (1, 20000, 1297, 840, True, 0.0),
                                                 (2, 300000, 1297, 840, False, 0.9)])
def test_bucket_c_abi(oracle, I, N, W, H, ties, culled):
    """gsplat_hip_isect_bucket_count_accutile / _sort_accutile bit for bit
    against the oracle's sorted ellipse lists: tiles_per_gauss, ids, flatten
    ids, tile offsets, M and the longest list. Scenes: several images, depth
    ties (the tile sort's id order), the edge-case opacities and conics, a
    round with more tile rows than one chunk of the scatter (every case here),
    and 600,000 Gaussians (two rounds of 1024 per grid / scatter block)."""
    rng = np.random.default_rng(I * 7 + N)
    means, radii, conics, opac, depths = projected_scene(rng, I, N, W, H)
    means, radii, conics, opac = _with_edge_cases(rng, means, radii, conics, opac)
    if ties:
        depths = np.round(depths * 2.0).astype(np.float32) / 2.0
    if culled:
        radii[rng.random((I, N)) < culled] = 0
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    print(f"bucket accutile I={I} N={N} {W}x{H} ties={ties} culled={culled}", flush=True)
    lib = _bucket_lib()
    rc, M, longest, tpg, ids, flat, offs = _bucket(lib, means, radii, conics, opac, depths, I, tw, th)
    assert rc == 0, lib.gsplat_hip_last_error()
    ref = oracle.isect_tile(means, radii, depths, I, TS, tw, th, sort=True, conics=conics, opacities=opac)
    eoffs = oracle.isect_offset(ref["isect_ids"], I, tw, th)
    assert M == ref["isect_ids"].size
    lens = np.diff(np.append(eoffs.ravel(), M))
    assert longest == lens.max()
    np.testing.assert_array_equal(tpg, ref["tiles_per_gauss"].ravel())
    np.testing.assert_array_equal(ids, ref["isect_ids"])
    np.testing.assert_array_equal(flat, ref["flatten_ids"])
    np.testing.assert_array_equal(offs, eoffs)


def test_bucket_long_list_and_grid_limit(oracle):
    """A tile list longer than the LDS tile sort holds (20,000 ellipses on one
    tile, a quarter at one depth): the bucketed C ABI sorts it (split by the
    leading depth bits into LDS-sorted runs). A tile grid the ellipse bucket
    path does not support (201 x 131 corner points) takes the depth-presorted
    path. Both give the oracle's lists; supported() marks the grid limit."""
    lib = _bucket_lib()
    assert lib.gsplat_hip_isect_bucket_accutile_supported(1, 160, 90)      # 2560x1440 at 16 px
    assert not lib.gsplat_hip_isect_bucket_accutile_supported(1, 200, 130)
    g = gsplat()
    rng = np.random.default_rng(12)
    n = 20000
    m = np.stack([rng.uniform(17, 31, n), rng.uniform(17, 31, n)], -1).astype(np.float32)[None]
    r = np.full((1, n, 2), 6, np.int32)
    co = np.tile(np.array([1 / 4, 0.0, 1 / 4], np.float32), (1, n, 1))
    op = rng.uniform(0.2, 1.0, (1, n)).astype(np.float32)
    d = rng.uniform(1, 9, (1, n)).astype(np.float32)
    d[:, ::4] = 3.0
    rc, M, longest, tpg, ids, flat, offs = _bucket(lib, m, r, co, op, d, 1, 4, 4)
    assert rc == 0, lib.gsplat_hip_last_error()
    assert longest > 16384
    ref = oracle.isect_tile(m, r, d, 1, TS, 4, 4, sort=True, conics=co, opacities=op)
    np.testing.assert_array_equal(ids, ref["isect_ids"])
    np.testing.assert_array_equal(flat, ref["flatten_ids"])
    np.testing.assert_array_equal(offs, oracle.isect_offset(ref["isect_ids"], 1, 4, 4))
    cases = [(m, r, co, op, d, 4, 4)]
    sm, sr, sc, so, sd = projected_scene(rng, 1, 3000, 3200, 2080)
    cases.append((sm, sr, sc, so, sd, 200, 130))
    for cm, cr, cc, cop, cd, tw, th in cases:
        print(f"accutile intersect_tile_offsets n={cd.size} grid {tw}x{th}", flush=True)
        out = g._gsplat_core.intersect_tile_offsets_forward(_inputs(cm, cr, cd, cc, cop), 1, TS, tw, th)
        ref = oracle.isect_tile(cm, cr, cd, 1, TS, tw, th, sort=True, conics=cc, opacities=cop)
        np.testing.assert_array_equal(host(out["tiles_per_gauss"]), ref["tiles_per_gauss"])
        np.testing.assert_array_equal(host(out["isect_ids"]), ref["isect_ids"])
        np.testing.assert_array_equal(host(out["flatten_ids"]), ref["flatten_ids"])
        np.testing.assert_array_equal(host(out["tile_offsets"]), oracle.isect_offset(ref["isect_ids"], 1, tw, th))


def test_bucket_largest_ellipse_grid(oracle):
    """The largest tile grid the ellipse bucket path accepts (37 x 691 =
    25,567 corner points: the scatter's dynamic LDS plus its static block-scan
    words fill the 160 KiB workgroup LDS) runs count and sort through the C
    ABI and gives the oracle's lists; one more tile row is refused."""
    lib = _bucket_lib()
    tw, th = 36, 690
    assert lib.gsplat_hip_isect_bucket_accutile_supported(1, tw, th)
    assert not lib.gsplat_hip_isect_bucket_accutile_supported(1, tw, th + 1)
    rng = np.random.default_rng(25567)
    W, H = tw * TS, th * TS
    means, radii, conics, opac, depths = projected_scene(rng, 1, 4000, W, H)
    print(f"bucket accutile largest grid {tw}x{th}", flush=True)
    rc, M, longest, tpg, ids, flat, offs = _bucket(lib, means, radii, conics, opac, depths, 1, tw, th)
    assert rc == 0, lib.gsplat_hip_last_error()
    ref = oracle.isect_tile(means, radii, depths, 1, TS, tw, th, sort=True, conics=conics, opacities=opac)
    assert M == ref["isect_ids"].size
    np.testing.assert_array_equal(tpg, ref["tiles_per_gauss"].ravel())
    np.testing.assert_array_equal(ids, ref["isect_ids"])
    np.testing.assert_array_equal(flat, ref["flatten_ids"])
    np.testing.assert_array_equal(offs, oracle.isect_offset(ref["isect_ids"], 1, tw, th))


@pytest.mark.parametrize("name", ["sh3_1m", "multiview_3m"])
def test_render_model_full_size(name):
    """The training render step at full size: AccuTile lists give the same
    images, and parameter gradients to the chain's 1e-3 (float atomics sum
    them in another order: at most one element per million may reach 1e-2,
    where a sum cancels heavily)."""
    import torch

    from gsplat_core import render as R
    from gsplat_core.scenes import make_scene

    sc = make_scene(name, seed=0, with_target=False)
    print(f"accutile render {name}: N={sc.n} C={sc.n_cameras}", flush=True)

    def p(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda().requires_grad_(True)

    params = [p(sc.means), p(sc.quats), p(sc.log_scales), p(sc.features_dc), p(sc.features_rest),
              p(sc.opacity_logits)]
    vm, Ks = torch.from_numpy(sc.viewmats).cuda(), torch.from_numpy(sc.Ks).cuda()
    cot = None
    res = []
    for acc in (False, True):
        for q in params:
            q.grad = None
        out = R.render_sh_model(*params, vm, Ks, sc.width, sc.height, sc.tile_size, sc.sh_degree,
                                background=sc.background, far_plane=sc.far_plane, accutile=acc)
        if cot is None:
            cot = torch.randn(out["render_colors"].shape, device="cuda", generator=torch.Generator("cuda").manual_seed(1))
        (out["render_colors"] * cot).sum().backward()
        res.append((host(out["render_colors"]), host(out["render_alphas"]), out["isect_ids"].numel(),
                    [host(q.grad) for q in params]))
    (ca, aa, ma, ga), (cc, ac, mc, gc) = res
    print(f"AABB {ma} entries, AccuTile {mc}", flush=True)
    assert mc < ma
    np.testing.assert_array_equal(ca, cc)
    np.testing.assert_array_equal(aa, ac)
    for k, x, y in zip(("means", "quats", "log_scales", "features_dc", "features_rest", "opacity_logits"), gc, ga):
        assert_close_rel_summation(x, y, 1e-3, k)  # both HIP; only the summation order differs
