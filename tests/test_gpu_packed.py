"""GPU parity for the packed layout (upstream gsplat's packed=True path;
rejected by the reference at gsplat_intersect.cpp:115-118 and
gsplat_rasterize.cpp:48-51): the packed projection equals the dense one at
the visible pairs bit for bit, and its backward equals the dense backward
with the cotangents scattered (same kernel); the packed intersection is
bit-exact with the oracle; the packed rasterizer renders what the dense one
renders; the whole packed chain gives the dense chain's images and
gradients."""
import numpy as np
import pytest
from scipy.spatial.transform import Rotation

from _helpers import FLOOR_ORDERED, assert_close_rel, assert_close_rel_summation, dev, gsplat, host, projected_scene

pytestmark = pytest.mark.gpu
TS = 16


def _scene(rng, B, C, N, W=320, H=240):
    means = (rng.normal(size=(B, N, 3)) * [0.8, 0.6, 0.5] + [0, 0, 4.0]).astype(np.float32)
    quats = rng.normal(size=(B, N, 4)).astype(np.float32)
    scales = np.exp(rng.uniform(-4, -1.5, (B, N, 3))).astype(np.float32)
    opac = rng.uniform(0.01, 1, (B, N)).astype(np.float32)
    view = np.zeros((B, C, 4, 4), np.float32)
    for b in range(B):
        for c in range(C):
            view[b, c, :3, :3] = Rotation.from_euler("xyz", rng.normal(scale=0.15, size=3)).as_matrix()
            view[b, c, :3, 3] = rng.normal(scale=0.4, size=3)
            view[b, c, 3, 3] = 1
    Ks = np.zeros((B, C, 3, 3), np.float32)
    Ks[..., 0, 0], Ks[..., 1, 1], Ks[..., 0, 2], Ks[..., 1, 2], Ks[..., 2, 2] = 300, 290, W / 2, H / 2, 1
    return means, quats, scales, opac, view, Ks


@pytest.mark.parametrize("B,C,N,opac,comp", [(1, 1, 1000, False, False), (1, 3, 777, True, False),
                                             (2, 2, 3001, True, True), (1, 4, 64, False, True)])
def test_projection_packed_equals_dense(oracle, B, C, N, opac, comp):
    rng = np.random.default_rng(N)
    means, quats, scales, op, view, Ks = _scene(rng, B, C, N)
    g = gsplat()
    inputs = {"means": dev(means), "quats": dev(quats), "scales": dev(scales), "viewmats": dev(view), "Ks": dev(Ks)}
    if opac:
        inputs["opacities"] = dev(op)
    kw = dict(calc_compensations=comp)
    print(f"packed projection B={B} C={C} N={N} opac={opac} comp={comp}", flush=True)
    dn = g.projection_ewa_3dgs_fused_forward(inputs, 320, 240, **kw)
    pk = g.projection_ewa_3dgs_packed_forward(inputs, 320, 240, **kw)
    radii = host(dn["radii"])
    vis = np.all(radii > 0, -1).reshape(-1)
    flat = np.flatnonzero(vis)
    nnz = flat.size
    assert 0 < nnz < vis.size
    cam = flat // N
    np.testing.assert_array_equal(host(pk["batch_ids"]), cam // C)
    np.testing.assert_array_equal(host(pk["camera_ids"]), cam % C)
    np.testing.assert_array_equal(host(pk["gaussian_ids"]), flat % N)
    np.testing.assert_array_equal(host(pk["indptr"]), np.concatenate([[0], np.cumsum(np.bincount(cam, minlength=B * C))]))
    for k, w in (("radii", 2), ("means2d", 2), ("depths", 1), ("conics", 3)) + ((("compensations", 1),) if comp else ()):
        d = host(dn[k]).reshape(vis.size, -1)[flat]
        np.testing.assert_array_equal(host(pk[k]).reshape(nnz, -1), d, err_msg=k)
    # the oracle's packed layout where both see the same visible pairs
    e = oracle.projection_packed_forward(means, view, Ks, 320, 240, quats=quats, scales=scales,
                                         opacities=op if opac else None, calc_compensations=comp)
    if e["gaussian_ids"].size == nnz and (e["camera_ids"] == host(pk["camera_ids"])).all():
        assert_close_rel(host(pk["conics"]), e["conics"], 1e-5, "conics", floor_rel=FLOOR_ORDERED)

    # backward: the dense backward with the cotangents scattered to their pairs
    rng2 = np.random.default_rng(1)
    v_m2 = rng2.normal(size=(nnz, 2)).astype(np.float32)
    v_d = rng2.normal(size=(nnz,)).astype(np.float32)
    v_c = rng2.normal(size=(nnz, 3)).astype(np.float32)
    cot_p = {"v_means2d": dev(v_m2), "v_depths": dev(v_d), "v_conics": dev(v_c)}
    fwd_p = {"batch_ids": pk["batch_ids"], "camera_ids": pk["camera_ids"], "gaussian_ids": pk["gaussian_ids"],
             "conics": pk["conics"]}
    dense_cot = {}
    for k, v, w in (("v_means2d", v_m2, 2), ("v_depths", v_d, 1), ("v_conics", v_c, 3)):
        full = np.zeros((vis.size, w), np.float32)
        full[flat] = v.reshape(nnz, w)
        dense_cot[k] = dev(full.reshape(host(dn[k[2:]]).shape))
    fwd_d = {"radii": dn["radii"], "conics": dn["conics"]}
    if comp:
        v_comp = rng2.normal(size=(nnz,)).astype(np.float32)
        cot_p["v_compensations"] = dev(v_comp)
        fwd_p["compensations"] = pk["compensations"]
        full = np.zeros(vis.size, np.float32)
        full[flat] = v_comp
        dense_cot["v_compensations"] = dev(full.reshape(host(dn["compensations"]).shape))
        fwd_d["compensations"] = dn["compensations"]
    bp = g.projection_ewa_3dgs_packed_backward(inputs, fwd_p, cot_p, 320, 240, viewmats_requires_grad=True)
    bd = g.projection_ewa_3dgs_fused_backward(inputs, fwd_d, dense_cot, 320, 240, viewmats_requires_grad=True)
    for k in ("v_means", "v_quats", "v_scales", "v_viewmats"):
        np.testing.assert_array_equal(host(bp[k]), host(bd[k]), err_msg=k)


@pytest.mark.parametrize("B,C,N,logits,viewgrad", [(1, 1, 2000, True, False), (1, 3, 3001, True, True),
                                                     (2, 2, 777, True, True), (1, 2, 500, False, False)])
def test_activated_projection_packed(B, C, N, logits, viewgrad):
    """The activated packed projection (activations in the packed kernels,
    per-row opacities, the backward reading the forward's rank structure)
    against its composition from the separate operators: gaussian_activations,
    projection_packed and a gather of the opacities by Gaussian id. Rows and
    opacities bit for bit; gradients w.r.t. means, raw quaternions,
    log-scales, opacity logits and view matrices within 1e-4 relative (the
    opacity gradient sums a Gaussian's rows in another order)."""
    import torch

    from gsplat_core.autograd import activated_projection_packed, gaussian_activations, projection_packed

    rng = np.random.default_rng(N + C)
    means, quats, scales, op, view, Ks = _scene(rng, B, C, N)
    log_scales = np.log(scales).astype(np.float32)
    lg = rng.normal(size=(B, N)).astype(np.float32)
    print(f"activated packed projection B={B} C={C} N={N} logits={logits} viewgrad={viewgrad}", flush=True)

    def run(fused):
        m, q, ls, vm = (dev(a).requires_grad_(True) for a in (means, quats, log_scales, view))
        lo = dev(lg).requires_grad_(True) if logits else None
        K = dev(Ks)
        if fused:
            out = activated_projection_packed(m, q, ls, lo, vm if viewgrad else vm.detach(), K, 320, 240)
            out = {k: v for k, v in out.items()}
        else:
            qa, sa, oa = gaussian_activations(q, ls, lo if logits else torch.zeros((B, N), device="cuda"))
            out = projection_packed(m, qa, sa, vm if viewgrad else vm.detach(), K, 320, 240)
            if logits:
                out["opacities"] = oa.reshape(-1).index_select(0, (out["batch_ids"].long() * N +
                                                                   out["gaussian_ids"].long()))
        g = torch.Generator(device="cuda").manual_seed(7)
        loss = 0
        for k in ("means2d", "depths", "conics") + (("opacities",) if logits else ()):
            loss = loss + (out[k] * torch.randn(out[k].shape, device="cuda", generator=g)).sum()
        loss.backward()
        torch.cuda.synchronize()
        res = {k: host(v) for k, v in out.items() if k != "compensations"}
        res.update({"v_means": host(m.grad), "v_quats": host(q.grad), "v_log_scales": host(ls.grad)})
        if logits:
            res["v_logits"] = host(lo.grad)
        if viewgrad:
            res["v_viewmats"] = host(vm.grad)
        return res

    a, b = run(True), run(False)
    assert a["means2d"].shape[0] > 0
    a.pop("rank")
    if not logits:
        assert a.pop("opacities").size == 0
    for k in a:
        if k.startswith("v_"):
            assert np.abs(b[k]).max() > 0, k
            assert_close_rel_summation(a[k], b[k], 1e-4, k)
        else:
            np.testing.assert_array_equal(a[k], b[k], err_msg=k)


def test_activated_packed_speculation():
    """A repeated shape writes its rows speculatively (outputs sized by the
    previous count, filled before the count reaches the host): kept when the
    count fits, redone when it does not. Four calls of one shape -- few
    visible pairs, then many (over the capacity), many again (kept), few
    again (kept) -- each give the rows, indptr and opacities of the exact
    composition (gaussian_activations + projection_packed)."""
    import torch

    from gsplat_core.autograd import activated_projection_packed, gaussian_activations, projection_packed

    B, C, N = 1, 2, 4001  # a shape of its own
    rng = np.random.default_rng(99)
    means, quats, scales, op, view, Ks = _scene(rng, B, C, N)
    few = means.copy()
    few[:, : N * 3 // 4, 2] = -5.0  # three quarters behind the cameras
    lg = rng.normal(size=(B, N)).astype(np.float32)
    for name, m in (("few", few), ("many", means), ("many again", means), ("few again", few)):
        out = activated_projection_packed(dev(m), dev(quats), dev(np.log(scales)), dev(lg), dev(view), dev(Ks), 320,
                                          240)
        qa, sa, oa = gaussian_activations(dev(quats), dev(np.log(scales)), dev(lg))
        ref = projection_packed(dev(m), qa, sa, dev(view), dev(Ks), 320, 240)
        torch.cuda.synchronize()
        print(f"speculation {name}: nnz {out['camera_ids'].numel()}", flush=True)
        for k in ("batch_ids", "camera_ids", "gaussian_ids", "indptr", "radii", "means2d", "depths", "conics"):
            np.testing.assert_array_equal(host(out[k]), host(ref[k]), err_msg=f"{name} {k}")
        np.testing.assert_array_equal(host(out["opacities"]), host(oa).reshape(-1)[host(ref["gaussian_ids"])],
                                      err_msg=name)


@pytest.mark.parametrize("B,C,K", [(1, 1, 3), (1, 3, 3), (2, 2, 5)])
def test_packed_rows(B, C, K):
    """packed_rows_gather takes each row's (batch, camera, Gaussian) slot of a
    dense array; packed_rows_scatter puts rows back at their slots by the rank
    structure, zeros elsewhere (the gather's adjoint), and the viewspace
    gradient of the activated packed backward is the same scatter of the
    means2d rows' cotangent."""
    import torch

    from gsplat_core.autograd import activated_projection_packed

    rng = np.random.default_rng(B * 10 + C)
    N = 2500
    means, quats, scales, op, view, Ks = _scene(rng, B, C, N)
    g = gsplat()
    m = dev(means)
    vsp = torch.zeros((B, C, N, 2), device="cuda", requires_grad=True)
    out = activated_projection_packed(m, dev(quats), dev(np.log(scales)), None, dev(view), dev(Ks), 320, 240,
                                      viewspace_points=vsp)
    bid, cid, gid = (host(out[k]) for k in ("batch_ids", "camera_ids", "gaussian_ids"))
    nnz = cid.size
    assert 0 < nnz < B * C * N
    dense = rng.normal(size=(B, C, N, K)).astype(np.float32)
    ids = {"camera_ids": out["camera_ids"], "gaussian_ids": out["gaussian_ids"]}
    if B > 1:
        ids["batch_ids"] = out["batch_ids"]
    rows = host(g._gsplat_core.packed_rows_gather(dev(dense), ids))
    np.testing.assert_array_equal(rows, dense[bid, cid, gid])
    v = rng.normal(size=(nnz, K)).astype(np.float32)
    back = host(g._gsplat_core.packed_rows_scatter(dev(v), out["rank"], B, C, N))
    exp = np.zeros_like(dense)
    exp[bid, cid, gid] = v
    np.testing.assert_array_equal(back, exp)
    # the viewspace proxy's gradient: the means2d rows' cotangent at their slots
    w = torch.from_numpy(rng.normal(size=(nnz, 2)).astype(np.float32)).cuda()
    (out["means2d"] * w).sum().backward()
    exp2 = np.zeros((B, C, N, 2), np.float32)
    exp2[bid, cid, gid] = host(w)
    np.testing.assert_array_equal(host(vsp.grad), exp2)


@pytest.mark.parametrize("B,C,degree,R,N", [(1, 1, 3, 15, 2500), (1, 3, 3, 15, 2500), (2, 2, 1, 3, 2501),
                                            (1, 1, 3, 15, 130001), (1, 2, 2, 8, 1500), (2, 1, 0, 0, 777)])
def test_sh_camera_colors_packed(B, C, degree, R, N):
    """The packed layout's camera colours (written and read at the pairs'
    packed rows through the rank structure) equal the dense camera colours
    gathered at the rows, bit for bit, and their backward equals the dense
    backward of the rows' cotangents scattered to their slots (zeros
    elsewhere). Slab and general kernels, one to three cameras, two batches,
    and the slab forward's resident-grid walk."""
    import torch

    from gsplat_core.autograd import activated_projection_packed

    rng = np.random.default_rng(B * 100 + C * 10 + degree)
    means, quats, scales, op, view, Ks = _scene(rng, B, C, N)
    g = gsplat()
    out = activated_projection_packed(dev(means), dev(quats), dev(np.log(scales)), None, dev(view), dev(Ks), 320, 240)
    bid, cid, gid = (host(out[k]) for k in ("batch_ids", "camera_ids", "gaussian_ids"))
    nnz = cid.size
    assert 0 < nnz < B * C * N
    dc = rng.normal(scale=0.3, size=(B, N, 3)).astype(np.float32)
    rest = rng.normal(scale=0.1, size=(B, N, R, 3)).astype(np.float32)
    base = {"means": dev(means), "viewmats": dev(view), "features_dc": dev(dc), "features_rest": dev(rest)}
    print(f"packed sh colours: B={B} C={C} degree={degree} R={R} N={N} nnz={nnz}", flush=True)
    dense = host(g._gsplat_core.sh_camera_colors_forward(degree, base))
    rows = host(g._gsplat_core.sh_camera_colors_packed_forward(degree, dict(base, rank=out["rank"]), nnz))
    np.testing.assert_array_equal(rows, dense[bid, cid, gid])
    v = rng.normal(size=(nnz, 3)).astype(np.float32)
    vd = np.zeros((B, C, N, 3), np.float32)
    vd[bid, cid, gid] = v
    e = g._gsplat_core.sh_camera_colors_backward(degree, base, {"v_colors": dev(vd)})
    a = g._gsplat_core.sh_camera_colors_packed_backward(degree, dict(base, rank=out["rank"]), {"v_colors": dev(v)})
    for k in ("v_means", "v_features_dc", "v_features_rest"):
        np.testing.assert_array_equal(host(a[k]), host(e[k]), err_msg=k)
    torch.cuda.synchronize()


def _packed_image_ids(rng, layout, I, nnz):
    """Row image ids: grouped by image (the packed projection's order), grouped
    with empty images (first, inner and last), or not grouped (the sorted
    intersection then takes the depth-presorted path after the read-back)."""
    if layout == "grouped":
        return np.sort(rng.integers(0, I, nnz)).astype(np.int32)
    if layout == "gaps":
        return np.sort(rng.choice(np.array([1, 3], np.int32), nnz)).astype(np.int32)
    return rng.integers(0, I, nnz).astype(np.int32)


@pytest.mark.parametrize("layout", ["grouped", "gaps", "shuffled"])
@pytest.mark.parametrize("accutile", [False, True])
@pytest.mark.parametrize("sort", [False, True])
def test_isect_packed_vs_oracle(oracle, accutile, sort, layout):
    rng = np.random.default_rng(17)
    I, nnz, W, H = 5 if layout == "gaps" else 4, 30000, 640, 480
    means, radii, conics, opac, depths = (a[0] for a in projected_scene(rng, 1, nnz, W, H))
    img = _packed_image_ids(rng, layout, I, nnz)
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    g = gsplat()
    inp = {"means2d": dev(means), "radii": dev(radii), "depths": dev(depths), "image_ids": dev(img)}
    kw = {}
    if accutile:
        inp["conics"], inp["opacities"] = dev(conics), dev(opac)
        kw = {"conics": conics, "opacities": opac}
    print(f"packed isect accutile={accutile} sort={sort} layout={layout}", flush=True)
    out = g.intersect_tile_forward(inp, I, TS, tw, th, sort=sort)
    ref = oracle.isect_tile_packed(means, radii, depths, img, I, TS, tw, th, sort=sort, **kw)
    np.testing.assert_array_equal(host(out["tiles_per_gauss"]), ref["tiles_per_gauss"])
    np.testing.assert_array_equal(host(out["isect_ids"]), ref["isect_ids"])
    np.testing.assert_array_equal(host(out["flatten_ids"]), ref["flatten_ids"])
    # int64 image ids (upstream's dtype) give the same lists
    inp["image_ids"] = dev(img.astype(np.int64))
    out2 = g.intersect_tile_forward(inp, I, TS, tw, th, sort=sort)
    np.testing.assert_array_equal(host(out2["isect_ids"]), ref["isect_ids"])
    if sort:  # the lists with their tile offsets, in one call and split around the read-back
        offs = oracle.isect_offset(ref["isect_ids"], I, tw, th)
        from gsplat_core import _gsplat_core as _C

        for o in (_C.intersect_tile_offsets_forward(inp, I, TS, tw, th),
                  _C.intersect_tile_offsets_end(_C.intersect_tile_offsets_begin(inp, I, TS, tw, th))):
            np.testing.assert_array_equal(host(o["isect_ids"]), ref["isect_ids"])
            np.testing.assert_array_equal(host(o["flatten_ids"]), ref["flatten_ids"])
            np.testing.assert_array_equal(host(o["tiles_per_gauss"]), ref["tiles_per_gauss"])
            np.testing.assert_array_equal(host(o["tile_offsets"]), offs)


@pytest.mark.parametrize("nnz", [1, 2047])
def test_isect_packed_small(oracle, nnz):
    """Packed sorted intersections of 1 and 2047 rows over three images (the
    tile-bucket path with images that hold no segment, and one segment; the
    binding takes inputs without rows as the dense layout)."""
    rng = np.random.default_rng(nnz + 3)
    I, W, H = 3, 200, 150
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    means, radii, conics, opac, depths = (a[0] for a in projected_scene(rng, 1, max(nnz, 1), W, H))
    means, radii, depths = means[:nnz], radii[:nnz], depths[:nnz]
    img = np.sort(rng.integers(0, I, nnz)).astype(np.int32)
    from gsplat_core import _gsplat_core as _C

    inp = {"means2d": dev(means), "radii": dev(radii), "depths": dev(depths), "image_ids": dev(img)}
    print(f"packed isect small nnz={nnz}", flush=True)
    o = _C.intersect_tile_offsets_forward(inp, I, TS, tw, th)
    ref = oracle.isect_tile_packed(means, radii, depths, img, I, TS, tw, th, sort=True)
    np.testing.assert_array_equal(host(o["isect_ids"]), ref["isect_ids"])
    np.testing.assert_array_equal(host(o["flatten_ids"]), ref["flatten_ids"])
    np.testing.assert_array_equal(host(o["tile_offsets"]), oracle.isect_offset(ref["isect_ids"], I, tw, th))


def _chain(g, torch, means, quats, scales, op, colors, view, Ks, W, H, packed, cot):
    B, N = means.shape[0], means.shape[1]
    C = view.shape[1]
    params = [torch.from_numpy(a).cuda() for a in (means, quats, scales)]
    inputs = {"means": params[0], "quats": params[1], "scales": params[2], "viewmats": dev(view), "Ks": dev(Ks)}
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    if packed:
        pr = g.projection_ewa_3dgs_packed_forward(inputs, W, H)
        cid = pr["camera_ids"].long()
        gid = pr["gaussian_ids"].long()
        rows_op = dev(op)[0][gid]
        rows_col = dev(colors)[0][gid]
        it = g.intersect_tile_forward({"means2d": pr["means2d"], "radii": pr["radii"], "depths": pr["depths"],
                                       "image_ids": pr["camera_ids"], "gaussian_ids": pr["gaussian_ids"]},
                                      C, TS, tw, th)
        m2, con, opr, colr = pr["means2d"], pr["conics"], rows_op, rows_col
    else:
        pr = g.projection_ewa_3dgs_fused_forward(inputs, W, H)
        it = g.intersect_tile_forward({"means2d": pr["means2d"], "radii": pr["radii"], "depths": pr["depths"]},
                                      C, TS, tw, th)
        m2, con = pr["means2d"], pr["conics"]
        opr = dev(op)[:, None].expand(-1, C, -1).contiguous()
        colr = dev(colors)[:, None].expand(-1, C, -1, -1).contiguous()
    offs = g.intersect_offset_forward(it["isect_ids"], C, tw, th)
    rin = {"means2d": m2, "conics": con, "colors": colr, "opacities": opr, "tile_offsets": offs,
           "flatten_ids": it["flatten_ids"]}
    f = g.rasterize_to_pixels_3dgs_forward(rin, W, H, TS)
    b = g.rasterize_to_pixels_3dgs_backward(rin, f, {"v_render_colors": dev(cot)}, W, H, TS, False)
    fo = {"radii": pr["radii"], "conics": pr["conics"]}
    if packed:
        fo.update({"batch_ids": pr["batch_ids"], "camera_ids": pr["camera_ids"], "gaussian_ids": pr["gaussian_ids"]})
        pb = g.projection_ewa_3dgs_packed_backward(inputs, fo, {"v_means2d": b["v_means2d"], "v_conics": b["v_conics"]},
                                                   W, H)
        v_op = torch.zeros((N,), device="cuda").index_add_(0, gid, b["v_opacities"])
        v_col = torch.zeros((N, colors.shape[-1]), device="cuda").index_add_(0, gid, b["v_colors"])
    else:
        pb = g.projection_ewa_3dgs_fused_backward(inputs, fo, {"v_means2d": b["v_means2d"], "v_conics": b["v_conics"]},
                                                  W, H)
        v_op = b["v_opacities"].sum(1)[0]
        v_col = b["v_colors"].sum(1)[0]
    return f, {"v_means": pb["v_means"], "v_quats": pb["v_quats"], "v_scales": pb["v_scales"], "v_opac": v_op,
               "v_colors": v_col}, it


def test_packed_chain_equals_dense():
    import torch

    rng = np.random.default_rng(5)
    B, C, N, W, H = 1, 3, 20000, 320, 240
    means, quats, scales, op, view, Ks = _scene(rng, B, C, N, W, H)
    colors = rng.uniform(0, 1, (B, N, 3)).astype(np.float32)
    cot = rng.normal(size=(C, H, W, 3)).astype(np.float32)
    g = gsplat()
    fd, gd, itd = _chain(g, torch, means, quats, scales, op, colors, view, Ks, W, H, False, cot)
    fp, gp, itp = _chain(g, torch, means, quats, scales, op, colors, view, Ks, W, H, True, cot)
    print(f"dense entries {itd['isect_ids'].numel()}, packed {itp['isect_ids'].numel()}", flush=True)
    np.testing.assert_array_equal(host(itp["isect_ids"]), host(itd["isect_ids"]))
    np.testing.assert_array_equal(host(fp["render_colors"]), host(fd["render_colors"]))
    np.testing.assert_array_equal(host(fp["render_alphas"]), host(fd["render_alphas"]))
    for k in gd:
        assert_close_rel(host(gp[k]), host(gd[k]), 1e-4, k)


def test_packed_errors():
    g = gsplat()
    m = dev(np.zeros((3, 2), np.float32))
    r = dev(np.ones((3, 2), np.int32))
    d = dev(np.ones((3,), np.float32))
    with pytest.raises(RuntimeError, match="image_ids"):
        g.intersect_tile_forward({"means2d": m, "radii": r, "depths": d, "gaussian_ids": dev(np.arange(3))}, 1, TS, 4,
                                 4)
    with pytest.raises(RuntimeError, match="image_ids"):
        g.intersect_tile_forward({"means2d": m, "radii": r, "depths": d, "image_ids": dev(np.zeros(2, np.int32))}, 1,
                                 TS, 4, 4)


@pytest.mark.parametrize("name", ["sh3_1m", "multiview_3m"])
def test_render_model_packed_full_size(name):
    """The training render step at full size over the packed layout: the same
    images, parameter and viewspace gradients to the chain's 1e-3 (summed in
    another order: at most one element per million may reach 1e-2, where a
    sum cancels heavily)."""
    import torch

    from gsplat_core import render as R
    from gsplat_core.scenes import make_scene

    sc = make_scene(name, seed=0, with_target=False)
    print(f"packed render {name}: N={sc.n} C={sc.n_cameras}", flush=True)

    def p(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda().requires_grad_(True)

    params = [p(sc.means), p(sc.quats), p(sc.log_scales), p(sc.features_dc), p(sc.features_rest),
              p(sc.opacity_logits)]
    vm, Ks = torch.from_numpy(sc.viewmats).cuda(), torch.from_numpy(sc.Ks).cuda()
    vsp = torch.zeros((1, sc.n_cameras, sc.n, 2), device="cuda", requires_grad=True)
    cot = None
    res = []
    for packed in (False, True):
        for q in params + [vsp]:
            q.grad = None
        out = R.render_sh_model(*params, vm, Ks, sc.width, sc.height, sc.tile_size, sc.sh_degree,
                                viewspace_points=vsp, background=sc.background, far_plane=sc.far_plane,
                                packed=packed)
        if cot is None:
            cot = torch.randn(out["render_colors"].shape, device="cuda", generator=torch.Generator("cuda").manual_seed(2))
        (out["render_colors"] * cot).sum().backward()
        res.append((host(out["render_colors"]), host(out["render_alphas"]), host(out["isect_ids"]),
                    [host(q.grad) for q in params] + [host(vsp.grad)]))
    (ca, aa, ia, ga), (cp, ap, ip, gp) = res
    np.testing.assert_array_equal(ia, ip)
    np.testing.assert_array_equal(ca, cp)
    np.testing.assert_array_equal(aa, ap)
    names = ("means", "quats", "log_scales", "features_dc", "features_rest", "opacity_logits", "viewspace")
    for k, x, y in zip(names, gp, ga):
        assert_close_rel_summation(x, y, 1e-3, k)  # both HIP; only the summation order differs
