"""End-to-end parity of the training step on the GPU against the oracle:
render_sh_model / render_rgb_model + the image loss (L1, or L1 + DSSIM of
image_loss_components, scanner_points_training_utils.py:1147-1182) through
torch autograd (the HIP
kernels and the VJP routing of gsplat_projection.cpp:1130-1208,
gsplat_rasterize.cpp:749-795, gsplat_spherical_harmonics.cpp:670-705),
against the oracle's operators composed with float64 glue VJPs
(tests/_oracle_chain.py, pinned by tests/test_oracle_chain.py) and the image
loss oracle's VJP (oracle/image_loss.py, pinned by
tests/test_oracle_image_loss.py).

Workloads: the random-scene forward render (10k Gaussians, 256x256,
opacities in the projection; render_random_3dgs_png.py:61-168) and the
image-fitting step (100k Gaussians, 512x512, RGB colours, L1 forward and
backward; train_image_fitting_3dgs_mlx.py:165-237, 431-454) at full size,
and the SH-degree-3 step (sh3_1m's distributions) at 1 and 3 cameras, with
either loss.

Bars: the parameter activations within 1e-6 relative of float64; projection
outputs within 1e-5 relative of the oracle's on those activations (radius flips
counted and printed, at most MAX_RADIUS_FLIPS; the oracle's later stages take the
GPU's radii), SH colours within 1e-5; tile counts, sorted ids, flatten ids
and tile offsets bit-exact with the oracle's intersection of the GPU's
projection; images within 1e-4 max-abs, last_ids exact; the loss within
1e-6 (L1 + DSSIM: 1e-5 relative); every parameter gradient (means, quaternions, log-scales, opacity
logits, SH features or colours, and the viewspace proxy) within 1e-3
relative (floor 1e-2 of the tensor's largest magnitude: the rasterizer's float
atomics sum in another order); activations and projection outputs with the
1e-4 floor."""
import numpy as np
import pytest

import _oracle_chain as ch
from _helpers import FLOOR_ORDERED, MAX_RADIUS_FLIPS, assert_close_rel, dev, host
from oracle import image_loss as il

pytestmark = pytest.mark.gpu

GRAD_RTOL = 1e-3
IMG_ATOL = 1e-4


SSIM_LAMBDA, SSIM_WINDOW = 0.2, 11


def _gpu_step(sc, C=None, sh=True, backward=True, loss_mode="l1"):
    import torch

    from gsplat_core import render as R
    from gsplat_core.autograd import activated_projection, gaussian_activations, sh_camera_colors

    C = C or sc.n_cameras
    vm, K = dev(sc.viewmats[:, :C]), dev(sc.Ks[:, :C])
    keys = ["means", "quats", "log_scales", "opacity_logits"] + (["features_dc", "features_rest"] if sh else
                                                                  ["colors"])
    p = {k: dev(getattr(sc, k)).requires_grad_(backward) for k in keys}
    W, H, ts = sc.width, sc.height, sc.tile_size
    if sh:
        vsp = torch.zeros((1, C, sc.n, 2), device="cuda", requires_grad=backward)
        out = R.render_sh_model(p["means"], p["quats"], p["log_scales"], p["features_dc"], p["features_rest"],
                                p["opacity_logits"], vm, K, W, H, ts, sc.sh_degree, viewspace_points=vsp,
                                background=sc.background, far_plane=sc.far_plane)
    else:
        vsp = None
        out = R.render_rgb_model(p["means"], p["quats"], p["log_scales"], p["colors"], p["opacity_logits"], vm, K,
                                 W, H, ts, background=sc.background, opacities_in_projection=sc.opacities_in_projection,
                                 far_plane=sc.far_plane)
    loss = None
    if backward:
        # C cameras as one [C, H, W, 3] batch: the mean of the per-camera
        # losses, as the reference's loss functions average them
        loss = R.image_training_loss(out["render_colors"], dev(sc.target[:C]), loss_mode, SSIM_LAMBDA, SSIM_WINDOW)
        loss.backward()
    with torch.no_grad():
        proj = activated_projection(p["means"], p["quats"], p["log_scales"], p["opacity_logits"], vm, K, W, H,
                                    eps2d=0.3, near_plane=0.01, far_plane=sc.far_plane,
                                    opacities_in_projection=sc.opacities_in_projection)
        # the activations the projection kernels applied (bit for bit)
        act = gaussian_activations(p["quats"], p["log_scales"], p["opacity_logits"])
        if sh:
            colors = sh_camera_colors(sc.sh_degree, p["means"], vm, p["features_dc"], p["features_rest"])
        else:
            colors = p["colors"][:, None].expand(-1, C, -1, -1)
    torch.cuda.synchronize()
    fwd = {k: host(proj[k]) for k in ("means2d", "depths", "conics", "radii", "opacities")}
    fwd["act"] = [host(a) for a in act]
    fwd["colors"] = np.ascontiguousarray(host(colors))
    for k in ("render_colors", "render_alphas", "last_ids", "tile_offsets", "flatten_ids", "isect_ids",
              "tiles_per_gauss"):
        fwd[k] = host(out[k])
    grads = {k: host(v.grad) for k, v in p.items()} if backward else {}
    if backward and vsp is not None:
        grads["viewspace"] = host(vsp.grad)
    return fwd, grads, (float(loss.detach()) if loss is not None else None)


def _check_forward(oracle, sc, fwd, C, sh):
    """GPU intermediates against the oracle's own forward; intersection and
    raster bit-exact / 1e-4 on the GPU's projection."""
    W, H, ts = sc.width, sc.height, sc.tile_size
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    N = sc.n
    # the GPU's float32 activations against float64, then the oracle's
    # projection of exactly those values
    q32, s32, o32 = fwd["act"]
    for got, want, k in zip(fwd["act"], ch.activations(sc.quats, sc.log_scales, sc.opacity_logits),
                            ("quats", "scales", "opacities")):
        assert_close_rel(got, want, 1e-6, k, floor_rel=FLOOR_ORDERED)
    np.testing.assert_array_equal(fwd["opacities"], o32)
    pr = oracle.projection_forward(sc.means, sc.viewmats[:, :C], sc.Ks[:, :C], W, H, quats=q32, scales=s32,
                                   opacities=o32 if sc.opacities_in_projection else None, far_plane=sc.far_plane)
    on_g, on_o = (fwd["radii"] > 0).all(-1), (pr["radii"] > 0).all(-1)
    flips = int(np.sum(np.any(fwd["radii"] != pr["radii"], -1)))
    print(f"{sc.name}: N={N} C={C} visible={int(on_g.sum())} radius flips={flips}", flush=True)
    assert flips <= MAX_RADIUS_FLIPS, flips
    both = on_g & on_o
    for k in ("means2d", "depths", "conics"):
        assert_close_rel(fwd[k][both], pr[k][both], 1e-5, k, floor_rel=FLOOR_ORDERED)
    if sh:
        col, _ = ch.sh_colours(oracle, sc.means, sc.features_dc, sc.features_rest, sc.viewmats[:, :C], sc.sh_degree)
        assert np.abs(fwd["colors"] - col).max() <= 1e-5
    # intersection of the GPU projection: bit-exact
    isect = oracle.isect_tile(fwd["means2d"], fwd["radii"], fwd["depths"], C, ts, tw, th)
    np.testing.assert_array_equal(fwd["tiles_per_gauss"], isect["tiles_per_gauss"])
    np.testing.assert_array_equal(fwd["isect_ids"], isect["isect_ids"])
    np.testing.assert_array_equal(fwd["flatten_ids"], isect["flatten_ids"])
    np.testing.assert_array_equal(fwd["tile_offsets"], oracle.isect_offset(isect["isect_ids"], C, tw, th))
    # raster of the same inputs
    opac_img = np.ascontiguousarray(np.broadcast_to(fwd["opacities"].reshape(1, 1, N), (1, C, N)))
    bg = np.tile(np.asarray(sc.background, np.float32)[None], (C, 1))
    rf = oracle.raster_forward(fwd["means2d"], fwd["conics"], fwd["colors"], opac_img, fwd["tile_offsets"],
                               fwd["flatten_ids"], W, H, ts, backgrounds=bg)
    err = np.abs(fwd["render_colors"] - rf["render_colors"]).max()
    assert err <= IMG_ATOL, err
    assert np.abs(fwd["render_alphas"] - rf["render_alphas"]).max() <= IMG_ATOL
    np.testing.assert_array_equal(fwd["last_ids"], rf["last_ids"])
    print(f"{sc.name}: {fwd['isect_ids'].size} intersections, image max-abs err {err:.2e}", flush=True)
    return rf


def _check_gradients(oracle, sc, fwd, grads, loss, C, sh, loss_mode="l1"):
    target = sc.target[:C]
    img = fwd["render_colors"]
    want_loss = il.image_loss_components(img, target, loss_mode, SSIM_LAMBDA, SSIM_WINDOW)["loss"]
    assert abs(loss - want_loss) <= (1e-6 if loss_mode == "l1" else 1e-5 * abs(want_loss)), (loss, want_loss)
    v_img = il.loss_vjp(img, target, loss_mode, SSIM_LAMBDA, SSIM_WINDOW).astype(np.float32)
    p = {k: getattr(sc, k) for k in grads if k != "viewspace"}
    exp = ch.chain(oracle, p, sc.viewmats[:, :C], sc.Ks[:, :C], sc.width, sc.height, sc.tile_size, fwd,
                   target=target, sh_degree=sc.sh_degree if sh else None, background=sc.background,
                   v_render_colors=v_img)
    for k in grads:
        assert np.isfinite(grads[k]).all(), k
        assert np.abs(exp[k]).max() > 0, k
        assert_close_rel(grads[k], exp[k], GRAD_RTOL, k)


@pytest.mark.parametrize("loss_mode", ["l1", "l1_dssim"])
@pytest.mark.parametrize("name,C,n,W,H", [("sh3_1m", 1, 8000, 320, 208), ("multiview_3m", 3, 6000, 240, 136),
                                         ("multiview_3m", 8, 6000, 240, 136)])
def test_sh_training_step_vs_oracle_chain(oracle, name, C, n, W, H, loss_mode):
    from gsplat_core.scenes import make_scene

    sc = make_scene(name, seed=5 + C, n=n, width=W, height=H)
    fwd, grads, loss = _gpu_step(sc, C=C, sh=True, loss_mode=loss_mode)
    _check_forward(oracle, sc, fwd, C, True)
    _check_gradients(oracle, sc, fwd, grads, loss, C, True, loss_mode)


def test_random_forward_full_size(oracle):
    """The random-scene forward render at its full size: 10,000 Gaussians,
    256x256, opacities in the projection, forward only."""
    from gsplat_core.scenes import make_scene

    sc = make_scene("random_forward", seed=0)
    assert sc.n == 10_000 and (sc.width, sc.height) == (256, 256)
    fwd, _, _ = _gpu_step(sc, sh=False, backward=False)
    _check_forward(oracle, sc, fwd, 1, False)


def test_image_fit_full_size(oracle):
    """The image-fitting step at its full size: 100,000 Gaussians, 512x512,
    RGB colours, L1 loss forward and backward to every parameter."""
    from gsplat_core.scenes import make_scene

    sc = make_scene("image_fit", seed=0)
    assert sc.n == 100_000 and (sc.width, sc.height) == (512, 512)
    fwd, grads, loss = _gpu_step(sc, sh=False)
    _check_forward(oracle, sc, fwd, 1, False)
    _check_gradients(oracle, sc, fwd, grads, loss, 1, False)


def test_sh3_1m_full_frame(oracle):
    """The headline SH-degree-3 step at full size, whole frame: 1,000,000
    Gaussians, 1297x840, about 5.4M intersections, L1 forward and backward
    to every parameter, against the oracle chain (about 30 s of CPU)."""
    from gsplat_core.scenes import make_scene

    sc = make_scene("sh3_1m", seed=0)
    assert sc.n == 1_000_000 and (sc.width, sc.height) == (1297, 840)
    fwd, grads, loss = _gpu_step(sc, sh=True)
    _check_forward(oracle, sc, fwd, 1, True)
    _check_gradients(oracle, sc, fwd, grads, loss, 1, True)
