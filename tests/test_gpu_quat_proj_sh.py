"""GPU parity: quat_scale_to_covar_preci, fused projection and spherical
harmonics (HIP through the binding, C++ API and C ABI) against the oracle on
identical seeded inputs, plus the reference's known answers.

Tolerances (from the build's parity contract): float32 forward outputs within
1e-5 relative, gradients within 1e-3 relative (see _helpers.assert_close_rel);
integer radii exact."""
import numpy as np
import pytest
from scipy.spatial.transform import Rotation

from _helpers import FLOOR_ATOMIC, FLOOR_ORDERED, MAX_RADIUS_FLIPS, assert_close_rel, dev, gsplat, host

pytestmark = pytest.mark.gpu

FWD_RTOL = 1e-5
GRAD_RTOL = 1e-3


# ------------------------------------------------------------------ quat/scale
def _floor(camera_model, grad=False):
    """The small-element floor of a projection check: 1e-4 of the largest
    magnitude for the pinhole camera. The equidistant fisheye (camera model 2)
    takes atan2 and sqrt from the device math library, which differ from the
    host libm's in the last ulp; cancellation in near-zero means2d and
    gradient elements turns that into ~1e-3 relative differences below 1e-2
    of the largest magnitude. Orthographic gradients (camera model 1) are
    sums of terms of the tensor's largest magnitude: measured differences
    reach 1.8e-7 of that magnitude (about 3 float32 ulps), so elements below
    1e-3 of it are held to 1e-6 of it."""
    if camera_model == 2:
        return FLOOR_ATOMIC
    return 1e-3 if grad and camera_model == 1 else FLOOR_ORDERED


def test_quat_known_answers():
    g = gsplat()
    quats = np.array([[1, 0, 0, 0], [2, 0, 0, 0]], np.float32)
    scales = np.array([[2, 3, 4], [0.5, 2, 4]], np.float32)
    out = g.quat_scale_to_covar_preci_forward({"quats": dev(quats), "scales": dev(scales)})
    np.testing.assert_allclose(host(out["covars"]), [[4, 0, 0, 9, 0, 16], [0.25, 0, 0, 4, 0, 16]], atol=1e-6)
    np.testing.assert_allclose(host(out["precis"]), [[0.25, 0, 0, 1 / 9, 0, 1 / 16], [4, 0, 0, 0.25, 0, 1 / 16]],
                               atol=1e-6)
    full = g.quat_scale_to_covar_preci_forward({"quats": dev(quats), "scales": dev(scales)}, True, False, False)
    assert tuple(full["covars"].shape) == (2, 3, 3) and tuple(full["precis"].shape) == (0,)


@pytest.mark.parametrize("triu", [True, False])
def test_quat_random_vs_oracle(oracle, triu):
    g = gsplat()
    rng = np.random.default_rng(0)
    n = 5000
    quats = rng.normal(size=(n, 4)).astype(np.float32)
    scales = np.exp(rng.uniform(-3, 1, (n, 3))).astype(np.float32)
    out = g.quat_scale_to_covar_preci_forward({"quats": dev(quats), "scales": dev(scales)}, True, True, triu)
    ec, ep = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, True, triu)
    assert_close_rel(host(out["covars"]), ec, FWD_RTOL, "covars", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(out["precis"]), ep, FWD_RTOL, "precis", floor_rel=FLOOR_ORDERED)
    shape = (n, 6) if triu else (n, 3, 3)
    vc = rng.normal(size=shape).astype(np.float32)
    vp = rng.normal(size=shape).astype(np.float32)
    bwd = g.quat_scale_to_covar_preci_backward({"quats": dev(quats), "scales": dev(scales)},
                                               {"v_covars": dev(vc), "v_precis": dev(vp)}, triu)
    eq, es = oracle.quat_scale_to_covar_preci_backward(quats, scales, vc, vp, triu)
    assert_close_rel(host(bwd["v_quats"]), eq, GRAD_RTOL, "v_quats", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(bwd["v_scales"]), es, GRAD_RTOL, "v_scales", floor_rel=FLOOR_ORDERED)
    # only one cotangent
    bwd1 = g.quat_scale_to_covar_preci_backward({"quats": dev(quats), "scales": dev(scales)}, {"v_precis": dev(vp)},
                                                triu)
    eq1, es1 = oracle.quat_scale_to_covar_preci_backward(quats, scales, None, vp, triu)
    assert_close_rel(host(bwd1["v_quats"]), eq1, GRAD_RTOL, "v_quats precis-only", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(bwd1["v_scales"]), es1, GRAD_RTOL, "v_scales precis-only", floor_rel=FLOOR_ORDERED)


def test_quat_errors():
    g = gsplat()
    with pytest.raises(RuntimeError, match=r"quats must have shape \[\.\.\., 4\]"):
        g.quat_scale_to_covar_preci_forward({"quats": dev(np.zeros((3, 3), np.float32)),
                                             "scales": dev(np.zeros((3, 3), np.float32))})
    with pytest.raises(RuntimeError, match="missing input: scales"):
        g.quat_scale_to_covar_preci_forward({"quats": dev(np.zeros((3, 4), np.float32))})


# ------------------------------------------------------------------ projection
def _scene(rng, B, C, N, spread=0.6, depth=4.0):
    means = (rng.normal(size=(B, N, 3)) * [spread, spread * 0.8, 0.5] + [0, 0, depth]).astype(np.float32)
    quats = rng.normal(size=(B, N, 4)).astype(np.float32)
    scales = np.exp(rng.uniform(-4, -1.5, (B, N, 3))).astype(np.float32)
    opac = rng.uniform(0.01, 1, (B, N)).astype(np.float32)
    view = np.zeros((B, C, 4, 4), np.float32)
    for b in range(B):
        for c in range(C):
            view[b, c, :3, :3] = Rotation.from_euler("xyz", rng.normal(scale=0.1, size=3)).as_matrix()
            view[b, c, :3, 3] = rng.normal(scale=0.2, size=3)
            view[b, c, 3, 3] = 1
    Ks = np.zeros((B, C, 3, 3), np.float32)
    Ks[..., 0, 0], Ks[..., 1, 1], Ks[..., 0, 2], Ks[..., 1, 2], Ks[..., 2, 2] = 400, 380, 160, 120, 1
    return means, quats, scales, opac, view, Ks


def _proj_both(oracle, means, view, Ks, W, H, **kw):
    g = gsplat()
    inputs = {"means": dev(means), "viewmats": dev(view), "Ks": dev(Ks)}
    for k in ("covars", "quats", "scales", "opacities"):
        if kw.get(k) is not None:
            inputs[k] = dev(kw[k])
    pk = {k: kw[k] for k in ("eps2d", "near_plane", "far_plane", "radius_clip", "calc_compensations",
                             "camera_model") if k in kw}
    got = g.projection_ewa_3dgs_fused_forward(inputs, W, H, **pk)
    exp = oracle.projection_forward(means, view, Ks, W, H, covars=kw.get("covars"), quats=kw.get("quats"),
                                    scales=kw.get("scales"), opacities=kw.get("opacities"), **pk)
    return got, exp


@pytest.mark.parametrize("B,C,use_covars,use_opac,calc_comp,camera_model", [
    (1, 1, False, False, False, 0), (1, 3, False, True, True, 0), (2, 2, True, False, True, 0),
    (1, 2, True, True, False, 1), (1, 1, False, True, False, 2)])
def test_projection_forward_vs_oracle(oracle, B, C, use_covars, use_opac, calc_comp, camera_model):
    rng = np.random.default_rng(B * 10 + C)
    means, quats, scales, opac, view, Ks = _scene(rng, B, C, 4000)
    kw = dict(opacities=opac if use_opac else None, calc_compensations=calc_comp, camera_model=camera_model,
              near_plane=0.01, far_plane=100.0)
    if use_covars:
        cov, _ = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, False, True)
        kw["covars"] = cov
    else:
        kw["quats"], kw["scales"] = quats, scales
    got, exp = _proj_both(oracle, means, view, Ks, 320, 240, **kw)
    r_got, r_exp = host(got["radii"]), exp["radii"]
    # radii are ceil() of float expressions evaluated in the same order; a
    # log() ulp (opacity-aware extent) may flip one at an integer boundary
    flips = np.sum(np.any(r_got != r_exp, axis=-1))
    print(f"[projection] radius flips: {flips} of {r_exp.shape[-2]}", flush=True)
    assert flips <= MAX_RADIUS_FLIPS, f"{flips} radius mismatches"
    both = np.all(r_got > 0, -1) & np.all(r_exp > 0, -1)
    assert both.sum() > 100
    for k in ("means2d", "conics", "depths"):
        assert_close_rel(host(got[k])[both], exp[k][both], FWD_RTOL, k, floor_rel=_floor(camera_model))
    if calc_comp:
        assert_close_rel(host(got["compensations"])[both], exp["compensations"][both], FWD_RTOL, "compensations",
                         floor_rel=_floor(camera_model))
    else:
        assert tuple(got["compensations"].shape) == (0,)
    culled = np.all(r_got == 0, -1)
    assert np.all(host(got["conics"])[culled] == 0) and np.all(host(got["depths"])[culled] == 0)


def test_projection_known_answers_and_culling(oracle):
    g = gsplat()
    eye = np.eye(4, dtype=np.float32).reshape(1, 1, 4, 4)
    K = np.array([[[[50, 0, 32], [0, 50, 32], [0, 0, 1]]]], np.float32)
    means = np.array([[[0, 0, 1], [0, 0, 0.001], [0, 0, 200], [0.25, -0.25, 2]]], np.float32)
    quats = np.tile(np.array([1, 0, 0, 0], np.float32), (1, 4, 1))
    scales = np.array([[[0.1] * 3, [0.1] * 3, [0.1] * 3, [0.001] * 3]], np.float32)
    out = g.projection_ewa_3dgs_fused_forward({"means": dev(means), "quats": dev(quats), "scales": dev(scales),
                                               "viewmats": dev(eye), "Ks": dev(K)}, 64, 64, near_plane=0.01,
                                              far_plane=100.0, radius_clip=2.0)
    r = host(out["radii"])[0, 0]
    assert r[0, 0] > 2 and r[0, 1] > 2 and np.all(r[1:] == 0)
    assert tuple(out["compensations"].shape) == (0,)
    e = oracle.projection_forward(means, eye, K, 64, 64, quats=quats, scales=scales, near_plane=0.01,
                                  far_plane=100.0, radius_clip=2.0)
    np.testing.assert_array_equal(r, e["radii"][0, 0])


@pytest.mark.parametrize("use_covars,calc_comp,C,camera_model", [(False, False, 1, 0), (False, True, 2, 0),
                                                                 (True, True, 3, 0), (False, True, 2, 1),
                                                                 (True, False, 1, 1), (False, True, 2, 2),
                                                                 (True, False, 1, 2)])
def test_projection_backward_vs_oracle(oracle, use_covars, calc_comp, C, camera_model):
    g = gsplat()
    rng = np.random.default_rng(7 + C)
    B, N = 1, 3000
    means, quats, scales, _, view, Ks = _scene(rng, B, C, N)
    if camera_model == 1:  # orthographic: keep the means inside the 320x240 view
        means[..., :2] *= 0.25
    kw = dict(calc_compensations=calc_comp, near_plane=0.01, far_plane=100.0, camera_model=camera_model)
    cov = None
    if use_covars:
        cov, _ = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, False, True)
        kw["covars"] = cov
    else:
        kw["quats"], kw["scales"] = quats, scales
    got, exp = _proj_both(oracle, means, view, Ks, 320, 240, **kw)
    radii = exp["radii"]
    vm2 = rng.normal(size=exp["means2d"].shape).astype(np.float32)
    vd = rng.normal(size=exp["depths"].shape).astype(np.float32)
    vc = rng.normal(size=exp["conics"].shape).astype(np.float32)
    vcomp = rng.normal(size=exp["depths"].shape).astype(np.float32)
    inputs = {"means": dev(means), "viewmats": dev(view), "Ks": dev(Ks)}
    if use_covars:
        inputs["covars"] = dev(cov)
    else:
        inputs["quats"], inputs["scales"] = dev(quats), dev(scales)
    fwd = {"radii": dev(radii), "conics": dev(exp["conics"])}
    cot = {"v_means2d": dev(vm2), "v_depths": dev(vd), "v_conics": dev(vc)}
    if calc_comp:
        fwd["compensations"] = dev(exp["compensations"])
        cot["v_compensations"] = dev(vcomp)
    out = g.projection_ewa_3dgs_fused_backward(inputs, fwd, cot, 320, 240, viewmats_requires_grad=True,
                                               camera_model=camera_model)
    e = oracle.projection_backward(means, view, Ks, 320, 240, radii, exp["conics"], vm2, vd, vc, covars=cov,
                                   quats=None if use_covars else quats, scales=None if use_covars else scales,
                                   compensations=exp["compensations"] if calc_comp else None,
                                   v_compensations=vcomp if calc_comp else None, viewmats_requires_grad=True,
                                   camera_model=camera_model)
    assert (radii > 0).any(axis=-1).sum() > 1000
    for k in e:
        assert_close_rel(host(out[k]), e[k], GRAD_RTOL, k, floor_rel=_floor(camera_model, grad=True))
    # an absent v_depths means zeros
    cot0 = dict(cot, v_depths=dev(np.zeros_like(vd)))
    cot_absent = {k: v for k, v in cot.items() if k != "v_depths"}
    a = g.projection_ewa_3dgs_fused_backward(inputs, fwd, cot0, 320, 240, viewmats_requires_grad=True,
                                             camera_model=camera_model)
    b = g.projection_ewa_3dgs_fused_backward(inputs, fwd, cot_absent, 320, 240, viewmats_requires_grad=True,
                                             camera_model=camera_model)
    for k in a:
        np.testing.assert_allclose(host(b[k]), host(a[k]), rtol=1e-6, atol=1e-30, err_msg=k)


# ------------------------------------------------------------------------- SH
C0, C1 = 0.2820947917738781, 0.48860251190292


def test_sh_known_answers():
    g = gsplat()
    dirs = np.array([[0, 0, 1], [1, 0, 0]], np.float32)
    coeffs = np.array([[[1, 2, 3], [0.1, 0.2, 0.3], [0.4, 0.5, 0.6], [0.7, 0.8, 0.9]],
                       [[4, 5, 6], [0, 0, 0], [0, 0, 0], [0, 0, 0]]], np.float32)
    masks = np.array([True, False])
    out = host(g.spherical_harmonics_forward(1, {"dirs": dev(dirs), "coeffs": dev(coeffs), "masks": dev(masks)}))
    np.testing.assert_allclose(out[0], [C0 + C1 * 0.4, 2 * C0 + C1 * 0.5, 3 * C0 + C1 * 0.6], atol=1e-6)
    assert np.all(out[1] == 0)
    b = g.spherical_harmonics_backward(1, {"dirs": dev(dirs[:1]), "coeffs": dev(coeffs[:1])},
                                       {"v_colors": dev(np.array([[1, 2, 3]], np.float32))})
    np.testing.assert_allclose(host(b["v_dirs"])[0], [-C1 * 5, -C1 * 1.4, 0], atol=5e-4)
    np.testing.assert_allclose(host(b["v_coeffs"])[0, 2], [C1, 2 * C1, 3 * C1], atol=1e-6)


@pytest.mark.parametrize("degree,K,use_masks", [(0, 1, False), (1, 4, True), (2, 16, False), (3, 16, True),
                                                (4, 25, False), (3, 25, False)])
def test_sh_vs_oracle(oracle, degree, K, use_masks):
    g = gsplat()
    rng = np.random.default_rng(degree * 7 + K)
    n = 20011  # not a multiple of the block size
    dirs = rng.normal(size=(n, 3)).astype(np.float32)
    dirs[:3] = 0.0  # zero directions: DC only
    coeffs = rng.normal(size=(n, K, 3)).astype(np.float32)
    masks = rng.random(n) < 0.8 if use_masks else None
    v_colors = rng.normal(size=(n, 3)).astype(np.float32)
    inputs = {"dirs": dev(dirs), "coeffs": dev(coeffs)}
    if use_masks:
        inputs["masks"] = dev(masks)
    got = host(g.spherical_harmonics_forward(degree, inputs))
    exp = oracle.sh_forward(degree, dirs, coeffs, masks)
    assert_close_rel(got, exp, FWD_RTOL, "colors", floor_rel=FLOOR_ORDERED)
    b = g.spherical_harmonics_backward(degree, inputs, {"v_colors": dev(v_colors)})
    ed, ec = oracle.sh_backward(degree, dirs, coeffs, v_colors, masks)
    assert_close_rel(host(b["v_coeffs"]), ec, GRAD_RTOL, "v_coeffs", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(b["v_dirs"]), ed, GRAD_RTOL, "v_dirs", floor_rel=FLOOR_ORDERED)
    nb = g.spherical_harmonics_backward(degree, inputs, {"v_colors": dev(v_colors)}, compute_v_dirs=False)
    assert "v_dirs" not in nb
    assert_close_rel(host(nb["v_coeffs"]), ec, GRAD_RTOL, "v_coeffs (no dirs)", floor_rel=FLOOR_ORDERED)


def test_sh_errors():
    g = gsplat()
    with pytest.raises(RuntimeError, match="fewer SH bases"):
        g.spherical_harmonics_forward(3, {"dirs": dev(np.zeros((2, 3), np.float32)),
                                          "coeffs": dev(np.zeros((2, 9, 3), np.float32))})
    with pytest.raises(RuntimeError, match="degree 0..4"):
        g.spherical_harmonics_forward(5, {"dirs": dev(np.zeros((2, 3), np.float32)),
                                          "coeffs": dev(np.zeros((2, 36, 3), np.float32))})
