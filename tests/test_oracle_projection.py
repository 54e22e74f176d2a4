"""Pins the oracle's EWA projection: the reference's closed-form isotropic
pinhole oracle and culling cases (gsplat_core/test/test.cpp:60-130, 261-437),
a textbook EWA restatement built from scipy rotations and matrix products
(Zwicker et al. 2002: Sigma_2d = J W Sigma W^T J^T), and float64 finite
differences of the forward for every backward output, v_viewmats included."""
import numpy as np
import pytest
from scipy.spatial.transform import Rotation


def reference_pinhole(x, y, z, variance, opacity, W, H, fx, fy, cx, cy, eps2d, calc_comp):
    """Closed form for an isotropic Gaussian (test.cpp:60-130)."""
    f = np.float32
    tan_fovx = f(0.5) * f(W) / f(fx)
    tan_fovy = f(0.5) * f(H) / f(fy)
    lim_x_pos = (f(W) - f(cx)) / f(fx) + f(0.3) * tan_fovx
    lim_x_neg = f(cx) / f(fx) + f(0.3) * tan_fovx
    lim_y_pos = (f(H) - f(cy)) / f(fy) + f(0.3) * tan_fovy
    lim_y_neg = f(cy) / f(fy) + f(0.3) * tan_fovy
    rz = f(1) / f(z)
    rz2 = rz * rz
    tx = f(z) * min(lim_x_pos, max(-lim_x_neg, f(x) * rz))
    ty = f(z) * min(lim_y_pos, max(-lim_y_neg, f(y) * rz))
    j00, j02, j11, j12 = f(fx) * rz, -f(fx) * tx * rz2, f(fy) * rz, -f(fy) * ty * rz2
    v = f(variance)
    c00 = v * (j00 * j00 + j02 * j02)
    c01 = v * (j02 * j12)
    c11 = v * (j11 * j11 + j12 * j12)
    det_orig = c00 * c11 - c01 * c01
    c00 += f(eps2d)
    c11 += f(eps2d)
    det = c00 * c11 - c01 * c01
    comp = np.sqrt(max(f(0.005) * f(0.005), det_orig / det))
    extend = f(3.33)
    ob = f(opacity) * (comp if calc_comp else f(1))
    if ob >= f(1 / 255):
        extend = min(extend, np.sqrt(f(2) * np.log(ob / f(1 / 255))))
    return dict(radii=[int(np.ceil(extend * np.sqrt(c00))), int(np.ceil(extend * np.sqrt(c11)))],
                means2d=[f(fx) * f(x) * rz + f(cx), f(fy) * f(y) * rz + f(cy)], depth=f(z),
                conics=[c11 / det, -c01 / det, c00 / det], compensation=comp)


EYE = np.eye(4, dtype=np.float32).reshape(1, 1, 4, 4)


def _K(fx, fy, cx, cy):
    return np.array([[[[fx, 0, cx], [0, fy, cy], [0, 0, 1]]]], np.float32)


@pytest.mark.parametrize("use_covars", [False, True])
def test_closed_form_pinhole(oracle, use_covars):
    # test.cpp:261-350
    means = np.array([[[0, 0, 1], [0.25, -0.25, 2]]], np.float32)
    quats = np.array([[[1, 0, 0, 0], [1, 0, 0, 0]]], np.float32)
    scales = np.array([[[0.1] * 3, [0.2] * 3]], np.float32)
    covars = np.array([[[0.01, 0, 0, 0.01, 0, 0.01], [0.04, 0, 0, 0.04, 0, 0.04]]], np.float32)
    opac = np.array([[0.8, 0.6]], np.float32)
    kw = dict(covars=covars) if use_covars else dict(quats=quats, scales=scales)
    out = oracle.projection_forward(means, EYE, _K(50, 50, 32, 32), 64, 64, opacities=opac, eps2d=0.3,
                                    near_plane=0.01, far_plane=100, calc_compensations=True, **kw)
    assert out["radii"].shape == (1, 1, 2, 2) and out["compensations"].shape == (1, 1, 2)
    for i, (m, var, o) in enumerate([((0, 0, 1), 0.01, 0.8), ((0.25, -0.25, 2), 0.04, 0.6)]):
        e = reference_pinhole(*m, var, o, 64, 64, 50, 50, 32, 32, 0.3, True)
        assert list(out["radii"][0, 0, i]) == e["radii"]
        np.testing.assert_allclose(out["means2d"][0, 0, i], e["means2d"], atol=1e-4)
        np.testing.assert_allclose(out["depths"][0, 0, i], e["depth"], atol=1e-5)
        np.testing.assert_allclose(out["conics"][0, 0, i], e["conics"], atol=1e-4)
        np.testing.assert_allclose(out["compensations"][0, 0, i], e["compensation"], atol=1e-4)


def test_culling_cases(oracle):
    # test.cpp:352-437: near, far, radius_clip=2 (both radii <= clip culls)
    means = np.array([[[0, 0, 1], [0, 0, 0.001], [0, 0, 200], [0.25, -0.25, 2]]], np.float32)
    quats = np.tile(np.array([1, 0, 0, 0], np.float32), (1, 4, 1))
    scales = np.array([[[0.1] * 3, [0.1] * 3, [0.1] * 3, [0.001] * 3]], np.float32)
    out = oracle.projection_forward(means, EYE, _K(50, 50, 32, 32), 64, 64, quats=quats, scales=scales,
                                    near_plane=0.01, far_plane=100, radius_clip=2.0)
    r = out["radii"][0, 0]
    assert r[0, 0] > 2 and r[0, 1] > 2
    assert np.all(r[1:] == 0)
    assert out["compensations"].shape == (0,)
    # culled entries are all-zero
    assert np.all(out["conics"][0, 0, 1:] == 0) and np.all(out["depths"][0, 0, 1:] == 0)


def test_offscreen_cull_and_radius_clip_and(oracle):
    """GPU semantics (gsplat_projection.metal:314-326): off-screen Gaussians are
    culled; radius clip culls only when both radii are <= clip."""
    means = np.array([[[5.0, 0, 1], [0, 0, 1]]], np.float32)  # first projects to x = 282 >> 64
    covars = np.array([[[0.01, 0, 0, 0.01, 0, 0.01], [0.0004, 0, 0, 0.0004, 0, 0.0004]]], np.float32)
    out = oracle.projection_forward(means, EYE, _K(50, 50, 32, 32), 64, 64, covars=covars)
    assert np.all(out["radii"][0, 0, 0] == 0)
    rx, ry = out["radii"][0, 0, 1]
    assert rx > 0
    # anisotropic: rx ~ 3, ry ~ 2 -> clip at 2 keeps it (AND), clip at 3 culls
    cov = np.array([[[0.01, 0, 0, 0.01, 0, 0.01], [0.0016, 0, 0, 0.0004, 0, 0.0004]]], np.float32)
    o2 = oracle.projection_forward(means, EYE, _K(50, 50, 32, 32), 64, 64, covars=cov)
    rx, ry = o2["radii"][0, 0, 1]
    assert rx != ry
    keep = oracle.projection_forward(means, EYE, _K(50, 50, 32, 32), 64, 64, covars=cov, radius_clip=float(min(rx, ry)))
    assert np.all(keep["radii"][0, 0, 1] == [rx, ry])
    cull = oracle.projection_forward(means, EYE, _K(50, 50, 32, 32), 64, 64, covars=cov, radius_clip=float(max(rx, ry)))
    assert np.all(cull["radii"][0, 0, 1] == 0)


def _random_scene(rng, B, C, N, dtype=np.float64):
    means = rng.normal(size=(B, N, 3)) * [0.6, 0.5, 0.4] + [0, 0, 4]
    quats = rng.normal(size=(B, N, 4))
    scales = np.exp(rng.uniform(-3, -1.5, size=(B, N, 3)))
    viewmats = np.zeros((B, C, 4, 4))
    for b in range(B):
        for c in range(C):
            R = Rotation.from_euler("xyz", rng.normal(scale=0.05, size=3)).as_matrix()
            viewmats[b, c, :3, :3] = R
            viewmats[b, c, :3, 3] = rng.normal(scale=0.1, size=3)
            viewmats[b, c, 3, 3] = 1
    Ks = np.zeros((B, C, 3, 3))
    Ks[..., 0, 0] = 300
    Ks[..., 1, 1] = 280
    Ks[..., 0, 2] = 160
    Ks[..., 1, 2] = 120
    Ks[..., 2, 2] = 1
    return [a.astype(dtype) for a in (means, quats, scales, viewmats, Ks)]


def test_textbook_ewa(oracle):
    """Independent restatement: world->camera with [R|t], Sigma_c = R Sigma R^T
    with Sigma = R_q diag(s^2) R_q^T (scipy), J of the pinhole projection at the
    camera-space mean, conic = (J Sigma_c J^T + eps I)^-1."""
    rng = np.random.default_rng(3)
    means, quats, scales, viewmats, Ks = _random_scene(rng, 1, 2, 200)
    out = oracle.projection_forward(means, viewmats, Ks, 320, 240, quats=quats, scales=scales)
    Rq = Rotation.from_quat(quats[0][:, [1, 2, 3, 0]]).as_matrix()
    Sig = Rq @ (scales[0][:, :, None] ** 2 * np.swapaxes(Rq, -1, -2))
    checked = 0
    for c in range(2):
        R, t = viewmats[0, c, :3, :3], viewmats[0, c, :3, 3]
        fx, fy, cx, cy = Ks[0, c, 0, 0], Ks[0, c, 1, 1], Ks[0, c, 0, 2], Ks[0, c, 1, 2]
        for n in range(200):
            if out["radii"][0, c, n, 0] == 0:
                continue
            p = R @ means[0, n] + t
            x, y, z = p
            # inside the 1.3x frustum the clamp is inactive
            if abs(x / z) > 0.5 or abs(y / z) > 0.4:
                continue
            J = np.array([[fx / z, 0, -fx * x / z**2], [0, fy / z, -fy * y / z**2]])
            S2 = J @ R @ Sig[n] @ R.T @ J.T + 0.3 * np.eye(2)
            inv = np.linalg.inv(S2)
            np.testing.assert_allclose(out["means2d"][0, c, n], [fx * x / z + cx, fy * y / z + cy], rtol=1e-12)
            np.testing.assert_allclose(out["conics"][0, c, n], [inv[0, 0], inv[0, 1], inv[1, 1]], rtol=1e-7)
            np.testing.assert_allclose(out["depths"][0, c, n], z, rtol=1e-12)
            r = np.ceil(3.33 * np.sqrt(np.diag(S2)))
            np.testing.assert_array_equal(out["radii"][0, c, n], r)
            checked += 1
    assert checked > 100


def _fisheye_project(p, fx, fy, cx, cy):
    """Equidistant fisheye: image radius = f * theta, theta = angle to the
    optical axis (the model of gsplat_projection.metal:170-200)."""
    x, y, z = p
    r = np.hypot(x, y)
    theta = np.arctan2(r, z)
    return np.array([fx * theta * x / r + cx, fy * theta * y / r + cy])


@pytest.mark.parametrize("camera_model", [1, 2])
def test_textbook_ortho_and_fisheye(oracle, camera_model):
    """Orthographic (mean2d = f * (x, y) + c, J = diag(f) on x, y) and
    equidistant fisheye (J by central differences of the projection written
    above) against the oracle's camera models; conic = (J Sigma_c J^T + eps)^-1."""
    rng = np.random.default_rng(5 + camera_model)
    means, quats, scales, viewmats, Ks = _random_scene(rng, 1, 1, 150)
    out = oracle.projection_forward(means, viewmats, Ks, 320, 240, quats=quats, scales=scales,
                                    camera_model=camera_model)
    Rq = Rotation.from_quat(quats[0][:, [1, 2, 3, 0]]).as_matrix()
    Sig = Rq @ (scales[0][:, :, None] ** 2 * np.swapaxes(Rq, -1, -2))
    R, t = viewmats[0, 0, :3, :3], viewmats[0, 0, :3, 3]
    fx, fy, cx, cy = Ks[0, 0, 0, 0], Ks[0, 0, 1, 1], Ks[0, 0, 0, 2], Ks[0, 0, 1, 2]
    checked = 0
    for n in range(150):
        if out["radii"][0, 0, n, 0] == 0:
            continue
        p = R @ means[0, n] + t
        if camera_model == 1:
            m2 = np.array([fx * p[0] + cx, fy * p[1] + cy])
            J = np.array([[fx, 0, 0], [0, fy, 0]])
            tol = 1e-9
        else:
            m2 = _fisheye_project(p, fx, fy, cx, cy)
            h = 1e-6
            J = np.stack([(_fisheye_project(p + h * e, fx, fy, cx, cy) - _fisheye_project(p - h * e, fx, fy, cx, cy))
                          / (2 * h) for e in np.eye(3)], axis=1)
            tol = 1e-5  # the model's 1e-7 regularisers and the difference step
        S2 = J @ R @ Sig[n] @ R.T @ J.T + 0.3 * np.eye(2)
        inv = np.linalg.inv(S2)
        np.testing.assert_allclose(out["means2d"][0, 0, n], m2, rtol=tol)
        np.testing.assert_allclose(out["conics"][0, 0, n], [inv[0, 0], inv[0, 1], inv[1, 1]], rtol=tol,
                                   atol=tol * np.abs(inv).max())
        np.testing.assert_allclose(out["depths"][0, 0, n], p[2], rtol=1e-12)
        checked += 1
    assert checked > 50


def _proj_loss(oracle, means, quats, scales, covars, viewmats, Ks, cot, fixed_radii, calc_comp, camera_model=0):
    kw = dict(covars=covars) if covars is not None else dict(quats=quats, scales=scales)
    out = oracle.projection_forward(means, viewmats, Ks, 320, 240, calc_compensations=calc_comp,
                                    camera_model=camera_model, **kw)
    assert np.array_equal(out["radii"] > 0, fixed_radii > 0)  # no culling change under perturbation
    loss = np.sum(out["means2d"] * cot["v_means2d"]) + np.sum(out["depths"] * cot["v_depths"]) + \
        np.sum(out["conics"] * cot["v_conics"])
    if calc_comp:
        loss += np.sum(out["compensations"] * cot["v_compensations"])
    return loss


@pytest.mark.parametrize("use_covars", [False, True])
@pytest.mark.parametrize("calc_comp", [False, True])
@pytest.mark.parametrize("camera_model", [0, 1, 2])  # pinhole, orthographic, fisheye
def test_backward_finite_differences(oracle, use_covars, calc_comp, camera_model):
    rng = np.random.default_rng(5)
    B, C, N = 1, 2, 6
    means, quats, scales, viewmats, Ks = _random_scene(rng, B, C, N)
    means[..., 0] *= 0.3
    means[..., 1] *= 0.3
    covars = None
    if use_covars:
        covars, _ = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, False, True)
        covars = np.ascontiguousarray(covars)
    kw = dict(covars=covars) if use_covars else dict(quats=quats, scales=scales)
    fwd = oracle.projection_forward(means, viewmats, Ks, 320, 240, calc_compensations=calc_comp,
                                    camera_model=camera_model, **kw)
    assert np.all(fwd["radii"] > 0)
    cot = {"v_means2d": rng.normal(size=fwd["means2d"].shape), "v_depths": rng.normal(size=fwd["depths"].shape),
           "v_conics": rng.normal(size=fwd["conics"].shape) * 10,
           "v_compensations": rng.normal(size=fwd["depths"].shape)}
    bwd = oracle.projection_backward(means, viewmats, Ks, 320, 240, fwd["radii"], fwd["conics"], cot["v_means2d"],
                                     cot["v_depths"], cot["v_conics"],
                                     compensations=fwd["compensations"] if calc_comp else None,
                                     v_compensations=cot["v_compensations"] if calc_comp else None,
                                     viewmats_requires_grad=True, camera_model=camera_model, **kw)
    params = {"means": means, "viewmats": viewmats}
    if use_covars:
        params["covars"] = covars
    else:
        params["quats"] = quats
        params["scales"] = scales
    h = 1e-6
    for name, arr in params.items():
        grad = bwd["v_" + name]
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            if name == "viewmats" and idx[-2] == 3:
                continue  # bottom row is not an input of the projection
            a0 = arr[idx]
            arr[idx] = a0 + h
            lp = _proj_loss(oracle, means, quats, scales, covars, viewmats, Ks, cot, fwd["radii"], calc_comp,
                            camera_model)
            arr[idx] = a0 - h
            lm = _proj_loss(oracle, means, quats, scales, covars, viewmats, Ks, cot, fwd["radii"], calc_comp,
                            camera_model)
            arr[idx] = a0
            num[idx] = (lp - lm) / (2 * h)
        if name == "covars":
            # triu cotangent convention: off-diagonal grads hold the sum of the
            # symmetric pair (gsplat_projection.cpp:1089-1095); the triu forward
            # input is read once per symmetric pair, so FD gives the same sum.
            pass
        scale = np.abs(num).max()
        # central differences with h = 1e-6 in float64 leave ~1e-7 absolute
        # noise; the orthographic quaternion gradients are smaller, so their
        # relative bound is looser
        rtol = 2e-5 if camera_model == 0 else 1e-4
        np.testing.assert_allclose(grad, num, rtol=rtol, atol=2e-6 * scale, err_msg=name)
