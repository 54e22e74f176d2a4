"""Pins the oracle's quat_scale_to_covar_preci against the reference's known
answers (gsplat_core/test/test.cpp:1690-1954) and against independent math
(scipy rotations, matrix inverse, float64 finite differences)."""
import numpy as np
import pytest
from scipy.spatial.transform import Rotation


def test_forward_known_answers(oracle):
    # test.cpp:1690-1757
    quats = np.array([[1, 0, 0, 0], [2, 0, 0, 0]], np.float32)
    scales = np.array([[2, 3, 4], [0.5, 2, 4]], np.float32)
    covars, precis = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, True, True)
    np.testing.assert_allclose(covars, [[4, 0, 0, 9, 0, 16], [0.25, 0, 0, 4, 0, 16]], atol=1e-6)
    np.testing.assert_allclose(precis, [[0.25, 0, 0, 1 / 9, 0, 1 / 16], [4, 0, 0, 0.25, 0, 1 / 16]], atol=1e-6)
    full, empty = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, False, False)
    assert full.shape == (2, 3, 3) and empty.shape == (0,)
    np.testing.assert_allclose(full[0], np.diag([4, 9, 16]), atol=1e-6)


def _rot_wxyz(q):
    q = np.asarray(q, np.float64)
    return Rotation.from_quat(q[..., [1, 2, 3, 0]]).as_matrix()  # scipy wants xyzw


def test_forward_matches_scipy_rotation_and_inverse(oracle):
    # test.cpp:1832-1876 inputs plus random ones; R from scipy (independent).
    rng = np.random.default_rng(0)
    quats = np.concatenate([np.array([[0.35, 0.2, -0.4, 0.8], [2.0, -1.0, 0.5, 0.25], [1, 0, 0, 0]]),
                            rng.normal(size=(64, 4))]).astype(np.float64)
    scales = np.concatenate([np.array([[0.5, 1.5, 2.5], [2.0, 0.75, 1.25], [0.25, 3.0, 4.0]]),
                             np.exp(rng.uniform(-2, 1, size=(64, 3)))]).astype(np.float64)
    covars, precis = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, True, False)
    R = _rot_wxyz(quats)
    expect_cov = R @ (scales[:, :, None] ** 2 * np.swapaxes(R, -1, -2))
    expect_pre = R @ (scales[:, :, None] ** -2 * np.swapaxes(R, -1, -2))
    np.testing.assert_allclose(covars, expect_cov, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(precis, expect_pre, rtol=1e-10, atol=1e-12)
    eye = covars @ precis
    np.testing.assert_allclose(eye, np.broadcast_to(np.eye(3), eye.shape), atol=1e-9)
    # float32 instantiation agrees with float64 to fp32 precision
    c32, p32 = oracle.quat_scale_to_covar_preci_forward(quats.astype(np.float32), scales.astype(np.float32), True, True, True)
    c64, p64 = oracle.quat_scale_to_covar_preci_forward(quats, scales, True, True, True)
    np.testing.assert_allclose(c32, c64, rtol=1e-5, atol=1e-6 * np.abs(c64).max())
    np.testing.assert_allclose(p32, p64, rtol=1e-5, atol=1e-6 * np.abs(p64).max())


def test_backward_known_answers(oracle):
    # test.cpp:1878-1954
    quats = np.array([[1, 0, 0, 0], [0.9238795, 0.3826834, 0, 0]], np.float32)
    scales = np.array([[2, 3, 4], [0.5, 1.5, 2.5]], np.float32)
    v_covars = np.array([[0.1, 0, 0, 0.2, 0, 0.3], [-0.2, 0.05, 0.1, 0.4, -0.15, 0.25]], np.float32)
    v_precis = np.array([[0.4, 0, 0, 0.5, 0, 0.6], [0.3, -0.25, 0.35, -0.1, 0.2, 0.45]], np.float32)
    v_quats, v_scales = oracle.quat_scale_to_covar_preci_backward(quats, scales, v_covars, v_precis, True)
    np.testing.assert_allclose(v_scales[0], [0.3, 1.2 - 1 / 27, 2.4 - 0.01875], atol=3e-3)
    np.testing.assert_allclose(v_quats[0], 0.0, atol=3e-3)
    zq, zs = oracle.quat_scale_to_covar_preci_backward(quats, scales, None, None, True)
    assert np.all(zq == 0) and np.all(zs == 0)


def _loss(oracle, q, s, vc, vp, triu):
    c, p = oracle.quat_scale_to_covar_preci_forward(q, s, vc is not None, vp is not None, triu)
    out = 0.0
    if vc is not None:
        out += np.sum(c * vc)
    if vp is not None:
        out += np.sum(p * vp)
    return out


@pytest.mark.parametrize("triu", [True, False])
@pytest.mark.parametrize("which", ["covar", "preci", "both"])
def test_backward_finite_differences(oracle, triu, which):
    """Analytic VJP (float64 instantiation) against central differences of the
    float64 forward. For triu the cotangent of an off-diagonal entry applies
    to the symmetric pair, which is what the forward's triu output encodes."""
    rng = np.random.default_rng(1)
    n = 16
    q = rng.normal(size=(n, 4))
    s = np.exp(rng.uniform(-1, 0.5, size=(n, 3)))
    shape = (n, 6) if triu else (n, 3, 3)
    vc = rng.normal(size=shape) if which in ("covar", "both") else None
    vp = rng.normal(size=shape) if which in ("preci", "both") else None
    if not triu:  # reference treats a full cotangent as-is; use symmetric ones
        vc = None if vc is None else 0.5 * (vc + np.swapaxes(vc, -1, -2))
        vp = None if vp is None else 0.5 * (vp + np.swapaxes(vp, -1, -2))
    v_q, v_s = oracle.quat_scale_to_covar_preci_backward(q, s, vc, vp, triu)
    h = 1e-6
    for arr, grad in ((q, v_q), (s, v_s)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            a0 = arr[idx]
            arr[idx] = a0 + h
            lp = _loss(oracle, q, s, vc, vp, triu)
            arr[idx] = a0 - h
            lm = _loss(oracle, q, s, vc, vp, triu)
            arr[idx] = a0
            num[idx] = (lp - lm) / (2 * h)
        np.testing.assert_allclose(grad, num, rtol=1e-5, atol=1e-7)
