"""Pins the oracle's spherical harmonics: the reference's closed forms
(gsplat_core/test/test.cpp:1388-1688), the real-SH basis against scipy's
complex spherical harmonics (with the Condon-Shortley phase), and float64
finite differences of the forward for v_dirs."""
import numpy as np
import pytest
import scipy.special as sp

C0 = 0.2820947917738781
C1 = 0.48860251190292

COEFFS_2x4 = np.array([[[1, 2, 3], [0.1, 0.2, 0.3], [0.4, 0.5, 0.6], [0.7, 0.8, 0.9]],
                       [[4, 5, 6], [0, 0, 0], [0, 0, 0], [0, 0, 0]]], np.float32)
DIRS_2 = np.array([[0, 0, 1], [1, 0, 0]], np.float32)


def test_forward_closed_forms(oracle):
    # test.cpp:1388-1457
    d0 = oracle.sh_forward(0, DIRS_2, COEFFS_2x4)
    np.testing.assert_allclose(d0, [[C0, 2 * C0, 3 * C0], [4 * C0, 5 * C0, 6 * C0]], atol=1e-6)
    d1 = oracle.sh_forward(1, DIRS_2, COEFFS_2x4)
    np.testing.assert_allclose(d1[0], [C0 + C1 * 0.4, 2 * C0 + C1 * 0.5, 3 * C0 + C1 * 0.6], atol=1e-6)
    np.testing.assert_allclose(d1[1], [4 * C0, 5 * C0, 6 * C0], atol=1e-6)
    masked = oracle.sh_forward(0, DIRS_2, COEFFS_2x4, masks=np.array([True, False]))
    np.testing.assert_allclose(masked[0], [C0, 2 * C0, 3 * C0], atol=1e-6)
    assert np.all(masked[1] == 0)


def _scipy_real_basis(degree, dirs):
    """Real SH in the 3DGS convention from scipy's complex Y_l^m (which includes
    the Condon-Shortley phase): m<0 -> sqrt2 Im Y_l^|m|, m=0 -> Y_l^0,
    m>0 -> sqrt2 Re Y_l^m, at index l^2 + l + m."""
    d = dirs / np.linalg.norm(dirs, axis=-1, keepdims=True)
    polar = np.arccos(np.clip(d[:, 2], -1, 1))
    azim = np.arctan2(d[:, 1], d[:, 0])
    out = np.zeros((len(d), (degree + 1) ** 2))
    for l in range(degree + 1):
        for m in range(-l, l + 1):
            Y = sp.sph_harm_y(l, abs(m), polar, azim)
            if m < 0:
                v = np.sqrt(2) * Y.imag
            elif m == 0:
                v = Y.real
            else:
                v = np.sqrt(2) * Y.real
            out[:, l * l + l + m] = v
    return out


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 4])
def test_basis_matches_scipy(oracle, degree):
    rng = np.random.default_rng(degree)
    n = 64
    K = (degree + 1) ** 2
    dirs = rng.normal(size=(n, 3))
    expect = _scipy_real_basis(degree, dirs)
    # v_coeffs = basis (x) v_colors exposes every basis value (test.cpp:1599-1607)
    v_colors = np.ones((n, 3))
    _, v_coeffs = oracle.sh_backward(degree, dirs, rng.normal(size=(n, K, 3)), v_colors, compute_v_dirs=False)
    np.testing.assert_allclose(v_coeffs[:, :, 0], expect, rtol=1e-12, atol=1e-13)
    # the forward is the basis-weighted sum
    coeffs = rng.normal(size=(n, K, 3))
    colors = oracle.sh_forward(degree, dirs, coeffs)
    np.testing.assert_allclose(colors, np.einsum("nk,nkc->nc", expect, coeffs), rtol=1e-11, atol=1e-12)


def test_backward_closed_form(oracle):
    # test.cpp:1563-1623
    dirs = np.array([[0, 0, 1]], np.float32)
    coeffs = COEFFS_2x4[:1]
    v_colors = np.array([[1, 2, 3]], np.float32)
    v_dirs, v_coeffs = oracle.sh_backward(1, dirs, coeffs, v_colors)
    np.testing.assert_allclose(v_coeffs[0, 0], [C0, 2 * C0, 3 * C0], atol=1e-6)
    np.testing.assert_allclose(v_coeffs[0, 2], [C1, 2 * C1, 3 * C1], atol=1e-6)
    np.testing.assert_allclose(v_dirs[0], [-C1 * 5, -C1 * 1.4, 0], atol=5e-4)
    nd, _ = oracle.sh_backward(1, dirs, coeffs, v_colors, compute_v_dirs=False)
    assert nd.shape == (0,)


def test_masks_and_inactive_bands(oracle):
    # test.cpp:1511-1561, 1625-1688 inputs: degree-4 coefficient ramp, masks
    dirs = np.array([[0.25, -0.5, 1.0], [-0.75, 0.1, 0.6], [0.2, 0.3, -0.4]], np.float32)
    coeffs = (0.01 * (1 + np.arange(3 * 25 * 3))).reshape(3, 25, 3).astype(np.float32)
    masks = np.array([True, False, True])
    v_colors = np.array([[0.3, -0.2, 0.7], [1, 2, 3], [-0.4, 0.5, 0.25]], np.float32)
    colors = oracle.sh_forward(4, dirs, coeffs, masks)
    assert np.all(colors[1] == 0)
    v_dirs, v_coeffs = oracle.sh_backward(4, dirs, coeffs, v_colors, masks)
    assert np.all(v_dirs[1] == 0) and np.all(v_coeffs[1] == 0)
    # degree 2 uses only 9 of the 25 bases: inactive gradient rows are zero
    _, vc2 = oracle.sh_backward(2, dirs, coeffs, v_colors)
    assert np.all(vc2[:, 9:] == 0) and np.any(vc2[:, :9] != 0)
    # zero direction: DC only, no direction gradient
    zd = np.zeros((1, 3), np.float32)
    c = oracle.sh_forward(3, zd, coeffs[:1, :16])
    np.testing.assert_allclose(c[0], C0 * coeffs[0, 0], rtol=1e-6)
    vd, _ = oracle.sh_backward(3, zd, coeffs[:1, :16], v_colors[:1])
    assert np.all(vd == 0)


@pytest.mark.parametrize("degree", [1, 2, 3, 4])
def test_dir_gradient_finite_differences(oracle, degree):
    rng = np.random.default_rng(10 + degree)
    n, K = 8, 25
    dirs = rng.normal(size=(n, 3))
    coeffs = rng.normal(size=(n, K, 3))
    v_colors = rng.normal(size=(n, 3))
    v_dirs, _ = oracle.sh_backward(degree, dirs, coeffs, v_colors)
    h = 1e-6
    num = np.zeros_like(dirs)
    for idx in np.ndindex(dirs.shape):
        a0 = dirs[idx]
        dirs[idx] = a0 + h
        lp = np.sum(oracle.sh_forward(degree, dirs, coeffs) * v_colors)
        dirs[idx] = a0 - h
        lm = np.sum(oracle.sh_forward(degree, dirs, coeffs) * v_colors)
        dirs[idx] = a0
        num[idx] = (lp - lm) / (2 * h)
    np.testing.assert_allclose(v_dirs, num, rtol=1e-6, atol=1e-8)
