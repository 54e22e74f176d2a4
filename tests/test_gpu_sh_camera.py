"""GPU parity of the fused camera-colour SH path against (1) the oracle's SH
wrapped in a numpy restatement of the caller glue of
scanner_points_training_utils.py:1005-1034 (camera centre -R^T t of each view
matrix, normalise means - campos with max(|d|, 1e-8), concat [dc, rest],
clip(SH + 0.5, 0, 1)), and (2) the unfused torch composition (elementwise ops
+ the SH operator) with autograd.

Tolerances: colours within 1e-5 relative, gradients within 1e-3 relative
(_helpers.assert_close_rel). Inputs are nudged away from the clip bounds so
the clip masks cannot differ by rounding."""
import numpy as np
import pytest

from _helpers import FLOOR_ORDERED, assert_close_rel, dev, gsplat, host

pytestmark = pytest.mark.gpu

FWD_RTOL = 1e-5
GRAD_RTOL = 1e-3


def _views(rng, B, C):
    """Random view matrices [B, C, 4, 4] and their centres -R^T t, computed
    with the kernel's float32 operation order (so a mean placed at a centre
    gives d = 0 exactly)."""
    from scipy.spatial.transform import Rotation

    vm = np.zeros((B, C, 4, 4), np.float32)
    vm[..., 3, 3] = 1
    vm[..., :3, :3] = Rotation.random(B * C, random_state=int(rng.integers(1 << 30))).as_matrix().reshape(B, C, 3, 3)
    vm[..., :3, 3] = rng.normal(size=(B, C, 3))
    R, t = vm[..., :3, :3], vm[..., :3, 3]
    campos = np.empty((B, C, 3), np.float32)
    for i in range(3):
        campos[..., i] = -((R[..., 0, i] * t[..., 0] + R[..., 1, i] * t[..., 1]) + R[..., 2, i] * t[..., 2])
    return vm, campos


def _oracle_forward(oracle, degree, means, campos, dc, rest):
    """colors [B, C, N, 3] and the per-camera normalised dirs / norms."""
    A = (degree + 1) ** 2
    B, N, _ = means.shape
    C = campos.shape[1]
    coeffs = np.concatenate([dc[:, :, None, :], rest[:, :, : A - 1, :]], axis=2).astype(np.float32)
    raw = np.zeros((B, C, N, 3), np.float32)
    dirs = np.zeros((B, C, N, 3), np.float32)
    norms = np.zeros((B, C, N), np.float32)
    for b in range(B):
        for c in range(C):
            d = (means[b] - campos[b, c]).astype(np.float32)
            nrm = np.sqrt(np.sum(d * d, axis=-1)).astype(np.float32)
            n = (d / np.maximum(nrm, np.float32(1e-8))[:, None]).astype(np.float32)
            dirs[b, c], norms[b, c] = n, nrm
            raw[b, c] = oracle.sh_forward(degree, n, coeffs[b])
    return raw, dirs, norms, coeffs


def _nudge_off_bounds(oracle, degree, means, campos, dc, rest):
    for _ in range(10):
        raw, _, _, _ = _oracle_forward(oracle, degree, means, campos, dc, rest)
        x = raw + 0.5
        near = (np.abs(x) < 1e-3) | (np.abs(x - 1) < 1e-3)
        if not near.any():
            return dc
        hit = near.any(axis=(1,)).any(axis=-1)  # [B, N]
        dc[hit] += 0.0123
    raise AssertionError("could not move the colours off the clip bounds")


def _oracle_backward(oracle, degree, means, campos, coeffs, raw, dirs, norms, v_colors, R):
    B, C, N, _ = raw.shape
    A = (degree + 1) ** 2
    x = raw + 0.5
    g = np.where((x >= 0) & (x <= 1), v_colors, 0).astype(np.float32)
    v_means = np.zeros((B, N, 3))
    v_co = np.zeros((B, N, A, 3))
    for b in range(B):
        for c in range(C):
            v_n, v_c = oracle.sh_backward(degree, dirs[b, c], coeffs[b], g[b, c])
            v_co[b] += v_c
            n = dirs[b, c].astype(np.float64)
            nrm = norms[b, c].astype(np.float64)[:, None]
            v_n = v_n.astype(np.float64)
            dot = np.sum(v_n * n, axis=-1, keepdims=True)
            v_means[b] += np.where(nrm >= 1e-8, (v_n - n * dot) / np.maximum(nrm, 1e-30), v_n / 1e-8)
    v_dc = v_co[:, :, 0]
    v_rest = np.zeros((B, N, R, 3))
    v_rest[:, :, : A - 1] = v_co[:, :, 1:]
    return v_means, v_dc, v_rest


# R == (degree+1)^2 - 1 with degree 0, 1, 3 takes the slab kernels (B = 2
# with N = 3001 also exercises their unaligned path); the rest the general ones
@pytest.mark.parametrize("degree,B,C,R", [(0, 1, 1, 0), (1, 1, 2, 3), (2, 2, 1, 15), (3, 1, 1, 15),
                                          (3, 2, 3, 15), (4, 1, 2, 24), (0, 1, 2, 15), (1, 2, 1, 15),
                                          (2, 1, 1, 8)])
def test_fused_vs_oracle(oracle, degree, B, C, R):
    g = gsplat()
    rng = np.random.default_rng(degree * 100 + C * 10 + R)
    N = 3001  # not a multiple of the block size
    means = (rng.normal(size=(B, N, 3)) * 2 + [0, 0, 6]).astype(np.float32)
    vm, campos = _views(rng, B, C)
    means[0, 5] = campos[0, 0]  # a Gaussian at a camera centre: DC only
    dc = rng.normal(scale=0.3, size=(B, N, 3)).astype(np.float32)
    rest = rng.normal(scale=0.1, size=(B, N, R, 3)).astype(np.float32)
    dc = _nudge_off_bounds(oracle, degree, means, campos, dc, rest)
    raw, dirs, norms, coeffs = _oracle_forward(oracle, degree, means, campos, dc, rest)
    inputs = {"means": dev(means), "viewmats": dev(vm), "features_dc": dev(dc), "features_rest": dev(rest)}
    colors = host(g._gsplat_core.sh_camera_colors_forward(degree, inputs))
    assert colors.shape == (B, C, N, 3)
    assert_close_rel(colors, np.clip(raw + 0.5, 0, 1), FWD_RTOL, "colors", floor_rel=FLOOR_ORDERED)
    v_colors = rng.normal(size=(B, C, N, 3)).astype(np.float32)
    out = g._gsplat_core.sh_camera_colors_backward(degree, inputs, {"v_colors": dev(v_colors)})
    ev_means, ev_dc, ev_rest = _oracle_backward(oracle, degree, means, campos, coeffs, raw, dirs, norms, v_colors, R)
    assert_close_rel(host(out["v_features_dc"]), ev_dc, GRAD_RTOL, "v_features_dc", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(out["v_features_rest"]), ev_rest, GRAD_RTOL, "v_features_rest", floor_rel=FLOOR_ORDERED)
    assert_close_rel(host(out["v_means"]), ev_means, GRAD_RTOL, "v_means", floor_rel=FLOOR_ORDERED)


# The slab forward is a resident grid: with a few hundred thousand Gaussians
# each wave walks several groups of 64 (prefetching the next), and with B = 2
# and odd N the second batch's groups are not 16-byte aligned.
@pytest.mark.parametrize("B,N", [(1, 400003), (2, 200001)])
def test_slab_forward_walks_groups(oracle, B, N):
    g = gsplat()
    rng = np.random.default_rng(N)
    degree, C = 3, 1
    means = (rng.normal(size=(B, N, 3)) * 2 + [0, 0, 6]).astype(np.float32)
    vm, campos = _views(rng, B, C)
    dc = rng.normal(scale=0.3, size=(B, N, 3)).astype(np.float32)
    rest = rng.normal(scale=0.1, size=(B, N, 15, 3)).astype(np.float32)
    raw, _, _, _ = _oracle_forward(oracle, degree, means, campos, dc, rest)
    inputs = {"means": dev(means), "viewmats": dev(vm), "features_dc": dev(dc), "features_rest": dev(rest)}
    colors = host(g._gsplat_core.sh_camera_colors_forward(degree, inputs))
    exp = np.clip(raw + 0.5, 0, 1)
    # the clip makes a rounding difference at a bound visible as a jump;
    # compare away from the bounds and require the clipped values to agree
    inner = (raw + 0.5 > 1e-4) & (raw + 0.5 < 1 - 1e-4)
    assert inner.mean() > 0.9
    assert_close_rel(colors[inner], exp[inner], FWD_RTOL, "colors", floor_rel=FLOOR_ORDERED)
    np.testing.assert_array_equal(colors[~inner] > 0.5, exp[~inner] > 0.5)


def test_fused_matches_unfused_torch_autograd(oracle):
    import torch

    from gsplat_core import render as Rn

    rng = np.random.default_rng(7)
    N, degree = 4099, 3
    means = (rng.normal(size=(1, N, 3)) * 2 + [0, 0, 6]).astype(np.float32)
    vm = np.eye(4, dtype=np.float32)[None, None].copy()
    vm[0, 0, :3, 3] = [0.3, -0.2, 0.5]
    campos = -vm[0, 0, :3, :3].T @ vm[0, 0, :3, 3]
    dc = rng.normal(scale=0.3, size=(1, N, 3)).astype(np.float32)
    rest = rng.normal(scale=0.05, size=(1, N, 15, 3)).astype(np.float32)
    dc = _nudge_off_bounds(oracle, degree, means, campos[None, None].astype(np.float32), dc, rest)
    v = rng.normal(size=(1, 1, N, 3)).astype(np.float32)

    def run(fn):
        m, d, r = (dev(a).requires_grad_(True) for a in (means, dc, rest))
        out = fn(m, d, r, dev(vm), degree)
        out.backward(dev(v))
        return host(out), host(m.grad), host(d.grad), host(r.grad)

    fused = run(Rn.sh_colors_for_camera)
    plain = run(Rn.sh_colors_for_camera_unfused)
    for a, e, name in zip(fused, plain, ["colors", "v_means", "v_dc", "v_rest"]):
        assert_close_rel(a, e, FWD_RTOL if name == "colors" else GRAD_RTOL, name, floor_rel=FLOOR_ORDERED)
    del torch


def test_errors():
    g = gsplat()
    z = lambda *s: dev(np.zeros(s, np.float32))  # noqa: E731
    with pytest.raises(RuntimeError, match="fewer SH bases"):
        g._gsplat_core.sh_camera_colors_forward(3, {"means": z(1, 4, 3), "viewmats": z(1, 1, 4, 4),
                                                    "features_dc": z(1, 4, 3), "features_rest": z(1, 4, 8, 3)})
    with pytest.raises(RuntimeError, match="features_dc"):
        g._gsplat_core.sh_camera_colors_forward(1, {"means": z(1, 4, 3), "viewmats": z(1, 1, 4, 4),
                                                    "features_dc": z(1, 5, 3), "features_rest": z(1, 4, 3, 3)})


# With the projection's radii, the forward skips the rows that no camera
# sees (radii not both positive in any camera: no tile, so no render reads
# them): colour 0. Every other row runs the same arithmetic as without radii,
# so its colours agree bit for bit with the unmasked kernel's. Slab and
# general kernels, one and three cameras, partial and unaligned groups, and
# the resident-grid walk.
@pytest.mark.parametrize("degree,B,C,R,N", [(3, 1, 1, 15, 3001), (3, 2, 1, 15, 200001), (3, 1, 3, 15, 3001),
                                            (1, 2, 2, 3, 3001), (0, 1, 1, 0, 777), (2, 1, 1, 8, 3001),
                                            (4, 2, 3, 24, 1500), (3, 1, 1, 15, 64)])
@pytest.mark.parametrize("unseen", [0.37, 0.0, 1.0])
def test_radii_skip_unseen_rows(degree, B, C, R, N, unseen):
    g = gsplat()
    rng = np.random.default_rng(degree * 1000 + B * 100 + C * 10 + int(unseen * 10))
    means = (rng.normal(size=(B, N, 3)) * 2 + [0, 0, 6]).astype(np.float32)
    vm, _ = _views(rng, B, C)
    dc = rng.normal(scale=0.3, size=(B, N, 3)).astype(np.float32)
    rest = rng.normal(scale=0.1, size=(B, N, R, 3)).astype(np.float32)
    # radii [B, C, N, 2]: unseen rows get zero or one-sided radii in every
    # camera; seen rows are seen by one random camera at least
    radii = rng.integers(1, 30, size=(B, C, N, 2)).astype(np.int32)
    seen_any = rng.random((B, N)) >= unseen
    for c in range(C):
        off = ~seen_any | (rng.random((B, N)) < 0.5)
        kind = rng.integers(0, 3, size=(B, N))
        radii[:, c, :, 0] = np.where(off & (kind != 1), 0, radii[:, c, :, 0])
        radii[:, c, :, 1] = np.where(off & (kind != 2), -1 * (kind == 0), radii[:, c, :, 1])
    first = rng.integers(0, C, size=(B, N))
    for c in range(C):
        pick = seen_any & (first == c)
        radii[:, c][pick] = np.maximum(radii[:, c][pick], 1)
    seen = ((radii[..., 0] > 0) & (radii[..., 1] > 0)).any(axis=1)  # [B, N]
    assert (seen == seen_any).all()
    base = {"means": dev(means), "viewmats": dev(vm), "features_dc": dev(dc), "features_rest": dev(rest)}
    masked = dict(base, radii=dev(radii))
    print(f"sh camera radii skip: degree={degree} B={B} C={C} R={R} N={N} unseen={unseen}", flush=True)
    full = host(g._gsplat_core.sh_camera_colors_forward(degree, base))
    part = host(g._gsplat_core.sh_camera_colors_forward(degree, masked))
    exp = np.where(seen[:, None, :, None], full, 0.0)
    np.testing.assert_array_equal(part, exp)
