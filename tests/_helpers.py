"""Shared helpers for the GPU parity tests (not collected by pytest)."""
from __future__ import annotations

import numpy as np
import pytest

try:
    import torch
except ImportError:  # pragma: no cover
    torch = None


def gpu_available() -> bool:
    return torch is not None and torch.cuda.is_available()


requires_gpu = pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")


def dev(a, dtype=None):
    """numpy -> contiguous torch tensor on cuda:0."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


# Radii are ceil() of float expressions that the kernels evaluate in the
# oracle's order; a last-ulp difference (sqrt, log of the opacity-aware
# extent) can still move one across an integer. The parity tests count such
# Gaussians, print the count and allow at most this many per check.
MAX_RADIUS_FLIPS = 2

FLOOR_ATOMIC = 1e-2  # sums whose float order differs from the oracle's (atomics, chained stages)
FLOOR_ORDERED = 1e-4  # per-element results computed without atomics (projection, SH, activations)


def assert_close_rel(actual, expected, rtol, name="", scale_floor=0.0, floor_rel=FLOOR_ATOMIC):
    """|a - e| <= rtol * max(|e|, s) elementwise with s = max(floor_rel *
    max|e|, scale_floor): relative to each element, but elements much smaller
    than the tensor's largest magnitude are held to rtol * s absolute
    (cancellation-prone values carry no relative information). Prints how
    many elements meet the bar only through that floor (off by more than
    rtol * |e|) and returns the count."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    if e.size == 0:
        return 0
    floor = max(np.abs(e).max() * floor_rel, scale_floor)
    err = np.abs(a - e)
    tol = rtol * np.maximum(np.abs(e), floor)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), e.shape)
        raise AssertionError(f"{name}: {bad.sum()} / {e.size} elements off; worst at {i}: got {a[i]!r}, "
                             f"expected {e[i]!r} (tol {tol[i]:.3g})")
    via_floor = int(np.count_nonzero(err > rtol * np.abs(e)))
    print(f"[parity] {name or 'tensor'}: rtol {rtol:g}, floor {floor_rel:g}*max; {via_floor} of {e.size} "
          f"elements pass only through the floor", flush=True)
    return via_floor


def assert_close_rel_summation(actual, expected, rtol, name="", outlier_rtol=1e-2, outliers_per_million=1.0):
    """assert_close_rel for two results of the same arithmetic summed in
    different orders (float atomics in another order, or over different but
    equivalent entry lists): every element within outlier_rtol, and at most
    outliers_per_million elements per million (at least 2) beyond rtol. Sums
    with heavy cancellation can differ by more than rtol between two valid
    float32 summation orders."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert_close_rel(a, e, outlier_rtol, name)
    if e.size == 0:
        return
    floor = np.abs(e).max() * 1e-2
    beyond = np.abs(a - e) > rtol * np.maximum(np.abs(e), floor)
    allowed = max(2, int(outliers_per_million * e.size / 1e6))
    assert beyond.sum() <= allowed, f"{name}: {beyond.sum()} / {e.size} elements beyond {rtol} (allowed {allowed})"


def gsplat():
    import gsplat_core

    return gsplat_core


def projected_scene(rng, I, N, W, H, anisotropy=30.0):
    """Random screen-space Gaussians as the projection would give them:
    2D covariances with eps2d = 0.3 added, conics = inverses, radii from the
    opacity-aware extent (gsplat_projection.metal:299-313)."""
    s1 = rng.uniform(0.4, 12.0, (I, N))
    s2 = s1 * rng.uniform(1.0, anisotropy, (I, N)) ** rng.choice([0.0, 1.0], (I, N), p=[0.3, 0.7])
    th = rng.uniform(0, np.pi, (I, N))
    c, s = np.cos(th), np.sin(th)
    cxx = c * c * s1 * s1 + s * s * s2 * s2 + 0.3
    cyy = s * s * s1 * s1 + c * c * s2 * s2 + 0.3
    cxy = c * s * (s1 * s1 - s2 * s2)
    det = cxx * cyy - cxy * cxy
    conics = np.stack([cyy / det, -cxy / det, cxx / det], -1).astype(np.float32)
    opac = rng.uniform(0.001, 1.0, (I, N)).astype(np.float32)
    extend = np.minimum(3.33, np.sqrt(2.0 * np.log(np.maximum(opac * 255.0, 1.0))))
    extend = np.where(rng.random((I, N)) < 0.3, 3.33, extend)  # some callers pass no opacities to the projection
    radii = np.stack([np.ceil(extend * np.sqrt(cxx)), np.ceil(extend * np.sqrt(cyy))], -1).astype(np.int32)
    means = np.stack([rng.uniform(-20, W + 20, (I, N)), rng.uniform(-20, H + 20, (I, N))], -1).astype(np.float32)
    depths = rng.uniform(0.5, 10.0, (I, N)).astype(np.float32)
    return means, radii, conics, opac, depths
