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


def assert_close_rel(actual, expected, rtol, name="", scale_floor=0.0):
    """|a - e| <= rtol * max(|e|, s) elementwise with s = rtol-scaled norm floor:
    relative to each element, but elements much smaller than the tensor's
    largest magnitude are held to rtol * max|e| * 1e-2 (cancellation-prone
    values carry no relative information)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    if e.size == 0:
        return
    floor = max(np.abs(e).max() * 1e-2, scale_floor)
    err = np.abs(a - e)
    tol = rtol * np.maximum(np.abs(e), floor)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), e.shape)
        raise AssertionError(f"{name}: {bad.sum()} / {e.size} elements off; worst at {i}: got {a[i]!r}, "
                             f"expected {e[i]!r} (tol {tol[i]:.3g})")


def gsplat():
    import gsplat_core

    return gsplat_core
