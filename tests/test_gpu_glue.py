"""GPU parity of the fused training-step glue against the framework (torch
fp32) compositions it replaces: the parameter activations
(scanner_points_training_utils.py:39-41, 306-316) and the image L1 term
(:1147-1160). Forward within 1e-6 relative (a different but equally exact
order of the same float operations; the L1 mean within 1e-5), gradients
within 1e-5 relative (L1: 1e-6, and the exact signs), plus
closed-form properties (unit quaternions, gradient orthogonal to q)."""
import numpy as np
import pytest

from _helpers import assert_close_rel, dev, gsplat, host

pytestmark = pytest.mark.gpu


def _inputs(rng, n):
    q = rng.normal(size=(1, n, 4)).astype(np.float32)
    q[0, 0] = [1e-12, 0, 0, 0]  # under the 1e-8 clamp
    # (an exactly zero quaternion is left out: the framework's sqrt backward
    # gives 0 * inf = NaN there, the fused kernel the clamp's v / 1e-8)
    ls = rng.normal(-4, 1.5, size=(1, n, 3)).astype(np.float32)
    lo = rng.normal(0, 3, size=(1, n)).astype(np.float32)
    lo[0, 2], lo[0, 3] = 40.0, -40.0  # saturated sigmoid
    return q, ls, lo


@pytest.mark.parametrize("n", [1, 1000, 100003])
def test_activations_vs_torch(n):
    import torch

    g = gsplat()
    from gsplat_core import render as R

    rng = np.random.default_rng(n)
    q, ls, lo = _inputs(rng, max(n, 4))
    vq, vs, vo = (rng.normal(size=a.shape).astype(np.float32) for a in (q, ls, lo))

    def run(fn):
        ts = [dev(a).requires_grad_(True) for a in (q, ls, lo)]
        outs = fn(*ts)
        torch.autograd.backward(outs, [dev(vq), dev(vs), dev(vo)])
        return [host(o) for o in outs], [host(t.grad) for t in ts]

    (fq, fs, fo), (gq, gs, go) = run(g.gaussian_activations)
    (eq, es, eo), (hq, hs, ho) = run(R.gaussian_activations_unfused)
    assert_close_rel(fq, eq, 1e-6, "quats")
    assert_close_rel(fs, es, 1e-6, "scales")
    assert_close_rel(fo, eo, 1e-6, "opacities")
    assert_close_rel(gq, hq, 1e-5, "v_quats")
    assert_close_rel(gs, hs, 1e-5, "v_log_scales")
    assert_close_rel(go, ho, 1e-5, "v_opacity_logits")
    # closed forms: unit quaternions where |q| >= 1e-8; gradient orthogonal to q there
    norms = np.linalg.norm(q[0].astype(np.float64), axis=-1)
    ok = norms >= 1e-8
    np.testing.assert_allclose(np.linalg.norm(fq[0][ok], axis=-1), 1.0, rtol=1e-6)
    dots = np.abs(np.sum(gq[0][ok].astype(np.float64) * q[0][ok], axis=-1))
    assert np.all(dots <= 1e-5 * np.linalg.norm(gq[0][ok], axis=-1) * norms[ok] + 1e-30)


def test_activations_partial_grads():
    import torch

    g = gsplat()
    rng = np.random.default_rng(3)
    q, ls, lo = _inputs(rng, 500)
    tq, tl, to = dev(q), dev(ls).requires_grad_(True), dev(lo)
    qn, s, o = g.gaussian_activations(tq, tl, to)
    (s.sum() * 2).backward()
    np.testing.assert_allclose(host(tl.grad), 2 * np.exp(ls), rtol=1e-6)
    assert tq.grad is None and to.grad is None
    del torch


@pytest.mark.parametrize("shape", [(1, 840, 1297, 3), (2, 33, 17, 3), (5,)])
def test_l1_vs_torch(shape):
    import torch

    g = gsplat()
    from gsplat_core import render as R

    rng = np.random.default_rng(sum(shape))
    a = rng.random(shape).astype(np.float32)
    b = rng.random(shape).astype(np.float32)
    b.reshape(-1)[:3] = a.reshape(-1)[:3]  # sign(0) = 0

    def run(fn):
        ta, tb = dev(a).requires_grad_(True), dev(b).requires_grad_(True)
        loss = fn(ta, tb)
        (loss * 3.0).backward()
        return host(loss), host(ta.grad), host(tb.grad)

    la, ga, gb = run(g.l1_loss)
    le, ha, hb = run(R.l1_loss_unfused)
    assert_close_rel(np.array([la]), np.array([le]), 1e-5, "loss")
    # g / n rounds once here; the framework may scale in another order (1 ulp)
    np.testing.assert_allclose(ga, ha, rtol=1e-6, atol=0)
    np.testing.assert_allclose(gb, hb, rtol=1e-6, atol=0)
    np.testing.assert_array_equal(np.sign(ga), np.sign(a - b))
    del torch
