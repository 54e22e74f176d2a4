"""GPU parity of the fused training-step glue against the framework (torch
fp32) compositions it replaces: the parameter activations
(scanner_points_training_utils.py:39-41, 306-316) and the image L1 term
(:1147-1160). Forward within 1e-6 relative (a different but equally exact
order of the same float operations; the L1 mean within 1e-5), gradients
within 1e-5 relative (L1: 1e-6, and the exact signs), plus
closed-form properties (unit quaternions, gradient orthogonal to q)."""
import numpy as np
import pytest

from _helpers import FLOOR_ORDERED, assert_close_rel, dev, gsplat, host

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
    assert_close_rel(fq, eq, 1e-6, "quats", floor_rel=FLOOR_ORDERED)
    assert_close_rel(fs, es, 1e-6, "scales", floor_rel=FLOOR_ORDERED)
    assert_close_rel(fo, eo, 1e-6, "opacities", floor_rel=FLOOR_ORDERED)
    assert_close_rel(gq, hq, 1e-5, "v_quats", floor_rel=FLOOR_ORDERED)
    assert_close_rel(gs, hs, 1e-5, "v_log_scales", floor_rel=FLOOR_ORDERED)
    assert_close_rel(go, ho, 1e-5, "v_opacity_logits", floor_rel=FLOOR_ORDERED)
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


# Whole 4096-float tiles of the partial sums with and without a ragged last
# one, more tiles than partial blocks (35M values: blocks walk several
# tiles), a tiny input, and operands 4 bytes off 16-byte alignment (the
# 4-byte paths of both kernels).
@pytest.mark.parametrize("shape,offset", [((1, 840, 1297, 3), 0), ((2, 33, 17, 3), 0), ((5,), 0),
                                          ((3, 1001, 17), 0), ((35_000_001,), 0), ((3, 1001, 17), 1)])
def test_l1_vs_torch(shape, offset):
    import torch

    g = gsplat()
    from gsplat_core import render as R

    rng = np.random.default_rng(sum(shape))
    a = rng.random(shape).astype(np.float32)
    b = rng.random(shape).astype(np.float32)
    b.reshape(-1)[:3] = a.reshape(-1)[:3]  # sign(0) = 0

    def run(fn):
        ta, tb = dev(a).requires_grad_(True), dev(b).requires_grad_(True)
        if offset:  # views one float into a larger buffer: 4-byte aligned only
            pa, pb = torch.zeros(a.size + offset, device="cuda"), torch.zeros(b.size + offset, device="cuda")
            pa[offset:] = ta.detach().reshape(-1)
            pb[offset:] = tb.detach().reshape(-1)
            ta = pa[offset:].reshape(shape).requires_grad_(True)
            tb = pb[offset:].reshape(shape).requires_grad_(True)
            assert ta.data_ptr() % 16 != 0
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


def _proj_scene(rng, B, C, N):
    from scipy.spatial.transform import Rotation

    means = (rng.normal(size=(B, N, 3)) * [0.6, 0.5, 0.5] + [0, 0, 4]).astype(np.float32)
    q = rng.normal(size=(B, N, 4)).astype(np.float32)
    ls = rng.uniform(-4, -1.5, (B, N, 3)).astype(np.float32)
    lo = rng.normal(0, 2, size=(B, N)).astype(np.float32)
    view = np.zeros((B, C, 4, 4), np.float32)
    view[..., 3, 3] = 1
    view[..., :3, :3] = Rotation.from_euler("xyz", rng.normal(scale=0.1, size=(B * C, 3))).as_matrix().reshape(
        B, C, 3, 3)
    view[..., :3, 3] = rng.normal(scale=0.2, size=(B, C, 3))
    Ks = np.zeros((B, C, 3, 3), np.float32)
    Ks[..., 0, 0], Ks[..., 1, 1], Ks[..., 0, 2], Ks[..., 1, 2], Ks[..., 2, 2] = 400, 380, 160, 120, 1
    return means, q, ls, lo, view, Ks


@pytest.mark.parametrize("B,C,in_proj,comp", [(1, 1, False, False), (1, 3, True, True), (2, 2, False, True)])
def test_activated_projection_vs_composition(B, C, in_proj, comp):
    """activated_projection equals gaussian_activations followed by
    projection_ewa_3dgs_fused: forward bit for bit; every gradient (raw
    parameters, view matrices, the viewspace proxy) within the chain's 1e-3
    gradient tolerance (the projection backward computes gradients with FMA
    contraction and fast division, and the fused path also applies the
    activation VJPs that way; typical differences are ~1e-6)."""
    import torch

    g = gsplat()
    rng = np.random.default_rng(B * 100 + C * 10 + in_proj)
    N = 3001
    means, q, ls, lo, view, Ks = _proj_scene(rng, B, C, N)
    kw = dict(eps2d=0.3, near_plane=0.01, far_plane=100.0, calc_compensations=comp)

    def run(fused):
        ts = [dev(a).requires_grad_(True) for a in (means, q, ls, lo, view)]
        vsp = torch.zeros((B, C, N, 2), device="cuda", requires_grad=True)
        K = dev(Ks)
        if fused:
            out = g.activated_projection(ts[0], ts[1], ts[2], ts[3], ts[4], K, 320, 240, viewspace_points=vsp,
                                         opacities_in_projection=in_proj, **kw)
            opac = out["opacities"]
        else:
            qn, sc, opac = g.gaussian_activations(ts[1], ts[2], ts[3])
            out = g.projection_ewa_3dgs_fused(ts[0], ts[4], K, 320, 240, quats=qn, scales=sc,
                                              opacities=opac if in_proj else None, viewspace_points=vsp, **kw)
        keys = ["means2d", "depths", "conics"] + (["compensations"] if comp else [])
        gen = torch.Generator(device="cpu").manual_seed(5)
        loss = sum((out[k] * torch.randn(out[k].shape, generator=gen).cuda()).sum() for k in keys)
        loss = loss + (opac * torch.randn(opac.shape, generator=gen).cuda()).sum()
        loss.backward()
        vals = {k: host(out[k]) for k in keys + ["radii"]}
        vals["opacities"] = host(opac)
        return vals, [host(t.grad) for t in ts] + [host(vsp.grad)]

    fv, fg = run(True)
    ev, eg = run(False)
    for k in ev:
        np.testing.assert_array_equal(fv[k], ev[k], err_msg=k)
    assert (fv["radii"] > 0).any(axis=-1).sum() > 100
    for name, a, e in zip(["means", "quats", "log_scales", "opacity_logits", "viewmats", "viewspace"], fg, eg):
        assert_close_rel(a, e, 1e-3, name)


def test_activated_projection_c_abi_and_errors():
    """The activated entry points through the C ABI: NULL logits skip the
    opacities; covars and opacities without logits are rejected."""
    import ctypes

    import torch

    import gsplat_core

    lib = ctypes.CDLL(gsplat_core._gsplat_core.__file__.rsplit("/", 1)[0] + "/libgsplat_hip.so")
    rng = np.random.default_rng(3)
    B, C, N = 1, 1, 500
    means, q, ls, lo, view, Ks = _proj_scene(rng, B, C, N)

    class Params(ctypes.Structure):
        _fields_ = [("image_width", ctypes.c_int32), ("image_height", ctypes.c_int32), ("eps2d", ctypes.c_float),
                    ("near_plane", ctypes.c_float), ("far_plane", ctypes.c_float), ("radius_clip", ctypes.c_float),
                    ("calc_compensations", ctypes.c_int32), ("camera_model", ctypes.c_int32),
                    ("use_covars", ctypes.c_int32), ("use_opacities", ctypes.c_int32)]

    p = Params(320, 240, 0.3, 0.01, 100.0, 0.0, 0, 0, 0, 0)
    tm, tq, tl, to, tv, tk = (dev(a) for a in (means, q, ls, lo, view, Ks))
    radii = torch.empty((B, C, N, 2), dtype=torch.int32, device="cuda")
    m2 = torch.empty((B, C, N, 2), device="cuda")
    dep = torch.empty((B, C, N), device="cuda")
    con = torch.empty((B, C, N, 3), device="cuda")
    opac = torch.full((B, N), -1.0, device="cuda")
    f = lib.gsplat_hip_activated_projection_fwd
    f.restype = ctypes.c_int
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    f.argtypes = [vp] * 6 + [i64] * 3 + [ctypes.POINTER(Params)] + [vp] * 7
    st = torch.cuda.current_stream().cuda_stream
    args = [tm.data_ptr(), tq.data_ptr(), tl.data_ptr(), None, tv.data_ptr(), tk.data_ptr(), B, C, N,
            ctypes.byref(p), radii.data_ptr(), m2.data_ptr(), dep.data_ptr(), con.data_ptr(), None,
            opac.data_ptr(), st]
    assert f(*args) != 0  # opacities requested without logits
    args[3] = to.data_ptr()
    assert f(*args) == 0
    torch.cuda.synchronize()
    assert_close_rel(host(opac), 1.0 / (1.0 + np.exp(-lo.astype(np.float64))), 1e-6, "opacities", floor_rel=FLOOR_ORDERED)
    p.use_covars = 1
    assert f(*args) != 0  # covars are not an activated input


def test_selective_adam_vs_torch_adam():
    """selective_adam_update (upstream gsplat's fused selective Adam) against
    torch.optim.Adam, an independent implementation: three steps with every
    row valid, then a masked step that must leave invalid rows untouched."""
    import torch

    g = gsplat()
    rng = np.random.default_rng(0)
    n, D = 100003, 3
    p0 = rng.normal(size=(n, D)).astype(np.float32)
    grads = [rng.normal(size=(n, D)).astype(np.float32) for _ in range(4)]
    ref = torch.nn.Parameter(torch.from_numpy(p0.copy()).cuda())
    opt = torch.optim.Adam([ref], lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    p = torch.from_numpy(p0.copy()).cuda()
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    for step in range(1, 4):
        ref.grad = torch.from_numpy(grads[step - 1]).cuda()
        opt.step()
        g._gsplat_core.selective_adam_update(p, ref.grad, m, v, torch.empty(0, device="cuda"), 1e-3, 0.9, 0.999, 1e-8,
                                            step)
        st = opt.state[ref]
        # torch updates the first moment as a lerp (m + (1 - b1)(g - m)),
        # upstream as b1 m + (1 - b1) g: last-bit differences that grow where
        # g - m cancels, so the bound is relative 2e-5 with an absolute floor
        for got, exp, name in ((p, ref.detach(), "param"), (m, st["exp_avg"], "exp_avg"),
                               (v, st["exp_avg_sq"], "exp_avg_sq")):
            e = host(exp)
            np.testing.assert_allclose(host(got), e, rtol=2e-5, atol=1e-6 * np.abs(e).max(),
                                       err_msg=f"{name} step {step}")
    valid = torch.from_numpy(rng.random(n) < 0.5).cuda()
    before = [host(t).copy() for t in (p, m, v)]
    ref.grad = torch.from_numpy(grads[3]).cuda()
    opt.step()
    g._gsplat_core.selective_adam_update(p, ref.grad, m, v, valid, 1e-3, 0.9, 0.999, 1e-8, 4)
    vm = host(valid)
    for got, old in zip((p, m, v), before):
        np.testing.assert_array_equal(host(got)[~vm], old[~vm])
    e = host(ref.detach())[vm]
    np.testing.assert_allclose(host(p)[vm], e, rtol=2e-5, atol=1e-6 * np.abs(e).max(), err_msg="masked step")
    # step 0: upstream's uncorrected form p -= lr m / (sqrt(v) + eps)
    q = torch.zeros((5, 2), device="cuda")
    gq = torch.ones((5, 2), device="cuda")
    mq, vq = torch.zeros_like(q), torch.zeros_like(q)
    g._gsplat_core.selective_adam_update(q, gq, mq, vq, torch.empty(0, device="cuda"), 0.1, 0.9, 0.999, 1e-8, 0)
    np.testing.assert_allclose(host(q), -0.1 * 0.1 / (np.sqrt(0.001) + 1e-8), rtol=1e-6)
