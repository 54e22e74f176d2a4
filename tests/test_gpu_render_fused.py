"""The RGB render step as one C++ call per direction (render_rgb_model's
default, the render_rgb_forward / render_rgb_backward binding) against the
same step composed in Python one operator at a time (fused=False): the same
kernels on the same inputs, so images, last ids and intersections must agree
bit for bit, and every parameter gradient up to the order of the
rasterizer's float atomics (which differs between any two runs): 1e-4
relative, at most one element per million up to 1e-2 -- one camera and
three, AABB and ellipse tile lists, opacities in the projection or not, with
and without a loss on the alphas. The composed path itself is checked against the oracle
in test_gpu_training_step.py."""
import numpy as np
import pytest

from _helpers import assert_close_rel_summation, dev, host

pytestmark = pytest.mark.gpu


def _run(sc, C, fused, accutile, alphas_loss):
    import torch

    from gsplat_core import render as R

    p = {k: dev(getattr(sc, k)).requires_grad_(True) for k in ("means", "quats", "log_scales", "colors",
                                                                 "opacity_logits")}
    vm = dev(sc.viewmats[:, :C]).requires_grad_(True)
    out = R.render_rgb_model(p["means"], p["quats"], p["log_scales"], p["colors"], p["opacity_logits"], vm,
                             dev(sc.Ks[:, :C]), sc.width, sc.height, sc.tile_size, background=sc.background,
                             opacities_in_projection=sc.opacities_in_projection, far_plane=sc.far_plane,
                             accutile=accutile, fused=fused)
    g = torch.Generator(device="cuda").manual_seed(3)
    w = torch.rand(out["render_colors"].shape, device="cuda", generator=g)
    loss = (out["render_colors"] * w).sum()
    if alphas_loss:
        loss = loss + 0.5 * out["render_alphas"].sum()
    loss.backward()
    torch.cuda.synchronize()
    res = {k: host(out[k]) for k in ("render_colors", "render_alphas", "last_ids", "radii", "tiles_per_gauss",
                                     "flatten_ids", "isect_ids", "tile_offsets")}
    res.update({"v_" + k: host(v.grad) for k, v in p.items()})
    res["v_viewmats"] = host(vm.grad)
    return res


@pytest.mark.parametrize("name,C,accutile,alphas_loss", [("random_forward", 1, False, False),
                                                         ("image_fit", 1, False, True),
                                                         ("image_fit", 1, True, False),
                                                         ("image_fit", 3, False, True),
                                                         ("image_fit", 3, True, True)])
def test_fused_equals_composed(name, C, accutile, alphas_loss):
    from gsplat_core.scenes import make_scene

    kw = {"n": 20000, "width": 200, "height": 152} if name == "image_fit" else {}
    sc = make_scene(name, seed=11, **kw)
    if C > sc.viewmats.shape[1]:  # more cameras: small rotations of the first
        from scipy.spatial.transform import Rotation

        v0 = sc.viewmats[:, :1]
        extra = []
        for k in range(1, C):
            v = v0.copy()
            v[0, 0, :3, :3] = Rotation.from_euler("y", 0.05 * k).as_matrix().astype(np.float32) @ v[0, 0, :3, :3]
            extra.append(v)
        sc.viewmats = np.concatenate([sc.viewmats[:, :1]] + extra, axis=1).astype(np.float32)
        sc.Ks = np.repeat(sc.Ks[:, :1], C, axis=1)
    print(f"fused render {name} C={C} accutile={accutile} alphas_loss={alphas_loss}", flush=True)
    a = _run(sc, C, True, accutile, alphas_loss)
    b = _run(sc, C, False, accutile, alphas_loss)
    assert a["isect_ids"].size > 0
    for k in a:
        if k.startswith("v_"):
            assert np.abs(b[k]).max() > 0, k
            assert_close_rel_summation(a[k], b[k], 1e-4, k)
        else:
            np.testing.assert_array_equal(a[k], b[k], err_msg=k)


# The step's loss and gradients in one call (render_rgb_model_l1_value_and_grad,
# the reference trainer's value_and_grad) against the same step through
# autograd (render_rgb_model, l1_loss, backward): the same kernels, so the
# loss, images and lists agree bit for bit and the gradients up to the order
# of the rasterizer's float atomics.
@pytest.mark.parametrize("C,accutile", [(1, False), (1, True), (3, False)])
def test_l1_value_and_grad_equals_autograd(C, accutile):
    import torch

    from gsplat_core import render as R
    from gsplat_core.scenes import make_scene

    sc = make_scene("image_fit", seed=5, n=20000, width=200, height=152)
    if C > 1:
        from scipy.spatial.transform import Rotation

        v0 = sc.viewmats[:, :1]
        extra = []
        for k in range(1, C):
            v = v0.copy()
            v[0, 0, :3, :3] = Rotation.from_euler("x", 0.04 * k).as_matrix().astype(np.float32) @ v[0, 0, :3, :3]
            extra.append(v)
        sc.viewmats = np.concatenate([v0] + extra, axis=1).astype(np.float32)
        sc.Ks = np.repeat(sc.Ks[:, :1], C, axis=1)
    rng = np.random.default_rng(C)
    target = dev(rng.uniform(0, 1, (C, sc.height, sc.width, 3)).astype(np.float32))
    names = ("means", "quats", "log_scales", "colors", "opacity_logits")
    p = {k: dev(getattr(sc, k)).requires_grad_(True) for k in names}
    args = (p["means"], p["quats"], p["log_scales"], p["colors"], p["opacity_logits"], dev(sc.viewmats[:, :C]),
            dev(sc.Ks[:, :C]))
    kw = dict(background=sc.background, opacities_in_projection=sc.opacities_in_projection,
              far_plane=sc.far_plane, accutile=accutile)
    print(f"l1 value_and_grad C={C} accutile={accutile}", flush=True)
    out = R.render_rgb_model(*args, sc.width, sc.height, sc.tile_size, **kw)
    loss = R.l1_loss(out["render_colors"], target.reshape(out["render_colors"].shape))
    loss.backward()
    loss2, render2, grads2 = R.render_rgb_model_l1_value_and_grad(*args, target, sc.width, sc.height, sc.tile_size,
                                                                   **kw)
    torch.cuda.synchronize()
    assert render2["isect_ids"].numel() > 0
    np.testing.assert_array_equal(host(loss2), host(loss))
    for k in render2:
        np.testing.assert_array_equal(host(render2[k]), host(out[k]), err_msg=k)
    for k in names:
        e = host(p[k].grad)
        assert np.abs(e).max() > 0, k
        assert_close_rel_summation(host(grads2["v_" + k]), e, 1e-4, k)
