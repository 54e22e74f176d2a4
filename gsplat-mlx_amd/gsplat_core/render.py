"""Caller-side composition of the operator chain (torch), mirroring the
reference training call sites:

  camera_center_from_viewmat  scanner_points_training_utils.py:1005-1008
  sh_colors_for_camera        scanner_points_training_utils.py:1011-1034
  render_sh_model             scanner_points_training_utils.py:1050-1121
  render_rgb_model            train_image_fitting_3dgs_mlx.py:165-237 /
                              render_random_3dgs_png.py:114-168
  l1_loss                     image L1 term of image_loss_components,
                              scanner_points_training_utils.py:1147-1160
  ssim_index                  scanner_points_training_utils.py:1131-1144
  image_loss_components       scanner_points_training_utils.py:1147-1172
  image_training_loss         scanner_points_training_utils.py:1175-1182

Every operator call goes through the differentiable wrappers in
``gsplat_core.autograd`` (HIP kernels). The parameter activations (quaternion
normalisation, exp of the log-scales, sigmoid of the opacity logits) run
inside the projection kernels (activated_projection); the SH colour glue and
the image losses (L1, and L1 + DSSIM from one pass) also run as fused HIP
kernels. The compositions they replace are
kept beside them (``*_unfused``, gaussian_activations + the projection) as the
reference for tests.
"""
from __future__ import annotations

import torch

from . import _gsplat_core as _C
from .autograd import (activated_projection, activated_projection_packed, image_loss, l1_loss as _l1_loss,
                       packed_rows, projection_ewa_3dgs_fused, rasterize_to_pixels_3dgs, render_rgb,
                       render_rgb_l1_value_and_grad,
                       sh_camera_colors, sh_camera_colors_packed, spherical_harmonics)


def normalize_quats(quats: torch.Tensor) -> torch.Tensor:
    """scanner_points_training_utils.py:39-41"""
    norm = torch.sqrt(torch.sum(quats * quats, dim=-1, keepdim=True))
    return quats / torch.clamp(norm, min=1.0e-8)


def camera_center_from_viewmat(viewmats: torch.Tensor) -> torch.Tensor:
    rot = viewmats[:, :, :3, :3]
    trans = viewmats[:, :, :3, 3]
    return -torch.matmul(rot.transpose(-1, -2), trans[..., None])[..., 0]


def sh_colors_for_camera(means, features_dc, features_rest, viewmats, sh_degree, radii=None):
    """scanner_points_training_utils.py:1011-1034. The normalisation, the
    coefficient concat / broadcast and the clip run inside the fused SH
    kernels when the camera centres need no gradient; otherwise the
    reference's composition of elementwise ops and the SH operator runs.
    radii (the projection's, fused path only): the rows no camera sees, which
    no render reads, are skipped in the forward (colour 0)."""
    if not viewmats.requires_grad:
        return sh_camera_colors(sh_degree, means, viewmats.contiguous(), features_dc, features_rest, radii)
    return sh_colors_for_camera_unfused(means, features_dc, features_rest, viewmats, sh_degree)


def sh_colors_for_camera_unfused(means, features_dc, features_rest, viewmats, sh_degree):
    active = (sh_degree + 1) ** 2
    dirs = means[:, None, :, :] - camera_center_from_viewmat(viewmats)[:, :, None, :]
    dirs = dirs / torch.clamp(torch.sqrt(torch.sum(dirs * dirs, dim=-1, keepdim=True)), min=1.0e-8)
    coeffs = torch.cat([features_dc[:, :, None, :], features_rest[:, :, : active - 1, :]], dim=2)
    coeffs = coeffs[:, None].expand(*dirs.shape[:-1], active, 3)
    colors = spherical_harmonics(sh_degree, dirs.reshape(-1, 3), coeffs.reshape(-1, active, 3))
    return torch.clamp((colors + 0.5).reshape(*dirs.shape[:-1], 3), 0.0, 1.0)


_BACKGROUNDS: dict = {}


def background_tensor(background, device) -> torch.Tensor:
    """[1, 3] background colour on `device`, made once per (colour, device):
    building it from a Python list each call is a host-to-device copy that
    waits for the stream to drain."""
    key = (tuple(float(c) for c in background), str(device))
    bg = _BACKGROUNDS.get(key)
    if bg is None:
        bg = torch.tensor([list(key[0])], dtype=torch.float32, device=device)
        _BACKGROUNDS[key] = bg
    return bg


def tile_grid(width: int, height: int, tile_size: int):
    return (width + tile_size - 1) // tile_size, (height + tile_size - 1) // tile_size


def _intersect_begin(proj, width, height, tile_size, images=1, opacities=None):
    """Sorted tile intersection up to its count read-back (finish with
    _intersect_end); with the rasterizer's opacities, the ellipse (AccuTile)
    tiles, which render the same images from fewer entries. Work queued in
    between runs on the GPU while the host waits for the count."""
    tw, th = tile_grid(width, height, tile_size)
    inputs = {"means2d": proj["means2d"].detach(), "radii": proj["radii"], "depths": proj["depths"].detach()}
    if opacities is not None:
        inputs["conics"] = proj["conics"].detach()
        inputs["opacities"] = opacities.detach()
    return _C.intersect_tile_offsets_begin(inputs, images, tile_size, tw, th)


def _intersect_end(pending):
    isect = _C.intersect_tile_offsets_end(pending)
    return isect, isect["tile_offsets"]


def _per_image(opacities, background, n_images, device):
    """Opacities [1, C, N] and backgrounds [C, 3] for C images of the same
    Gaussians (the expand's backward sums the opacity gradient over cameras)."""
    bg = background_tensor(background, device)
    if n_images == 1:
        return opacities[:, None], bg
    return opacities[:, None].expand(-1, n_images, -1).contiguous(), bg.expand(n_images, -1)


def _render_sh_packed(means, quats, log_scales, features_dc, features_rest, opacity_logits, viewmats, Ks, width,
                      height, tile_size, sh_degree, viewspace_points, background, far_plane, accutile):
    """render_sh_model over the packed layout: only the visible (camera,
    Gaussian) pairs are projected, intersected and rasterized."""
    C = viewmats.shape[1]
    fused_colors = not viewmats.requires_grad
    if not fused_colors:
        # the reference composition (view-matrix gradients), gathered per row below
        colors_all = sh_colors_for_camera(means, features_dc, features_rest, viewmats, sh_degree)  # [1, C, N, 3]
    # the parameter activations run inside the packed projection's kernels,
    # which also write each row's opacity
    pr = activated_projection_packed(means, quats, log_scales, opacity_logits, viewmats, Ks, width, height,
                                     viewspace_points=viewspace_points, eps2d=0.3, near_plane=0.01,
                                     far_plane=far_plane)
    cid, gid = pr["camera_ids"], pr["gaussian_ids"]
    m2 = pr["means2d"]
    opac = pr["opacities"]
    tw, th = tile_grid(width, height, tile_size)
    inputs = {"means2d": m2.detach(), "radii": pr["radii"], "depths": pr["depths"].detach(), "image_ids": cid,
              "gaussian_ids": gid}
    if accutile:
        inputs["conics"] = pr["conics"].detach()
        inputs["opacities"] = opac.detach()
    # sorted lists and tile offsets (the tile-bucket path writes the offsets
    # itself) in two calls around the count read-back: the rows' colours are
    # queued in between, so the GPU evaluates them while the host waits for
    # the count (written and, in the backward, read at the packed rows
    # through the projection's rank structure)
    pending = _C.intersect_tile_offsets_begin(inputs, C, tile_size, tw, th)
    if fused_colors:
        colors = sh_camera_colors_packed(sh_degree, means, viewmats.contiguous(), features_dc, features_rest,
                                         pr["rank"], cid.numel())
    else:
        colors = packed_rows(colors_all, pr["batch_ids"], cid, gid, pr["rank"])
    isect = _C.intersect_tile_offsets_end(pending)
    offsets = isect["tile_offsets"]
    bg = background_tensor(background, means.device)
    bg = bg if C == 1 else bg.expand(C, -1)
    render = rasterize_to_pixels_3dgs(m2, pr["conics"], colors, opac, offsets, isect["flatten_ids"], width, height,
                                      tile_size, backgrounds=bg)
    return {**render, "radii": pr["radii"], "camera_ids": cid, "gaussian_ids": gid,
            "tiles_per_gauss": isect["tiles_per_gauss"], "flatten_ids": isect["flatten_ids"],
            "isect_ids": isect["isect_ids"], "tile_offsets": offsets}


def render_sh_model(means, quats, log_scales, features_dc, features_rest, opacity_logits, viewmats, Ks, width,
                    height, tile_size, sh_degree, viewspace_points=None, background=(0.025, 0.025, 0.025),
                    far_plane=100.0, accutile=False, packed=False):
    """C cameras (viewmats [1, C, 4, 4]) rendered as C images of the same
    Gaussians; returns the render dict ([C, H, W, ...] images) plus radii,
    tiles_per_gauss and flatten_ids, like the reference. accutile: ellipse
    tile lists (same images, fewer intersections). packed: the packed layout
    (same images; per-pair arrays hold only the visible pairs)."""
    if packed:
        return _render_sh_packed(means, quats, log_scales, features_dc, features_rest, opacity_logits, viewmats, Ks,
                                 width, height, tile_size, sh_degree, viewspace_points, background, far_plane,
                                 accutile)
    C = viewmats.shape[1]
    # the parameter activations run inside the projection kernels
    proj = activated_projection(means, quats, log_scales, opacity_logits, viewmats, Ks, width, height,
                                viewspace_points=viewspace_points, eps2d=0.3, near_plane=0.01,
                                far_plane=far_plane, radius_clip=0.0, calc_compensations=False, camera_model=0)
    opac_img, bg = _per_image(proj["opacities"], background, C, means.device)
    pending = _intersect_begin(proj, width, height, tile_size, C, opac_img if accutile else None)
    # queued behind the intersection's count read-back: the GPU evaluates the
    # SH colours while the host waits for the count
    # rows no camera sees are in no tile list: with one camera their colours
    # are skipped (a prefetched 8-byte test per Gaussian; with C cameras the
    # test reads C radii per Gaussian and costs more than it saves)
    colors = sh_colors_for_camera(means, features_dc, features_rest, viewmats, sh_degree,
                                  radii=proj["radii"] if C == 1 else None)
    isect, offsets = _intersect_end(pending)
    render = rasterize_to_pixels_3dgs(proj["means2d"], proj["conics"], colors, opac_img,
                                      offsets, isect["flatten_ids"], width, height, tile_size, backgrounds=bg)
    return {**render, "radii": proj["radii"], "tiles_per_gauss": isect["tiles_per_gauss"],
            "flatten_ids": isect["flatten_ids"], "isect_ids": isect["isect_ids"], "tile_offsets": offsets}


def render_rgb_model(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, width, height, tile_size,
                     background=(0.0, 0.0, 0.0), opacities_in_projection=False, far_plane=1e10, accutile=False,
                     fused=True):
    """RGB colours per Gaussian; C cameras (viewmats [1, C, 4, 4]) as C images.
    accutile: ellipse tile lists (same images, fewer intersections). fused:
    the whole step as one C++ call per direction (the same operators; fused
    False composes them here, one autograd node each)."""
    C = viewmats.shape[1]
    if fused:
        bg = background_tensor(background, means.device)
        bg = bg if C == 1 else bg.expand(C, -1)
        return render_rgb(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, bg, width, height,
                          tile_size, far_plane=far_plane, opacities_in_projection=opacities_in_projection,
                          accutile=accutile)
    proj = activated_projection(means, quats, log_scales, opacity_logits, viewmats, Ks, width, height, eps2d=0.3,
                                near_plane=0.01, far_plane=far_plane,
                                opacities_in_projection=opacities_in_projection)
    opac_img, bg = _per_image(proj["opacities"], background, C, means.device)
    isect, offsets = _intersect_end(_intersect_begin(proj, width, height, tile_size, C,
                                                     opac_img if accutile else None))
    colors_img = colors[:, None] if C == 1 else colors[:, None].expand(-1, C, -1, -1).contiguous()
    render = rasterize_to_pixels_3dgs(proj["means2d"], proj["conics"], colors_img, opac_img, offsets,
                                      isect["flatten_ids"], width, height, tile_size, backgrounds=bg)
    return {**render, "radii": proj["radii"], "tiles_per_gauss": isect["tiles_per_gauss"],
            "flatten_ids": isect["flatten_ids"], "isect_ids": isect["isect_ids"], "tile_offsets": offsets}


def render_rgb_model_l1_value_and_grad(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, target, width,
                                       height, tile_size, background=(0.0, 0.0, 0.0), opacities_in_projection=False,
                                       far_plane=1e10, accutile=False):
    """render_rgb_model's step with the L1 image loss as one value_and_grad
    call (train_image_fitting_3dgs_mlx.py:165-237): returns (loss, the render
    dict, {"v_means", "v_quats", "v_log_scales", "v_colors",
    "v_opacity_logits"}); the same kernels as render_rgb_model followed by
    l1_loss and backward, with no autograd graph in between."""
    C = viewmats.shape[1]
    bg = background_tensor(background, means.device)
    bg = bg if C == 1 else bg.expand(C, -1)
    return render_rgb_l1_value_and_grad(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, target, bg,
                                        width, height, tile_size, far_plane=far_plane,
                                        opacities_in_projection=opacities_in_projection, accutile=accutile)


def l1_loss(image: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean(|image - target|) (fused HIP kernels)."""
    return _l1_loss(image, target)


def ssim_index(image: torch.Tensor, target: torch.Tensor, window_size: int) -> torch.Tensor:
    """Mean SSIM of window_size x window_size box statistics (zero padding,
    c1 = 0.01^2, c2 = 0.03^2) for image and target [B, H, W, C]."""
    return image_loss(image, target, window_size)[1]


def image_loss_components(image: torch.Tensor, target: torch.Tensor, loss_mode: str, ssim_lambda: float,
                          ssim_window_size: int) -> dict:
    """scanner_points_training_utils.py:1147-1172: {"loss", "l1", "ssim",
    "dssim"}; "l1_dssim" mixes (1 - ssim_lambda) L1 + ssim_lambda (1 - ssim) / 2,
    with both terms from one pass of the fused HIP kernels."""
    if loss_mode == "l1":
        l1 = _l1_loss(image, target)
        return {"loss": l1, "l1": l1, "ssim": torch.ones((), dtype=image.dtype, device=image.device),
                "dssim": torch.zeros((), dtype=image.dtype, device=image.device)}
    if loss_mode != "l1_dssim":
        raise ValueError(f"Unsupported loss mode: {loss_mode}")
    l1, ssim = image_loss(image, target, ssim_window_size)
    dssim = (1.0 - ssim) * 0.5
    loss = (1.0 - ssim_lambda) * l1 + ssim_lambda * dssim
    return {"loss": loss, "l1": l1, "ssim": ssim, "dssim": dssim}


def image_training_loss(image: torch.Tensor, target: torch.Tensor, loss_mode: str, ssim_lambda: float,
                        ssim_window_size: int) -> torch.Tensor:
    """scanner_points_training_utils.py:1175-1182."""
    return image_loss_components(image, target, loss_mode, ssim_lambda, ssim_window_size)["loss"]


def l1_loss_unfused(image: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    return torch.mean(torch.abs(image - target))


def gaussian_activations_unfused(quats, log_scales, opacity_logits):
    return normalize_quats(quats), torch.exp(log_scales), torch.sigmoid(opacity_logits)
