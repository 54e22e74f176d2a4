"""Differentiable wrappers: one torch.autograd.Function per reference primitive.

Each ``backward`` routes cotangents exactly as the reference ``Primitive::vjp``:
  * quat_scale_to_covar_preci -- gsplat_quat_scale_to_covar.cpp:582-613
  * projection_ewa_3dgs_fused -- gsplat_projection.cpp:1130-1208 (opacities and
    Ks get zero gradients; viewspace_points receives the means2d cotangent as
    the densification proxy; view matrices get a gradient only when they
    require one)
  * spherical_harmonics -- gsplat_spherical_harmonics.cpp:670-705 (v_dirs only
    when dirs require a gradient)
  * rasterize_to_pixels_3dgs -- gsplat_rasterize.cpp:749-795 (absgrad off)
Intersection outputs carry no gradient (the reference callers stop_gradient
them, scanner_points_training_utils.py:1093-1101).

More Functions fuse the training step's elementwise glue into HIP kernels
(no counterpart primitive in the reference; they replace the framework
composition at its call sites):
  * gaussian_activations -- normalize_quats / exp / sigmoid of the model
    parameters (scanner_points_training_utils.py:39-41, 306-316)
  * activated_projection -- those activations inside the projection kernels
  * sh_camera_colors -- the camera-colour SH glue (:1005-1034)
  * l1_loss -- the image L1 term of image_loss_components (:1147-1160)
  * image_loss -- its L1 and SSIM terms in one pass (:1123-1172)
"""
from __future__ import annotations

import torch

from . import _gsplat_core as _C


def _empty(ref: torch.Tensor) -> torch.Tensor:
    return torch.zeros(0, dtype=torch.float32, device=ref.device)


def _nonempty(t):
    return t is not None and t.numel() > 0


class _QuatScaleToCovarPreci(torch.autograd.Function):
    @staticmethod
    def forward(ctx, quats, scales, compute_covar, compute_preci, triu):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        out = _C.quat_scale_to_covar_preci_forward({"quats": quats, "scales": scales}, compute_covar, compute_preci,
                                                   triu)
        ctx.save_for_backward(quats, scales)
        ctx.flags = (compute_covar, compute_preci, triu)
        return out["covars"], out["precis"]

    @staticmethod
    def backward(ctx, v_covars, v_precis):
        quats, scales = ctx.saved_tensors
        compute_covar, compute_preci, triu = ctx.flags
        cot = {}
        if compute_covar:
            cot["v_covars"] = v_covars.contiguous() if v_covars is not None else None
        if compute_preci:
            cot["v_precis"] = v_precis.contiguous() if v_precis is not None else None
        cot = {k: v for k, v in cot.items() if v is not None}
        if not cot:
            return torch.zeros_like(quats), torch.zeros_like(scales), None, None, None
        out = _C.quat_scale_to_covar_preci_backward({"quats": quats, "scales": scales}, cot, triu)
        return out["v_quats"], out["v_scales"], None, None, None


def quat_scale_to_covar_preci(quats, scales, compute_covar=True, compute_preci=True, triu=True):
    return _QuatScaleToCovarPreci.apply(quats, scales, compute_covar, compute_preci, triu)


class _ProjectionEWA3DGSFused(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, covars, quats, scales, opacities, viewmats, Ks, viewspace_points, image_width,
                image_height, eps2d, near_plane, far_plane, radius_clip, calc_compensations, camera_model):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        inputs = {"means": means, "viewmats": viewmats, "Ks": Ks}
        for k, v in (("covars", covars), ("quats", quats), ("scales", scales), ("opacities", opacities),
                     ("viewspace_points", viewspace_points)):
            if _nonempty(v):
                inputs[k] = v
        out = _C.projection_ewa_3dgs_fused_forward(inputs, image_width, image_height, eps2d, near_plane, far_plane,
                                                   radius_clip, calc_compensations, camera_model)
        ctx.save_for_backward(means, covars, quats, scales, viewmats, Ks, out["radii"], out["conics"],
                              out["compensations"])
        ctx.params = (image_width, image_height, eps2d, calc_compensations, camera_model, _nonempty(covars))
        ctx.mark_non_differentiable(out["radii"])
        return out["means2d"], out["depths"], out["conics"], out["compensations"], out["radii"]

    @staticmethod
    def backward(ctx, v_means2d, v_depths, v_conics, v_compensations, _v_radii):
        means, covars, quats, scales, viewmats, Ks, radii, conics, comps = ctx.saved_tensors
        W, H, eps2d, calc_comp, camera_model, use_covars = ctx.params
        if camera_model not in (0, 1, 2):
            raise RuntimeError("GSPlatProjectionEWA3DGSFused vjp: unknown camera model.")
        shape2 = radii.shape
        v_means2d = torch.zeros(shape2, dtype=torch.float32, device=means.device) if v_means2d is None else v_means2d
        v_depths = _empty(means) if v_depths is None else v_depths  # empty = zeros
        v_conics = (torch.zeros(conics.shape, dtype=torch.float32, device=means.device) if v_conics is None
                    else v_conics)
        inputs = {"means": means, "viewmats": viewmats, "Ks": Ks}
        if use_covars:
            inputs["covars"] = covars
        else:
            inputs["quats"] = quats
            inputs["scales"] = scales
        fwd = {"radii": radii, "conics": conics}
        cot = {"v_means2d": v_means2d.contiguous(), "v_conics": v_conics.contiguous()}
        if v_depths.numel():
            cot["v_depths"] = v_depths.contiguous()
        if calc_comp:
            fwd["compensations"] = comps
            cot["v_compensations"] = (torch.zeros_like(comps) if v_compensations is None
                                      else v_compensations.contiguous())
        needs_viewmats = ctx.needs_input_grad[5]
        # The forward's own parameters govern the VJP (gsplat_projection.cpp:1151-1177);
        # near/far/radius_clip only affect culling, already encoded in radii.
        out = _C.projection_ewa_3dgs_fused_backward(inputs, fwd, cot, W, H, eps2d, camera_model, needs_viewmats)
        g_covars = out["v_covars"] if use_covars else (torch.zeros_like(covars) if covars is not None else None)
        g_quats = None if use_covars else out["v_quats"]
        g_scales = None if use_covars else out["v_scales"]
        g_opac = None
        g_view = out["v_viewmats"] if needs_viewmats else None
        g_vsp = v_means2d if ctx.needs_input_grad[7] else None
        return (out["v_means"], g_covars, g_quats, g_scales, g_opac, g_view, None, g_vsp) + (None,) * 8


def projection_ewa_3dgs_fused(means, viewmats, Ks, image_width, image_height, quats=None, scales=None, covars=None,
                              opacities=None, viewspace_points=None, eps2d=0.3, near_plane=0.01, far_plane=1e10,
                              radius_clip=0.0, calc_compensations=False, camera_model=0):
    """Differentiable projection; returns the reference binding's output dict."""
    e = _empty(means)
    m2, d, c, comp, r = _ProjectionEWA3DGSFused.apply(
        means, covars if covars is not None else e, quats if quats is not None else e,
        scales if scales is not None else e, opacities if opacities is not None else e, viewmats, Ks,
        viewspace_points if viewspace_points is not None else e, image_width, image_height, eps2d, near_plane,
        far_plane, radius_clip, calc_compensations, camera_model)
    return {"radii": r, "means2d": m2, "depths": d, "conics": c, "compensations": comp,
            "viewspace_points": viewspace_points}


class _ProjectionPacked(torch.autograd.Function):
    """projection_ewa_3dgs_packed_forward / _backward (upstream gsplat's
    fully_fused_projection(packed=True)); backward for all three camera models."""

    @staticmethod
    def forward(ctx, means, quats, scales, viewmats, Ks, image_width, image_height, eps2d, near_plane, far_plane,
                radius_clip, calc_compensations, camera_model):
        ctx.set_materialize_grads(False)
        inputs = {"means": means, "quats": quats, "scales": scales, "viewmats": viewmats, "Ks": Ks}
        out = _C.projection_ewa_3dgs_packed_forward(inputs, image_width, image_height, eps2d, near_plane, far_plane,
                                                    radius_clip, calc_compensations, camera_model)
        ctx.save_for_backward(means, quats, scales, viewmats, Ks, out["batch_ids"], out["camera_ids"],
                              out["gaussian_ids"], out["conics"], out["compensations"])
        ctx.params = (image_width, image_height, eps2d, calc_compensations, camera_model)
        for k in ("batch_ids", "camera_ids", "gaussian_ids", "indptr", "radii"):
            ctx.mark_non_differentiable(out[k])
        return (out["batch_ids"], out["camera_ids"], out["gaussian_ids"], out["indptr"], out["radii"],
                out["means2d"], out["depths"], out["conics"], out["compensations"])

    @staticmethod
    def backward(ctx, _b, _c, _g, _i, _r, v_means2d, v_depths, v_conics, v_compensations):
        means, quats, scales, viewmats, Ks, bid, cid, gid, conics, comps = ctx.saved_tensors
        W, H, eps2d, calc_comp, camera_model = ctx.params
        if camera_model not in (0, 1, 2):
            raise RuntimeError("projection_ewa_3dgs_packed vjp: unknown camera model.")
        nnz = cid.shape[0]
        v_means2d = means.new_zeros((nnz, 2)) if v_means2d is None else v_means2d.contiguous()
        v_conics = means.new_zeros((nnz, 3)) if v_conics is None else v_conics.contiguous()
        inputs = {"means": means, "quats": quats, "scales": scales, "viewmats": viewmats, "Ks": Ks}
        fwd = {"batch_ids": bid, "camera_ids": cid, "gaussian_ids": gid, "conics": conics}
        cot = {"v_means2d": v_means2d, "v_conics": v_conics}
        if v_depths is not None:
            cot["v_depths"] = v_depths.contiguous()
        if calc_comp:
            fwd["compensations"] = comps
            cot["v_compensations"] = torch.zeros_like(comps) if v_compensations is None else v_compensations.contiguous()
        needs_viewmats = ctx.needs_input_grad[3]
        out = _C.projection_ewa_3dgs_packed_backward(inputs, fwd, cot, W, H, eps2d, camera_model, needs_viewmats)
        return (out["v_means"], out["v_quats"], out["v_scales"], out["v_viewmats"] if needs_viewmats else None,
                None) + (None,) * 8


def projection_packed(means, quats, scales, viewmats, Ks, image_width, image_height, eps2d=0.3, near_plane=0.01,
                      far_plane=1e10, radius_clip=0.0, calc_compensations=False, camera_model=0):
    """Packed projection: a dict of the visible pairs' rows (batch_ids,
    camera_ids, gaussian_ids, indptr, radii, means2d, depths, conics,
    compensations), differentiable w.r.t. means, quats, scales, viewmats."""
    keys = ("batch_ids", "camera_ids", "gaussian_ids", "indptr", "radii", "means2d", "depths", "conics",
            "compensations")
    out = _ProjectionPacked.apply(means, quats, scales, viewmats, Ks, image_width, image_height, eps2d, near_plane,
                                  far_plane, radius_clip, calc_compensations, camera_model)
    return dict(zip(keys, out))


class _ActivatedProjectionPacked(torch.autograd.Function):
    """activated_projection_packed_forward / _backward: the packed projection
    with the parameter activations fused in (raw quaternions, log-scales,
    opacity logits), plus each visible pair's sigmoid opacity. The backward
    reads the forward's rank structure (no ids) and takes the opacities'
    cotangent per row."""

    @staticmethod
    def forward(ctx, means, quats, log_scales, opacity_logits, viewmats, Ks, viewspace_points, image_width,
                image_height, eps2d, near_plane, far_plane, radius_clip, calc_compensations, camera_model):
        ctx.set_materialize_grads(False)
        inputs = {"means": means, "quats": quats, "log_scales": log_scales, "viewmats": viewmats, "Ks": Ks}
        if _nonempty(opacity_logits):
            inputs["opacity_logits"] = opacity_logits
        out = _C.activated_projection_packed_forward(inputs, image_width, image_height, eps2d, near_plane,
                                                     far_plane, radius_clip, calc_compensations, camera_model)
        ctx.save_for_backward(means, quats, log_scales, opacity_logits, viewmats, Ks, out["conics"],
                              out["compensations"], out["rank"])
        ctx.params = (image_width, image_height, eps2d, calc_compensations, camera_model)
        ctx.vsp_shape = viewspace_points.shape
        for k in ("batch_ids", "camera_ids", "gaussian_ids", "indptr", "radii", "rank"):
            ctx.mark_non_differentiable(out[k])
        return (out["batch_ids"], out["camera_ids"], out["gaussian_ids"], out["indptr"], out["radii"],
                out["means2d"], out["depths"], out["conics"], out["compensations"], out["opacities"], out["rank"])

    @staticmethod
    def backward(ctx, _b, _c, _g, _i, _r, v_means2d, v_depths, v_conics, v_compensations, v_opacities, _rank):
        means, quats, log_scales, logits, viewmats, Ks, conics, comps, rank = ctx.saved_tensors
        W, H, eps2d, calc_comp, camera_model = ctx.params
        nnz = conics.shape[0]
        v_means2d = means.new_zeros((nnz, 2)) if v_means2d is None else v_means2d.contiguous()
        v_conics = means.new_zeros((nnz, 3)) if v_conics is None else v_conics.contiguous()
        inputs = {"means": means, "quats": quats, "log_scales": log_scales, "viewmats": viewmats, "Ks": Ks}
        if _nonempty(logits):
            inputs["opacity_logits"] = logits
        fwd = {"conics": conics, "rank": rank}
        cot = {"v_means2d": v_means2d, "v_conics": v_conics}
        if v_depths is not None:
            cot["v_depths"] = v_depths.contiguous()
        if calc_comp:
            fwd["compensations"] = comps
            cot["v_compensations"] = torch.zeros_like(comps) if v_compensations is None else v_compensations.contiguous()
        if v_opacities is not None:
            cot["v_opacities"] = v_opacities.contiguous()
        needs_viewmats = ctx.needs_input_grad[4]
        needs_vsp = ctx.needs_input_grad[6]
        out = _C.activated_projection_packed_backward(inputs, fwd, cot, W, H, eps2d, camera_model, needs_viewmats,
                                                      needs_vsp)
        g_logits = out["v_opacity_logits"] if ctx.needs_input_grad[3] else None
        g_vsp = out["v_viewspace"].reshape(ctx.vsp_shape) if needs_vsp else None
        return (out["v_means"], out["v_quats"], out["v_log_scales"], g_logits,
                out["v_viewmats"] if needs_viewmats else None, None, g_vsp) + (None,) * 8


def activated_projection_packed(means, quats, log_scales, opacity_logits, viewmats, Ks, image_width, image_height,
                                viewspace_points=None, eps2d=0.3, near_plane=0.01, far_plane=1e10, radius_clip=0.0,
                                calc_compensations=False, camera_model=0):
    """gaussian_activations followed by projection_packed, in the packed
    projection's kernels: a dict of the visible pairs' rows as
    projection_packed's plus "opacities", each row's sigmoid opacity (the
    rasterizer's), and "rank", the rank structure packed_rows scatters by;
    differentiable w.r.t. means, the raw parameters and viewmats.
    viewspace_points (dense [..., C, N, 2], optional) receives the means2d
    rows' gradient at their (camera, Gaussian) slots, as the dense
    projection's proxy does."""
    keys = ("batch_ids", "camera_ids", "gaussian_ids", "indptr", "radii", "means2d", "depths", "conics",
            "compensations", "opacities", "rank")
    e = _empty(means)
    out = _ActivatedProjectionPacked.apply(means, quats, log_scales,
                                           opacity_logits if opacity_logits is not None else e, viewmats, Ks,
                                           viewspace_points if viewspace_points is not None else e, image_width,
                                           image_height, eps2d, near_plane, far_plane, radius_clip,
                                           calc_compensations, camera_model)
    return dict(zip(keys, out))


class _PackedRows(torch.autograd.Function):
    """Packed rows [nnz, K] of dense [B, C, N, K] values at the rows'
    (batch, camera, Gaussian) ids; the backward scatters the rows' gradient
    to their slots by the activated packed projection's rank (zeros
    elsewhere)."""

    @staticmethod
    def forward(ctx, dense, batch_ids, camera_ids, gaussian_ids, rank):
        ctx.save_for_backward(rank)
        ctx.shape = dense.shape
        ids = {"camera_ids": camera_ids, "gaussian_ids": gaussian_ids}
        if dense.shape[0] > 1:
            ids["batch_ids"] = batch_ids
        return _C.packed_rows_gather(dense.contiguous(), ids)

    @staticmethod
    def backward(ctx, g):
        (rank,) = ctx.saved_tensors
        B, C, N, _K = ctx.shape
        return _C.packed_rows_scatter(g.contiguous(), rank, B, C, N), None, None, None, None


def packed_rows(dense, batch_ids, camera_ids, gaussian_ids, rank):
    """dense [B, C, N, K] at the packed rows' pairs, differentiable w.r.t.
    dense (rank: activated_projection_packed's)."""
    return _PackedRows.apply(dense, batch_ids, camera_ids, gaussian_ids, rank)


class _PackedViewspace(torch.autograd.Function):
    """Identity on the packed means2d whose backward also scatters their
    gradient into a dense viewspace_points [1, C, N, 2] proxy (the packed
    counterpart of the dense projection's proxy gradient)."""

    @staticmethod
    def forward(ctx, means2d, viewspace_points, camera_ids, gaussian_ids):
        ctx.save_for_backward(camera_ids, gaussian_ids)
        ctx.shape = viewspace_points.shape
        return means2d.view_as(means2d)

    @staticmethod
    def backward(ctx, g):
        cid, gid = ctx.saved_tensors
        vsp = None
        if ctx.needs_input_grad[1] and g is not None:
            vsp = g.new_zeros(ctx.shape)
            vsp[0, cid.long(), gid.long()] = g
        return g, vsp, None, None


def packed_viewspace(means2d, viewspace_points, camera_ids, gaussian_ids):
    return _PackedViewspace.apply(means2d, viewspace_points, camera_ids, gaussian_ids)


class _SphericalHarmonics(torch.autograd.Function):
    @staticmethod
    def forward(ctx, degrees_to_use, dirs, coeffs, masks):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        inputs = {"dirs": dirs, "coeffs": coeffs}
        if _nonempty(masks):
            inputs["masks"] = masks
        colors = _C.spherical_harmonics_forward(degrees_to_use, inputs)
        ctx.save_for_backward(dirs, coeffs, masks)
        ctx.degree = degrees_to_use
        return colors

    @staticmethod
    def backward(ctx, v_colors):
        dirs, coeffs, masks = ctx.saved_tensors
        inputs = {"dirs": dirs, "coeffs": coeffs}
        if _nonempty(masks):
            inputs["masks"] = masks
        compute_v_dirs = ctx.needs_input_grad[1]
        out = _C.spherical_harmonics_backward(ctx.degree, inputs, {"v_colors": v_colors.contiguous()},
                                              compute_v_dirs)
        return None, out["v_dirs"] if compute_v_dirs else None, out["v_coeffs"], None


def spherical_harmonics(degrees_to_use, dirs, coeffs, masks=None):
    return _SphericalHarmonics.apply(degrees_to_use, dirs, coeffs, masks if masks is not None else _empty(dirs))


class _ShCameraColors(torch.autograd.Function):
    """colors [B, C, N, 3] = clamp(SH(normalize(means - campos[c])) + 0.5, 0, 1)
    with campos[c] = -R^T t of viewmats[c] and the coefficient concat /
    broadcast of the reference caller (scanner_points_training_utils.py:
    1005-1034) fused into the kernels. The view matrices carry no gradient.
    With radii (the projection's [B, C, N, 2]), the forward skips the rows
    that no camera sees (radii not both positive in any camera: no tile, so
    no render reads them and the rasterizer gives them no colour gradient)
    and writes their colours as 0."""

    @staticmethod
    def forward(ctx, degrees_to_use, means, viewmats, features_dc, features_rest, radii):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        inputs = {"means": means, "viewmats": viewmats, "features_dc": features_dc, "features_rest": features_rest}
        if radii is not None:
            inputs["radii"] = radii
        colors = _C.sh_camera_colors_forward(degrees_to_use, inputs)
        ctx.save_for_backward(means, viewmats, features_dc, features_rest)
        ctx.degree = degrees_to_use
        return colors

    @staticmethod
    def backward(ctx, v_colors):
        means, viewmats, features_dc, features_rest = ctx.saved_tensors
        inputs = {"means": means, "viewmats": viewmats, "features_dc": features_dc, "features_rest": features_rest}
        out = _C.sh_camera_colors_backward(ctx.degree, inputs, {"v_colors": v_colors.contiguous()})
        return None, out["v_means"], None, out["v_features_dc"], out["v_features_rest"], None


def sh_camera_colors(degrees_to_use, means, viewmats, features_dc, features_rest, radii=None):
    """Fused camera colours; viewmats must not require grad. radii (optional,
    the projection's): the forward skips the rows no camera sees (colour 0)."""
    if viewmats.requires_grad:
        raise ValueError("sh_camera_colors: view-matrix gradients are not supported; detach viewmats.")
    return _ShCameraColors.apply(degrees_to_use, means, viewmats, features_dc, features_rest, radii)


class _ShCameraColorsPacked(torch.autograd.Function):
    """The camera colours of the packed layout's visible pairs: [nnz, 3], row
    r the colour of pair r (camera_ids / gaussian_ids of the packed
    projection), as _ShCameraColors computes it. rank is the packed
    projection's "rank" output (its count workspace), nnz its row count. The
    colours are written and their cotangents read at the pairs' packed rows,
    so no dense [B, C, N, 3] colours are formed."""

    @staticmethod
    def forward(ctx, degrees_to_use, means, viewmats, features_dc, features_rest, rank, nnz):
        ctx.set_materialize_grads(False)
        inputs = {"means": means, "viewmats": viewmats, "features_dc": features_dc, "features_rest": features_rest,
                  "rank": rank}
        rows = _C.sh_camera_colors_packed_forward(degrees_to_use, inputs, nnz)
        ctx.save_for_backward(means, viewmats, features_dc, features_rest, rank)
        ctx.degree = degrees_to_use
        return rows

    @staticmethod
    def backward(ctx, v_rows):
        means, viewmats, features_dc, features_rest, rank = ctx.saved_tensors
        inputs = {"means": means, "viewmats": viewmats, "features_dc": features_dc, "features_rest": features_rest,
                  "rank": rank}
        out = _C.sh_camera_colors_packed_backward(ctx.degree, inputs, {"v_colors": v_rows.contiguous()})
        return None, out["v_means"], None, out["v_features_dc"], out["v_features_rest"], None, None


def sh_camera_colors_packed(degrees_to_use, means, viewmats, features_dc, features_rest, rank, nnz):
    """Fused camera colours of the packed pairs ([nnz, 3]); viewmats must not
    require grad."""
    if viewmats.requires_grad:
        raise ValueError("sh_camera_colors_packed: view-matrix gradients are not supported; detach viewmats.")
    return _ShCameraColorsPacked.apply(degrees_to_use, means, viewmats, features_dc, features_rest, rank, int(nnz))


class _RasterizeToPixels3DGS(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, image_width,
                image_height, tile_size):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        inputs = {"means2d": means2d, "conics": conics, "colors": colors, "opacities": opacities,
                  "tile_offsets": tile_offsets, "flatten_ids": flatten_ids}
        if _nonempty(backgrounds):
            inputs["backgrounds"] = backgrounds
        if _nonempty(masks):
            inputs["masks"] = masks
        out = _C.rasterize_to_pixels_3dgs_forward(inputs, image_width, image_height, tile_size)
        ctx.save_for_backward(means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids,
                              out["render_alphas"], out["last_ids"])
        ctx.dims = (image_width, image_height, tile_size)
        ctx.mark_non_differentiable(out["last_ids"])
        return out["render_colors"], out["render_alphas"], out["last_ids"]

    @staticmethod
    def backward(ctx, v_render_colors, v_render_alphas, _v_last_ids):
        (means2d, conics, colors, opacities, backgrounds, masks, tile_offsets, flatten_ids, render_alphas,
         last_ids) = ctx.saved_tensors
        W, H, ts = ctx.dims
        inputs = {"means2d": means2d, "conics": conics, "colors": colors, "opacities": opacities,
                  "tile_offsets": tile_offsets, "flatten_ids": flatten_ids}
        use_bg = _nonempty(backgrounds)
        if use_bg:
            inputs["backgrounds"] = backgrounds
        if _nonempty(masks):
            inputs["masks"] = masks
        if v_render_colors is None:
            v_render_colors = torch.zeros(render_alphas.shape[:-1] + (colors.shape[-1],), dtype=torch.float32,
                                          device=colors.device)
        cot = {"v_render_colors": v_render_colors.contiguous()}
        if v_render_alphas is not None:  # absent = zeros
            cot["v_render_alphas"] = v_render_alphas.contiguous()
        out = _C.rasterize_to_pixels_3dgs_backward(
            inputs, {"render_alphas": render_alphas, "last_ids": last_ids}, cot, W, H, ts, False)
        return (out["v_means2d"], out["v_conics"], out["v_colors"], out["v_opacities"],
                out["v_backgrounds"] if use_bg else None, None, None, None, None, None, None)


def rasterize_to_pixels_3dgs(means2d, conics, colors, opacities, tile_offsets, flatten_ids, image_width, image_height,
                             tile_size, backgrounds=None, masks=None):
    """Differentiable rasterization; returns the reference binding's output dict."""
    e = _empty(means2d)
    rc, ra, li = _RasterizeToPixels3DGS.apply(means2d, conics, colors, opacities,
                                             backgrounds if backgrounds is not None else e,
                                             masks if masks is not None else e, tile_offsets, flatten_ids,
                                             image_width, image_height, tile_size)
    return {"render_colors": rc, "render_alphas": ra, "last_ids": li}


class _GaussianActivations(torch.autograd.Function):
    @staticmethod
    def forward(ctx, quats, log_scales, opacity_logits):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        out = _C.gaussian_activations_forward({"quats": quats, "log_scales": log_scales,
                                               "opacity_logits": opacity_logits})
        ctx.save_for_backward(quats, out["scales"], out["opacities"])
        return out["quats"], out["scales"], out["opacities"]

    @staticmethod
    def backward(ctx, v_quats, v_scales, v_opacities):
        quats, scales, opacities = ctx.saved_tensors
        need_q, need_s, need_o = ctx.needs_input_grad
        inputs = {"quats": quats} if need_q else {}
        fwd = {}
        if need_s:
            fwd["scales"] = scales
        if need_o:
            fwd["opacities"] = opacities
        cot = {}
        for key, v, need in (("v_quats", v_quats, need_q), ("v_scales", v_scales, need_s),
                             ("v_opacities", v_opacities, need_o)):
            if need and v is not None:
                cot[key] = v.contiguous()
        out = _C.gaussian_activations_backward(inputs, fwd, cot)
        return (out["v_quats"] if need_q else None, out["v_log_scales"] if need_s else None,
                out["v_opacity_logits"] if need_o else None)


def gaussian_activations(quats, log_scales, opacity_logits):
    """(quats / max(|quats|, 1e-8), exp(log_scales), sigmoid(opacity_logits))
    in one kernel per direction."""
    return _GaussianActivations.apply(quats, log_scales, opacity_logits)


class _ActivatedProjection(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, quats, log_scales, opacity_logits, viewmats, Ks, viewspace_points, image_width,
                image_height, eps2d, near_plane, far_plane, radius_clip, calc_compensations, camera_model,
                opacities_in_projection):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        inputs = {"means": means, "quats": quats, "log_scales": log_scales, "viewmats": viewmats, "Ks": Ks}
        if _nonempty(opacity_logits):
            inputs["opacity_logits"] = opacity_logits
        out = _C.activated_projection_forward(inputs, image_width, image_height, eps2d, near_plane, far_plane,
                                              radius_clip, calc_compensations, camera_model,
                                              opacities_in_projection)
        ctx.save_for_backward(means, quats, log_scales, opacity_logits, viewmats, Ks, out["radii"], out["conics"],
                              out["compensations"])
        ctx.params = (image_width, image_height, eps2d, calc_compensations, camera_model)
        ctx.mark_non_differentiable(out["radii"])
        return (out["means2d"], out["depths"], out["conics"], out["compensations"], out["radii"],
                out["opacities"])

    @staticmethod
    def backward(ctx, v_means2d, v_depths, v_conics, v_compensations, _v_radii, v_opacities):
        means, quats, log_scales, logits, viewmats, Ks, radii, conics, comps = ctx.saved_tensors
        W, H, eps2d, calc_comp, camera_model = ctx.params
        if camera_model not in (0, 1, 2):
            raise RuntimeError("GSPlatProjectionEWA3DGSFused vjp: unknown camera model.")
        dev = means.device
        v_means2d = torch.zeros(radii.shape, dtype=torch.float32, device=dev) if v_means2d is None else v_means2d
        v_conics = torch.zeros(conics.shape, dtype=torch.float32, device=dev) if v_conics is None else v_conics
        inputs = {"means": means, "quats": quats, "log_scales": log_scales, "viewmats": viewmats, "Ks": Ks}
        if _nonempty(logits):
            inputs["opacity_logits"] = logits
        fwd = {"radii": radii, "conics": conics}
        cot = {"v_means2d": v_means2d.contiguous(), "v_conics": v_conics.contiguous()}
        if v_depths is not None:  # absent = zeros
            cot["v_depths"] = v_depths.contiguous()
        if calc_comp:
            fwd["compensations"] = comps
            cot["v_compensations"] = (torch.zeros_like(comps) if v_compensations is None
                                      else v_compensations.contiguous())
        if v_opacities is not None:  # absent = zeros
            cot["v_opacities"] = v_opacities.contiguous()
        needs_viewmats = ctx.needs_input_grad[4]
        out = _C.activated_projection_backward(inputs, fwd, cot, W, H, eps2d, camera_model, needs_viewmats)
        g_logits = out["v_opacity_logits"] if ctx.needs_input_grad[3] else None
        g_view = out["v_viewmats"] if needs_viewmats else None
        g_vsp = v_means2d if ctx.needs_input_grad[6] else None
        return (out["v_means"], out["v_quats"], out["v_log_scales"], g_logits, g_view, None, g_vsp) + (None,) * 9


def activated_projection(means, quats, log_scales, opacity_logits, viewmats, Ks, image_width, image_height,
                         viewspace_points=None, eps2d=0.3, near_plane=0.01, far_plane=1e10, radius_clip=0.0,
                         calc_compensations=False, camera_model=0, opacities_in_projection=False):
    """gaussian_activations followed by projection_ewa_3dgs_fused, in the
    projection's kernels: takes the raw parameters (quaternions, log-scales,
    opacity logits) and returns the projection's dict plus the sigmoid
    opacities the rasterizer takes. With opacities_in_projection the
    projection also culls by opacity, as projection_ewa_3dgs_fused(...,
    opacities=...) does."""
    e = _empty(means)
    m2, d, c, comp, r, opac = _ActivatedProjection.apply(
        means, quats, log_scales, opacity_logits if opacity_logits is not None else e, viewmats, Ks,
        viewspace_points if viewspace_points is not None else e, image_width, image_height, eps2d, near_plane,
        far_plane, radius_clip, calc_compensations, camera_model, opacities_in_projection)
    return {"radii": r, "means2d": m2, "depths": d, "conics": c, "compensations": comp,
            "viewspace_points": viewspace_points, "opacities": opac}


_RENDER_RGB_SAVED = ("render_colors", "render_alphas", "last_ids", "radii", "means2d", "conics", "opacities",
                     "tiles_per_gauss", "isect_ids", "flatten_ids", "tile_offsets")


class _RenderRGB(torch.autograd.Function):
    """The RGB render step (activated projection, sorted tile intersection,
    rasterization) as one C++ call per direction: the same operators as the
    composed path, without the interpreter between them."""

    @staticmethod
    def forward(ctx, means, quats, log_scales, colors, opacity_logits, viewmats, Ks, backgrounds, image_width,
                image_height, tile_size, far_plane, opacities_in_projection, accutile):
        ctx.set_materialize_grads(False)
        inputs = {"means": means, "quats": quats, "log_scales": log_scales, "opacity_logits": opacity_logits,
                  "colors": colors, "viewmats": viewmats, "Ks": Ks}
        if _nonempty(backgrounds):
            inputs["backgrounds"] = backgrounds
        out = _C.render_rgb_forward(inputs, image_width, image_height, tile_size, 0.3, 0.01, far_plane,
                                    opacities_in_projection, accutile)
        ctx.save_for_backward(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, backgrounds,
                              *(out[k] for k in _RENDER_RGB_SAVED))
        ctx.dims = (image_width, image_height, tile_size, accutile)
        nd = [out[k] for k in ("last_ids", "radii", "tiles_per_gauss", "isect_ids", "flatten_ids", "tile_offsets")]
        ctx.mark_non_differentiable(*nd)
        return (out["render_colors"], out["render_alphas"], out["last_ids"], out["radii"], out["tiles_per_gauss"],
                out["flatten_ids"], out["isect_ids"], out["tile_offsets"])

    @staticmethod
    def backward(ctx, v_render_colors, v_render_alphas, *_):
        saved = ctx.saved_tensors
        means, quats, log_scales, colors, logits, viewmats, Ks, backgrounds = saved[:8]
        fwd = dict(zip(_RENDER_RGB_SAVED, saved[8:]))
        W, H, ts, accutile = ctx.dims
        inputs = {"means": means, "quats": quats, "log_scales": log_scales, "opacity_logits": logits,
                  "colors": colors, "viewmats": viewmats, "Ks": Ks}
        if _nonempty(backgrounds):
            inputs["backgrounds"] = backgrounds
        if v_render_colors is None:
            v_render_colors = torch.zeros_like(fwd["render_colors"])
        cot = {"v_render_colors": v_render_colors.contiguous()}
        if v_render_alphas is not None:  # absent = zeros
            cot["v_render_alphas"] = v_render_alphas.contiguous()
        needs_viewmats = ctx.needs_input_grad[5]
        out = _C.render_rgb_backward(inputs, fwd, cot, W, H, ts, 0.3, accutile, needs_viewmats)
        return (out["v_means"], out["v_quats"], out["v_log_scales"], out["v_colors"], out["v_opacity_logits"],
                out["v_viewmats"] if needs_viewmats else None) + (None,) * 8


def render_rgb(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, backgrounds, image_width,
               image_height, tile_size, far_plane=1e10, opacities_in_projection=False, accutile=False):
    """Differentiable RGB render step in one C++ call per direction."""
    e = _empty(means)
    rc, ra, li, radii, tpg, flat, ids, offs = _RenderRGB.apply(
        means, quats, log_scales, colors, opacity_logits, viewmats, Ks,
        backgrounds if backgrounds is not None else e, image_width, image_height, tile_size, far_plane,
        opacities_in_projection, accutile)
    return {"render_colors": rc, "render_alphas": ra, "last_ids": li, "radii": radii, "tiles_per_gauss": tpg,
            "flatten_ids": flat, "isect_ids": ids, "tile_offsets": offs}


def render_rgb_l1_value_and_grad(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, target, backgrounds,
                                 image_width, image_height, tile_size, far_plane=1e10, opacities_in_projection=False,
                                 accutile=False):
    """Loss, render outputs and parameter gradients of the RGB step with the
    L1 image loss in one C++ call, as the reference trainer's value_and_grad
    (train_image_fitting_3dgs_mlx.py:165-237): the forward of render_rgb,
    loss = mean |render_colors - target|, and the backward with d loss /
    d loss = 1, without an autograd graph. Returns (loss, render dict, grads
    dict with v_means, v_quats, v_log_scales, v_colors, v_opacity_logits)."""
    inputs = {"means": means.detach(), "quats": quats.detach(), "log_scales": log_scales.detach(),
              "opacity_logits": opacity_logits.detach(), "colors": colors.detach(), "viewmats": viewmats.detach(),
              "Ks": Ks.detach()}
    if _nonempty(backgrounds):
        inputs["backgrounds"] = backgrounds.detach()
    out = _C.render_rgb_l1_value_and_grad(inputs, target.detach(), image_width, image_height, tile_size, 0.3, 0.01,
                                          far_plane, opacities_in_projection, accutile)
    grads = {k: out[k] for k in ("v_means", "v_quats", "v_log_scales", "v_colors", "v_opacity_logits")}
    render = {k: out[k] for k in ("render_colors", "render_alphas", "last_ids", "radii", "tiles_per_gauss",
                                  "flatten_ids", "isect_ids", "tile_offsets")}
    return out["loss"], render, grads


class _L1Loss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, image, target):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        ctx.save_for_backward(image, target)
        return _C.l1_loss_forward(image, target)

    @staticmethod
    def backward(ctx, grad):
        image, target = ctx.saved_tensors
        v_image, v_target = _C.l1_loss_backward(image, target, grad.contiguous())
        return (v_image if ctx.needs_input_grad[0] else None, v_target if ctx.needs_input_grad[1] else None)


def l1_loss(image, target):
    """mean(|image - target|) as a 0-d tensor, forward and backward in HIP."""
    return _L1Loss.apply(image, target)


class _ImageLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, image, target, window_size, with_maps):
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled cotangent
        values, maps = _C.image_loss_forward(image, target, window_size, with_maps)
        ctx.window_size = window_size
        ctx.save_for_backward(image, target, maps)
        return values[0], values[1]

    @staticmethod
    def backward(ctx, g_l1, g_ssim):
        if ctx.needs_input_grad[1]:
            raise NotImplementedError("image_loss: no gradient with respect to the target")
        image, target, maps = ctx.saved_tensors
        e = _empty(image)
        v_image = _C.image_loss_backward(image, target, maps, ctx.window_size,
                                         g_l1.contiguous() if g_l1 is not None else e,
                                         g_ssim.contiguous() if g_ssim is not None else e)
        return v_image, None, None, None


def image_loss(image, target, window_size=11):
    """(mean|image - target|, ssim_index(image, target, window_size)) as two
    0-d tensors for image and target [B, H, W, C], forward and backward in
    HIP (both terms from one pass over the images)."""
    # the derivative maps only when a backward can follow
    with_maps = torch.is_grad_enabled() and image.requires_grad
    return _ImageLoss.apply(image, target, int(window_size), with_maps)
