"""gsplat_core for AMD Instinct MI355X (gfx950).

Drop-in for the reference package (python_package/gsplat_core/__init__.py:1-4,
``from ._gsplat_core import *``): the same ten operator functions, dict
inputs and output keys, computed by hand-written HIP kernels. Inputs are torch
tensors on a ROCm device; there is no CPU fallback -- importing fails loudly
when the compiled extension is missing (build it with
``python gsplat-mlx_amd/build.py``).
"""
import torch  # noqa: F401  (loads torch's HIP runtime before the extension)

try:
    from . import _gsplat_core  # noqa: F401
    from ._gsplat_core import *  # noqa: F401,F403
except ImportError as exc:  # pragma: no cover - exercised only on broken installs
    raise ImportError(
        "gsplat_core: the compiled extension (_gsplat_core / libgsplat_hip.so) is missing or failed to load; "
        "build it with `python gsplat-mlx_amd/build.py`."
    ) from exc

from .autograd import (  # noqa: E402,F401
    activated_projection,
    activated_projection_packed,
    gaussian_activations,
    image_loss,
    l1_loss,
    packed_rows,
    packed_viewspace,
    projection_ewa_3dgs_fused,
    projection_packed,
    quat_scale_to_covar_preci,
    rasterize_to_pixels_3dgs,
    sh_camera_colors,
    spherical_harmonics,
)

__all__ = [
    "dummy_add",
    "dummy_array_add",
    "projection_ewa_3dgs_fused_forward",
    "projection_ewa_3dgs_fused_backward",
    "intersect_tile_forward",
    "intersect_offset_forward",
    "intersect_tile_offsets_forward",
    "intersect_tile_offsets_begin",
    "intersect_tile_offsets_end",
    "rasterize_to_pixels_3dgs_forward",
    "rasterize_to_pixels_3dgs_backward",
    "spherical_harmonics_forward",
    "spherical_harmonics_backward",
    "quat_scale_to_covar_preci_forward",
    "quat_scale_to_covar_preci_backward",
    "sh_camera_colors_forward",
    "sh_camera_colors_backward",
    "gaussian_activations_forward",
    "gaussian_activations_backward",
    "activated_projection_forward",
    "activated_projection_backward",
    "activated_projection_packed_forward",
    "activated_projection_packed_backward",
    "packed_rows_gather",
    "packed_rows_scatter",
    "l1_loss_forward",
    "l1_loss_backward",
    "image_loss_forward",
    "image_loss_backward",
    "projection_ewa_3dgs_packed_forward",
    "projection_ewa_3dgs_packed_backward",
    "rasterize_to_indices_3dgs_forward",
    "selective_adam_update",
    "activated_projection",
    "activated_projection_packed",
    "gaussian_activations",
    "image_loss",
    "l1_loss",
    "projection_ewa_3dgs_fused",
    "projection_packed",
    "packed_rows",
    "packed_viewspace",
    "quat_scale_to_covar_preci",
    "rasterize_to_pixels_3dgs",
    "sh_camera_colors",
    "spherical_harmonics",
]
