// Fused EWA projection operator API; mirrors
// gsplat_core/include/gsplat_projection.h:12-77 of the reference.
#pragma once

#include "gsplat_common.h"

namespace gsplat_core {

struct ProjectionEWA3DGSFusedParams {
  int image_width;
  int image_height;
  float eps2d;
  float near_plane;
  float far_plane;
  float radius_clip;
  bool calc_compensations;
  int camera_model;
  bool use_covars;
  bool use_opacities;
};

struct ProjectionEWA3DGSFusedInput {
  array means;
  array covars;
  array quats;
  array scales;
  array opacities;
  array viewmats;
  array Ks;
  array viewspace_points;
  StreamOrDevice s;
  ProjectionEWA3DGSFusedParams params;
};

struct ProjectionEWA3DGSFusedBackwardInput {
  array means;
  array covars;
  array quats;
  array scales;
  array viewmats;
  array Ks;
  array radii;
  array conics;
  array compensations;
  array v_means2d;
  array v_depths;
  array v_conics;
  array v_compensations;
  StreamOrDevice s;
  ProjectionEWA3DGSFusedParams params;
  bool viewmats_requires_grad;
};

enum ProjectionEWA3DGSFusedOutputIndex {
  kMeans2D = 0,
  kDepths = 1,
  kConics = 2,
  kCompensations = 3,
  kRadii = 4,
};

enum ProjectionEWA3DGSFusedBackwardOutputIndex {
  kProjectionVMeans = 0,
  kProjectionVCovars = 1,
  kProjectionVQuats = 2,
  kProjectionVScales = 3,
  kProjectionVViewmats = 4,
};

std::vector<array> gsplat_projection_ewa_3dgs_fused(const ProjectionEWA3DGSFusedInput& input);

std::vector<array> gsplat_projection_ewa_3dgs_fused_backward(const ProjectionEWA3DGSFusedBackwardInput& input);

// Packed layout: upstream gsplat's fully_fused_projection(packed=True), the
// reference's intended projection_ewa_3dgs_packed_forward
// (note/gsplat_cuda_source_map.md:273-315). Only the visible (camera,
// Gaussian) pairs, nnz of them, ordered by (batch, camera, gaussian); each row
// equals the dense output of its pair. ids are int32; indptr [B*C + 1] holds
// each camera's first row. Reads the count back to the host (one sync).
enum ProjectionEWA3DGSPackedOutputIndex {
  kPackedBatchIds = 0,
  kPackedCameraIds = 1,
  kPackedGaussianIds = 2,
  kPackedIndptr = 3,
  kPackedRadii = 4,
  kPackedMeans2D = 5,
  kPackedDepths = 6,
  kPackedConics = 7,
  kPackedCompensations = 8,
};

std::vector<array> gsplat_projection_ewa_3dgs_packed(const ProjectionEWA3DGSFusedInput& input);

// Cotangents v_* [nnz, ...] of the packed outputs; the ids must be the
// forward's. Outputs as the dense backward (ProjectionEWA3DGSFusedBackward
// OutputIndex), equal to it with the cotangents scattered to their pairs.
struct ProjectionEWA3DGSPackedBackwardInput {
  array means;
  array covars;
  array quats;
  array scales;
  array viewmats;
  array Ks;
  array batch_ids;
  array camera_ids;
  array gaussian_ids;
  array conics;
  array compensations;
  array v_means2d;
  array v_depths;
  array v_conics;
  array v_compensations;
  StreamOrDevice s;
  ProjectionEWA3DGSFusedParams params;
  bool viewmats_requires_grad;
};

std::vector<array> gsplat_projection_ewa_3dgs_packed_backward(const ProjectionEWA3DGSPackedBackwardInput& input);

}  // namespace gsplat_core
