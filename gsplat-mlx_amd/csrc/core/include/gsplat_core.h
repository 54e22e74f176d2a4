// Umbrella header of the gsplat_core C++ operator API (MI355X build).
#pragma once

#include "gsplat_intersect.h"
#include "gsplat_projection.h"
#include "gsplat_quat_scale_to_covar.h"
#include "gsplat_rasterize.h"
#include "gsplat_render.h"
#include "gsplat_spherical_harmonics.h"
#include "gsplat_training_glue.h"
