// Host-side helpers shared between libvqk translation units.
#pragma once

#include <string.h>

#include "vqk_gemv.h"

namespace vqk {

// Fills the weight-dependent fields of a GEMV parameter block.
int gemv_fill_params(const vqk_weights *w, const Geom &g, GemvParams *p);

// Dynamic LDS bytes of the fast GEMV kernel for geometry g.
size_t gemv_fast_lds(const Geom &g);

// Validates and launches the fused GEMV for N = T * xkrep pairs.
int launch_gemv(const vqk_weights *w, const void *x, int32_t x_type, int64_t T,
                const uint32_t *eidx, int64_t N, int64_t xkrep, void *y, int32_t y_type,
                hipStream_t st);

}  // namespace vqk
