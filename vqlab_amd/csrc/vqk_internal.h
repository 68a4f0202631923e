// Host-side helpers shared between libvqk translation units.
#pragma once

#include <string.h>

#include "vqk_gemv.h"

namespace vqk {

// Fills the weight-dependent fields of a GEMV parameter block.
int gemv_fill_params(const vqk_weights *w, const Geom &g, GemvParams *p);

// Dynamic LDS bytes of the fast GEMV kernel for geometry g (xf: the wide-x
// instances).
size_t gemv_fast_lds(const Geom &g, bool xf = false);

// Validates and launches the fused GEMV for N = T * xkrep pairs.
int launch_gemv(const vqk_weights *w, const void *x, int32_t x_type, int64_t T,
                const uint32_t *eidx, int64_t N, int64_t xkrep, void *y, int32_t y_type,
                hipStream_t st);

// min(items, the current device's CU count): the grid of a kernel that
// keeps one workgroup per CU (vqk_big.hip).
int big_grid(int64_t items);

// ---- grouped expert GEMM pieces (vqk_gemm.hip): sort one routing, then run
// several projections over it with the register-decode segment kernel.
struct SegCall {
    const void *x;             // activations (x_type), or NULL with xg / xu:
    int32_t x_type;
    const float *xg, *xu;      //   row = fp16(silu(xg) * xu), fp32 rows of the module's IN
    int64_t xkrep;             // x row of pair n = n / xkrep
    void *y;                   // y[pair, OUT] in y_type
    int32_t y_type;
    int64_t N;                 // pairs (sorted) or dense rows (sort_ws == NULL)
    int32_t tok;               // sorted: the sort's tile rows (seg_tile_rows); 0 = 16
    int32_t ksplit;            // dense rows only: K slices, y holds ksplit fp32 partials
                               //   [ksplit][N][OUT] (0 or 1: no split)
    int32_t xparts;            // xg / xu hold xparts partial rows [xparts][N][IN] to add
};

// Rows per tile to sort N pairs into for module `w` over E experts:
// kSegTokNarrow when the routing puts at most ~2 pairs on an expert on
// average and w's d8 table is beyond LDS (more of it fits beside a narrow x
// chunk; the sort then picks 4- or 8-row tiles on device), else 16.
int seg_tile_rows(const vqk_weights *w, int64_t N, int64_t E);

// K slices for the segment kernel over N dense rows of `w`: enough that the
// launch fills the CUs once (at most 4 and the module's supersteps).
int seg_ksplit(const vqk_weights *w, int64_t N);

// Workspace of seg_sort for N pairs over E experts.
size_t seg_sort_bytes(int64_t N, int64_t E);

// True when the segment kernel takes module `w` for N pairs.
bool seg_ok(const vqk_weights *w, int64_t N);

// Counting sort of N pair experts (device uint32, out-of-range ids form dead
// tiles) into `ws`: pair order, records of tiles of at most `tok` rows (16
// or 4) and the tile count.
int seg_sort(const uint32_t *eidx, int64_t N, int64_t E, int tok, void *ws, hipStream_t st);

// One projection over a routing sorted into `sort_ws` (or over N dense rows
// of expert 0 when sort_ws is NULL).
int seg_run(const vqk_weights *w, const SegCall &c, const void *sort_ws, hipStream_t st);

}  // namespace vqk
