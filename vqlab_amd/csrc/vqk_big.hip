// k_gemv_big instances: the widths whose 2^BITS-entry table exceeds the
// LDS-resident limit of the block-per-lane GEMV (d8 >= 13 bits, d4 >= 14,
// d2 >= 15; 16 also serves unpacked uint16 codes), scale groups as the GEMV.
#include "vqk_big.h"
#include "vqk_internal.h"

namespace vqk {

namespace {
template <int D, int BITS, int GPB>
int go(const BigParams &p, dim3 grid, hipStream_t st) {
    return launch_with_lds<k_gemv_big<D, BITS, GPB>>(grid, dim3(kBigThreads), big_lds(D, p.IN), st, p);
}
}  // namespace

int launch_gemv_big(const BigParams &p, int D, int bits, int gpb, dim3 grid, hipStream_t st) {
    switch (D * 1000 + bits * 16 + gpb) {
        case 2241: return go<2, 15, 1>(p, grid, st);
        case 2257: return go<2, 16, 1>(p, grid, st);
        case 4225: return go<4, 14, 1>(p, grid, st);
        case 4226: return go<4, 14, 2>(p, grid, st);
        case 4241: return go<4, 15, 1>(p, grid, st);
        case 4242: return go<4, 15, 2>(p, grid, st);
        case 4257: return go<4, 16, 1>(p, grid, st);
        case 4258: return go<4, 16, 2>(p, grid, st);
        case 8209: return go<8, 13, 1>(p, grid, st);
        case 8212: return go<8, 13, 4>(p, grid, st);
        case 8225: return go<8, 14, 1>(p, grid, st);
        case 8228: return go<8, 14, 4>(p, grid, st);
        case 8241: return go<8, 15, 1>(p, grid, st);
        case 8244: return go<8, 15, 4>(p, grid, st);
        case 8257: return go<8, 16, 1>(p, grid, st);
        case 8260: return go<8, 16, 4>(p, grid, st);
        default: return set_error(VQK_ENOTIMPL, "no sliced-codebook GEMV for d=%d bits=%d gpb=%d", D, bits, gpb);
    }
}

void big_seg_weights(const vqk_weights *w, const Geom &g, BigSeg *s) {
    s->codes = static_cast<const uint32_t *>(w->codes);
    s->row_words = g.row_words;
    s->codebook = w->codebook;
    s->K = int32_t(g.K);
    s->scales = w->scales;
    s->ngrp = int32_t(g.NGRP);
    s->bpg = g.bpg;
    s->row_table = w->row_table;
    s->stored_rows = g.rows;
    s->E = int32_t(g.E);
    s->OUT = int32_t(g.OUT);
}

int big_plan_rows(BigParams *p, int64_t NB, int64_t OUT, int64_t total_rows) {
    int l = 0;
    while ((int64_t(1) << l) < NB) ++l;
    p->lpr_log2 = l;
    const int64_t per_step = int64_t(kBigThreads / kWave) * (kWave >> l);
    // as many row steps per item as keep one item per CU, at most kBigSteps
    int64_t steps = (total_rows + per_step * big_grid(INT32_MAX) - 1) / (per_step * big_grid(INT32_MAX));
    const int64_t fit = (OUT + per_step - 1) / per_step;
    steps = steps < 1 ? 1 : steps;
    steps = steps > fit ? fit : steps;
    p->steps = int32_t(steps < kBigSteps ? steps : kBigSteps);
    return int(p->steps * per_step);
}

int big_grid(int64_t items) {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return int(items < cus[dev] ? items : cus[dev]);
}

bool big_fits(const Geom &g, const vqk_weights *w) {
    return g.fast_ok && !cb_in_lds(g.D, g.BITS) && g.IN % 8 == 0 &&
           big_lds(g.D, g.IN) <= 160 * 1024 && g.OUT <= INT32_MAX && g.K <= INT32_MAX &&
           (reinterpret_cast<uintptr_t>(w->codebook) & 15) == 0;
}

}  // namespace vqk
