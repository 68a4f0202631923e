// Host entry points of the fused VQ GEMV: vqk_dense_gemv (_dense_fused,
// vq_switch.py:3339-3434) and vqk_moe_expert_gemv (_fused, vq_switch.py:2919-3249).
// Both validate on the host, pick the fast or the generic kernel and launch.
#include "vqk_gemv.h"
#include "vqk_internal.h"

namespace vqk {

static int lpr_log2_for(int64_t nb) {
    int l = 0;
    while ((int64_t(1) << l) < nb) ++l;
    return l;
}

int gemv_fill_params(const vqk_weights *w, const Geom &g, GemvParams *p) {
    memset(p, 0, sizeof *p);
    p->codes = w->codes;
    p->row_words = g.row_words;
    p->code_cols = w->code_cols;
    p->bits = g.packed ? g.BITS : 0;
    p->code_bytes = g.packed ? 4 : g.BITS / 8;
    p->codebook = w->codebook;
    p->K = int32_t(g.K);
    p->scales = w->scales;
    p->ngrp = int32_t(g.NGRP);
    p->bpg = g.bpg;
    p->G = g.G;
    p->row_table = w->row_table;
    p->stored_rows = g.rows;
    p->E = int32_t(g.E);
    p->OUT = int32_t(g.OUT);
    p->IN = int32_t(g.IN);
    p->NSUB = int32_t(g.NSUB);
    p->NB = int32_t(g.NB);
    p->lpr_log2 = lpr_log2_for(g.NB);
    return VQK_OK;
}

size_t gemv_fast_lds(const Geom &g, bool xf) {
    const size_t cb = cb_in_lds(g.D, g.BITS) ? (size_t(1) << g.BITS) * g.D * 2
                                              : size_t(gemv_hyb_bytes(xf));
    // x: NB blocks of 32 * D values at a 16-byte padded stride
    return cb + (xf ? size_t(g.NB) * (kBlock * g.D + 4) * 4 : size_t(g.NB) * (kBlock * g.D + 8) * 2);
}

int launch_gemv(const vqk_weights *w, const void *x, int32_t x_type, int64_t T,
                const uint32_t *eidx, int64_t N, int64_t xkrep, void *y, int32_t y_type,
                hipStream_t st) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    const bool xf = (x_type & VQK_X_KEEP) != 0;
    x_type &= ~int32_t(VQK_X_KEEP);
    if (!act_size(x_type) || !out_size(y_type))
        return set_error(VQK_EINVAL, "x/y type must be VQK_F16, VQK_BF16 or VQK_F32");
    if (xf && g.D == 2)
        return set_error(VQK_EINVAL, "VQK_X_KEEP is for d=4 and d=8 modules (the float-staged "
                                     "kernels); d=2 kernels take x as fp16");
    if ((!x || !y) && N > 0) return set_error(VQK_EINVAL, "x and y are required");
    if (N < 0 || T < 0 || xkrep < 1 || N != T * xkrep)
        return set_error(VQK_EINVAL, "pairs N=%lld must equal tokens T=%lld x xkrep=%lld",
                         (long long)N, (long long)T, (long long)xkrep);
    if (N > INT32_MAX) return set_error(VQK_ENOTIMPL, "N=%lld pairs is too many", (long long)N);
    if (N == 0) return VQK_OK;
    GemvParams p;
    gemv_fill_params(w, g, &p);
    p.eidx = eidx;
    p.x = x;
    p.x_type = x_type;
    p.x_stride = g.IN;
    p.xkrep = int32_t(xkrep);
    p.y = y;
    p.y_type = y_type;
    p.y_stride = g.OUT;
    const int64_t chunk = (65535 / xkrep) * xkrep;   // grid.y limit, whole tokens per chunk
    // wide x at d=4: fast instances for the unpacked widths, else the generic kernel
    const bool fast_x = !xf || g.D == 8 || gemv_fast_d4x_has(g.BITS);
    if (g.fast_ok && fast_x && gemv_fast_lds(g, xf) <= size_t(kLdsBytes)) {
        const int rpw = kWave >> p.lpr_log2;
        const int64_t steps_total = N * ((g.OUT + rpw - 1) / rpw);   // wave steps overall
        const int64_t target_waves = 2048;                          // ~8 per CU
        int64_t steps = (steps_total + target_waves - 1) / target_waves;
        steps = steps < 1 ? 1 : (steps > 16 ? 16 : steps);
        const int64_t per_wg = 4 * rpw * steps;
        p.steps = int32_t(steps);
        p.rows_per_wg = int32_t(per_wg);
        const size_t smem = gemv_fast_lds(g, xf);
        for (int64_t n0 = 0; n0 < N; n0 += chunk) {
            const int64_t nn = N - n0 < chunk ? N - n0 : chunk;
            p.pair0 = int32_t(n0);
            const dim3 grid(unsigned((g.OUT + per_wg - 1) / per_wg), unsigned(nn), 1);
            switch (g.D) {
                case 2: rc = launch_gemv_fast_d2(p, g.BITS, g.gpb, grid, smem, st); break;
                case 4:
                    rc = xf ? launch_gemv_fast_d4x(p, g.BITS, g.gpb, grid, smem, st)
                            : launch_gemv_fast_d4(p, g.BITS, g.gpb, grid, smem, st);
                    break;
                default:
                    rc = xf ? launch_gemv_fast_d8x(p, g.BITS, g.gpb, grid, smem, st)
                            : launch_gemv_fast_d8(p, g.BITS, g.gpb, grid, smem, st);
                    break;
            }
            if (rc) return rc;
        }
        return VQK_OK;
    }
    const size_t smem = size_t(g.IN) * (xf ? 4 : 2);
    if (smem > size_t(kLdsBytes)) return set_error(VQK_ENOTIMPL, "IN=%lld too wide", (long long)g.IN);
    for (int64_t n0 = 0; n0 < N; n0 += chunk) {
        const int64_t nn = N - n0 < chunk ? N - n0 : chunk;
        p.pair0 = int32_t(n0);
        const dim3 grid(unsigned((g.OUT + kThreads - 1) / kThreads), unsigned(nn), 1);
        switch (g.D) {
            case 2: rc = launch_with_lds<k_gemv_generic<2>>(grid, dim3(kThreads), smem, st, p); break;
            case 4:
                rc = xf ? launch_with_lds<k_gemv_generic<4, true>>(grid, dim3(kThreads), smem, st, p)
                        : launch_with_lds<k_gemv_generic<4>>(grid, dim3(kThreads), smem, st, p);
                break;
            default:
                rc = xf ? launch_with_lds<k_gemv_generic<8, true>>(grid, dim3(kThreads), smem, st, p)
                        : launch_with_lds<k_gemv_generic<8>>(grid, dim3(kThreads), smem, st, p);
                break;
        }
        if (rc) return rc;
    }
    return VQK_OK;
}

}  // namespace vqk

using namespace vqk;

extern "C" {

int vqk_dense_gemv(const vqk_weights *w, const void *x, int32_t x_type, int64_t N, void *y,
                   int32_t y_type, void *stream) {
    if (w && w->E != 1)
        return set_error(VQK_EINVAL, "dense GEMV takes one linear (E=1), got E=%lld",
                         (long long)w->E);
    return launch_gemv(w, x, x_type, N, nullptr, N, 1, y, y_type, hipStream_t(stream));
}

int vqk_moe_expert_gemv(const vqk_weights *w, const void *x, int32_t x_type, int64_t T,
                        const uint32_t *eidx, int64_t N, int64_t xkrep, void *y, int32_t y_type,
                        void *stream) {
    if (!eidx && N > 0) return set_error(VQK_EINVAL, "eidx is required");
    return launch_gemv(w, x, x_type, T, eidx, N, xkrep, y, y_type, hipStream_t(stream));
}

}  // extern "C"
