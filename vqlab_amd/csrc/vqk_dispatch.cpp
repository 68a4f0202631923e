// Options and the two dispatching entry points: VQSwitchLinear.__call__ and
// VQLinear.__call__'s choice between the fused GEMV and the matrix-core
// paths, with the reference's VQ_* flags as arguments (vqk_options) instead
// of module-global environment reads.
#include <stdlib.h>

#include "vqk_common.h"

using namespace vqk;

namespace {

constexpr int64_t kFusedMaxN = 512;       // vq_switch.py:43-45
constexpr int64_t kDenseFusedMaxN = 32;   // vq_dense.py:55-102

vqk_options resolved(const vqk_options *o) {
    vqk_options r;
    vqk_options_default(&r);
    if (o) {
        if (o->fused_max_n > 0) r.fused_max_n = o->fused_max_n;
        if (o->dense_fused_max_n > 0) r.dense_fused_max_n = o->dense_fused_max_n;
        r.decode_bf16io = o->decode_bf16io ? 1 : 0;
        r.prefill_bf16io = o->prefill_bf16io ? 1 : 0;
        r.crowded_grouped = o->crowded_grouped ? 1 : 0;
    }
    return r;
}

int64_t env_i64(const char *name, int64_t dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    char *end = nullptr;
    const long long n = strtoll(v, &end, 10);
    return (end && *end == 0) ? int64_t(n) : dflt;
}

// The grouped GEMM for N pairs of module w (else the fused GEMV). The
// crowded rule (N >= 4 and N >= 2E: the GEMV would read each expert's rows
// once per pair) has no counterpart in the reference's dispatch
// (vq_switch.py:5341-5350); crowded_grouped = 0 turns it off.
bool switch_grouped(const vqk_weights *w, const Geom &g, int64_t N, const vqk_options &o) {
    const bool crowded = o.crowded_grouped && N >= 4 && N >= 2 * g.E;
    if (N <= o.fused_max_n && !crowded) return false;
    return vqk_gemmseg_fits(g.D, g.K, g.G, w->pack_bits, g.IN) != 0;
}

// The reference's decode kernels that stage x as float, and so take bf16 x
// unrounded under VQ_DECODE_BF16IO (vq_switch.py:4412-4417): the unpacked d4
// kernel for K <= 1024 (`_SRC_FUSED`, vq_switch.py:106-150, chosen at
// 3172-3175) and every d8 kernel past the threadgroup-table limit K > 1024
// (`_D8_TG_MAX_K`, 2781; kernels at 153-237, 1316-1354, 1424-1660). The rest
// (d2, packed or large-K d4, d8 with K <= 1024) stage halfN and round.
bool float_staged(const Geom &g) {
    return (g.D == 8 && g.K > 1024) || (g.D == 4 && !g.packed && g.K <= 1024);
}

bool linear_fused(const Geom &g, int64_t N, const vqk_options &o) {
    return N <= o.dense_fused_max_n && vqk_dense_fits(g.K, g.IN, g.G, g.D) != 0;
}

}  // namespace

extern "C" {

void vqk_options_default(vqk_options *o) {
    if (!o) return;
    o->fused_max_n = kFusedMaxN;
    o->dense_fused_max_n = kDenseFusedMaxN;
    o->decode_bf16io = 0;
    o->prefill_bf16io = 0;
    o->crowded_grouped = 1;
}

void vqk_options_from_env(vqk_options *o) {
    if (!o) return;
    vqk_options_default(o);
    o->fused_max_n = env_i64("VQ_FUSED_MAX_N", kFusedMaxN);
    o->dense_fused_max_n = env_i64("VQ_DENSE_FUSED_MAX_N", kDenseFusedMaxN);
    o->decode_bf16io = env_i64("VQ_DECODE_BF16IO", 0) == 1;
    o->prefill_bf16io = env_i64("VQ_GEMMSEG_BF16IO", 0) == 1;
}

int vqk_switch_apply_workspace(const vqk_weights *w, int64_t N, const vqk_options *opt, size_t *bytes) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (!bytes || N < 0) return set_error(VQK_EINVAL, "bad arguments");
    const vqk_options o = resolved(opt);
    if (!switch_grouped(w, g, N, o)) {
        *bytes = 0;
        return VQK_OK;
    }
    return vqk_grouped_gemm_workspace(w, N, bytes);
}

int vqk_switch_apply(const vqk_weights *w, const void *x, int32_t x_type, int64_t T,
                     const uint32_t *eidx, int64_t N, int64_t xkrep, void *y, int32_t y_type,
                     void *workspace, size_t ws_bytes, const vqk_options *opt, void *stream) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (N < 0) return set_error(VQK_EINVAL, "N=%lld", (long long)N);
    const vqk_options o = resolved(opt);
    const bool grouped = switch_grouped(w, g, N, o);
    // the reference's default: fused (and grouped) outputs come back as fp16
    // and are cast to x's dtype by the caller (vq_switch.py:5306-5308, 5423);
    // the bf16-I/O flags keep one rounding only for bf16 x (_keep_bf16 =
    // flag and in_dtype == bf16, vq_switch.py:5306, 5369)
    const bool keep = (grouped ? o.prefill_bf16io : o.decode_bf16io) && x_type == VQK_BF16;
    const bool via = !keep;
    const int32_t yt = via ? (y_type | VQK_VIA_F16) : y_type;
    if (grouped)
        return vqk_grouped_gemm(w, x, x_type, T, eidx, N, xkrep, y, yt, workspace, ws_bytes, stream);
    const int32_t xt = keep && float_staged(g) ? (x_type | VQK_X_KEEP) : x_type;
    return vqk_moe_expert_gemv(w, x, xt, T, eidx, N, xkrep, y, yt, stream);
}

int vqk_linear_apply_workspace(const vqk_weights *w, int64_t N, const vqk_options *opt, size_t *bytes) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (!bytes || N < 0) return set_error(VQK_EINVAL, "bad arguments");
    const vqk_options o = resolved(opt);
    if (linear_fused(g, N, o)) {
        *bytes = 0;
        return VQK_OK;
    }
    return vqk_dense_gemm_workspace(w, N, bytes);
}

int vqk_linear_apply(const vqk_weights *w, const void *x, int32_t x_type, int64_t N, void *y,
                     int32_t y_type, void *workspace, size_t ws_bytes, const vqk_options *opt,
                     void *stream) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (N < 0) return set_error(VQK_EINVAL, "N=%lld", (long long)N);
    const vqk_options o = resolved(opt);
    if (linear_fused(g, N, o)) {
        // the reference has no fused d8 dense kernel (dense_fits refuses d8,
        // vq_switch.py:3290-3306): its d8 linears run decode-then-matmul in
        // x's type at every N (vq_dense.py:288-294), so bf16 / fp32 x is
        // taken unrounded here too
        const int32_t xt = g.D == 8 && x_type != VQK_F16 ? (x_type | VQK_X_KEEP) : x_type;
        return vqk_dense_gemv(w, x, xt, N, y, y_type, stream);
    }
    return vqk_dense_gemm(w, x, x_type, N, y, y_type, workspace, ws_bytes, stream);
}

}  // extern "C"
