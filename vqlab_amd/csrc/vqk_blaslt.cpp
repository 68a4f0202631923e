// The plain GEMM of the dense decode-then-matmul path (after the bit-exact
// weight decode), on hipBLASLt: y[N, M] = x[N, K] . W[M, K]^T in fp16 or bf16
// with fp32 accumulation, the reference's `xf @ w.T.astype(xf.dtype)`
// (vq_dense.py:288, 294). One hipBLASLt handle per device and one plan per
// shape are created on first use and kept for the process; the caller's
// workspace is the only device memory a call uses. The plan's algorithm is
// the fastest of the heuristic's first candidates whose scratch fits, timed
// on that first call with the caller's own buffers (the heuristic's first
// pick ran 35 % slower than its second on a config-5 linear); the timing
// synchronises the stream once per shape, and is skipped (first pick) while
// the stream is being captured into a graph or with VQK_GEMM_TUNE=0
// (VQK_GEMM_VERBOSE=1 prints each candidate's time to stderr).
#include <hipblaslt/hipblaslt.h>

#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <vector>

#include "vqk_common.h"

namespace vqk {
namespace {

struct LtPlan {
    int dev;
    int32_t type;
    int64_t m, n, k, ldw, ldx, ldy;
    size_t ws;
    hipblasLtMatmulDesc_t md;
    hipblasLtMatrixLayout_t lw, lx, ly;
    hipblasLtMatmulAlgo_t algo;
    bool ok;
};

std::mutex g_mu;
hipblasLtHandle_t g_handle[64];
std::vector<LtPlan> g_plans;

struct LtCall {             // the first call's operands, used to time candidates
    const void *W, *X;
    void *Y, *ws;
    hipStream_t st;
};

bool tuning_allowed(hipStream_t st) {
    const char *v = getenv("VQK_GEMM_TUNE");
    if (v && v[0] == '0') return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return false;
    return cs == hipStreamCaptureStatusNone;
}

// Average time of `algo` over a few runs on the caller's stream, or a
// negative value when it fails.
float time_algo(hipblasLtHandle_t h, const LtPlan &p, const hipblasLtMatmulAlgo_t &algo,
                const LtCall &c) {
    const float alpha = 1.f, beta = 0.f;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess) return -1.f;
    if (hipEventCreate(&e1) != hipSuccess) { hipEventDestroy(e0); return -1.f; }
    float ms = -1.f;
    bool ok = hipblasLtMatmul(h, p.md, &alpha, c.W, p.lw, c.X, p.lx, &beta, c.Y, p.ly, c.Y, p.ly,
                              &algo, p.ws ? c.ws : nullptr, p.ws, c.st) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipEventRecord(e0, c.st) == hipSuccess;
    for (int i = 0; ok && i < 3; ++i)
        ok = hipblasLtMatmul(h, p.md, &alpha, c.W, p.lw, c.X, p.lx, &beta, c.Y, p.ly, c.Y, p.ly,
                             &algo, p.ws ? c.ws : nullptr, p.ws, c.st) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipEventRecord(e1, c.st) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
         hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    return ok ? ms : -1.f;
}

bool make_plan(hipblasLtHandle_t h, LtPlan *p, const LtCall &c) {
    const hipDataType dt = p->type == VQK_BF16 ? HIP_R_16BF : HIP_R_16F;
    p->ok = false;
    if (hipblasLtMatmulDescCreate(&p->md, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return false;
    // column-major view: y^T [M, N] = W [M, K] (stored as W^T [K, M]) . x^T [K, N]
    const hipblasOperation_t tw = HIPBLAS_OP_T, tx = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p->md, HIPBLASLT_MATMUL_DESC_TRANSA, &tw, sizeof tw);
    hipblasLtMatmulDescSetAttribute(p->md, HIPBLASLT_MATMUL_DESC_TRANSB, &tx, sizeof tx);
    if (hipblasLtMatrixLayoutCreate(&p->lw, dt, uint64_t(p->k), uint64_t(p->m), p->ldw) ||
        hipblasLtMatrixLayoutCreate(&p->lx, dt, uint64_t(p->k), uint64_t(p->n), p->ldx) ||
        hipblasLtMatrixLayoutCreate(&p->ly, dt, uint64_t(p->m), uint64_t(p->n), p->ldy))
        return false;
    hipblasLtMatmulPreference_t pref;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
    uint64_t wsb = p->ws;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                          sizeof wsb);
    hipblasLtMatmulHeuristicResult_t res[16];
    int n = 0;
    const hipblasStatus_t s = hipblasLtMatmulAlgoGetHeuristic(h, p->md, p->lw, p->lx, p->ly, p->ly,
                                                              pref, 16, res, &n);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS) return false;
    const bool tune = tuning_allowed(c.st);
    const char *vv = getenv("VQK_GEMM_VERBOSE");   // print each candidate's time
    const bool verbose = vv && vv[0] == '1';
    float best = -1.f;
    for (int i = 0, tried = 0; i < n && tried < 8; ++i) {   // the heuristic's order
        if (res[i].workspaceSize > p->ws) continue;
        if (!tune) {
            p->algo = res[i].algo;
            p->ok = true;
            return true;
        }
        ++tried;
        const float ms = time_algo(h, *p, res[i].algo, c);
        if (verbose)
            fprintf(stderr, "vqk gemm M %lld N %lld K %lld: candidate %d (scratch %zu B) %.4f ms\n",
                    (long long)p->m, (long long)p->n, (long long)p->k, i,
                    size_t(res[i].workspaceSize), ms);
        if (ms >= 0.f && (best < 0.f || ms < best)) {
            best = ms;
            p->algo = res[i].algo;
            p->ok = true;
        }
    }
    return p->ok;
}

}  // namespace

// VQK_ENOTIMPL (with its message set) when hipBLASLt has no algorithm for
// the shape: the caller then takes its own GEMM kernel.
int lt_gemm_nt(int32_t type, const void *W, int64_t ldw, const void *X, int64_t ldx, void *Y,
               int64_t ldy, int64_t M, int64_t N, int64_t K, void *ws, size_t ws_bytes,
               hipStream_t st) {
    if ((type != VQK_F16 && type != VQK_BF16) || M <= 0 || N <= 0 || K <= 0)
        return set_error(VQK_ENOTIMPL, "library GEMM: type %d, M %lld N %lld K %lld", type,
                         (long long)M, (long long)N, (long long)K);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return set_error(VQK_ENOTIMPL, "library GEMM: no current device");
    const size_t wsc = ws ? (ws_bytes < (size_t(64) << 20) ? ws_bytes : (size_t(64) << 20)) : 0;
    LtPlan plan;
    hipblasLtHandle_t h;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_handle[dev] && hipblasLtCreate(&g_handle[dev]) != HIPBLAS_STATUS_SUCCESS) {
            g_handle[dev] = nullptr;
            return set_error(VQK_ENOTIMPL, "library GEMM: hipblasLtCreate failed");
        }
        h = g_handle[dev];
        const LtPlan *found = nullptr;
        for (const LtPlan &q : g_plans)
            if (q.dev == dev && q.type == type && q.m == M && q.n == N && q.k == K && q.ldw == ldw &&
                q.ldx == ldx && q.ldy == ldy && q.ws == wsc)
                found = &q;
        if (!found) {
            LtPlan q{};
            q.dev = dev; q.type = type; q.m = M; q.n = N; q.k = K;
            q.ldw = ldw; q.ldx = ldx; q.ldy = ldy; q.ws = wsc;
            make_plan(h, &q, LtCall{W, X, Y, ws, st});
            g_plans.push_back(q);
            found = &g_plans.back();
        }
        plan = *found;
    }
    if (!plan.ok)
        return set_error(VQK_ENOTIMPL, "library GEMM: no hipBLASLt algorithm for M %lld N %lld K %lld",
                         (long long)M, (long long)N, (long long)K);
    const float alpha = 1.f, beta = 0.f;
    const hipblasStatus_t s = hipblasLtMatmul(h, plan.md, &alpha, W, plan.lw, X, plan.lx, &beta, Y,
                                              plan.ly, Y, plan.ly, &plan.algo, wsc ? ws : nullptr,
                                              wsc, st);
    if (s != HIPBLAS_STATUS_SUCCESS)
        return set_error(VQK_EINVAL, "hipblasLtMatmul failed (status %d)", int(s));
    return VQK_OK;
}

}  // namespace vqk
