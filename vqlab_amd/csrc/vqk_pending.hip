// Entry points whose kernels are not written yet: each refuses explicitly.
#include "vqk_common.h"

using namespace vqk;

extern "C" {

int vqk_grouped_gemm_workspace(const vqk_weights *, int64_t, size_t *bytes) {
    if (bytes) *bytes = 0;
    return set_error(VQK_ENOTIMPL, "grouped GEMM not built yet");
}
int vqk_grouped_gemm(const vqk_weights *, const void *, int32_t, int64_t, const uint32_t *,
                     int64_t, int64_t, void *, int32_t, void *, size_t, void *) {
    return set_error(VQK_ENOTIMPL, "grouped GEMM not built yet");
}
int vqk_dense_gemm(const vqk_weights *, const void *, int32_t, int64_t, void *, int32_t, void *) {
    return set_error(VQK_ENOTIMPL, "dense GEMM not built yet");
}
int vqk_gemmseg_fits(int32_t, int64_t, int32_t, int32_t, int64_t) { return 0; }

}
