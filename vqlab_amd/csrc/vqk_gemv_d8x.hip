// Wide-x fast VQ GEMV instances for d=8 (x_type flag VQK_X_KEEP): x staged
// as fp32, fp32 products with the widened table entries. Same widths and
// scale groups as the fp16-x instances.
#include "vqk_gemv.h"

namespace vqk {

template <int BITS, int GPB>
static int go_d8x(const GemvParams &p, dim3 grid, size_t smem, hipStream_t st) {
    return launch_with_lds<k_gemv_fast<8, BITS, GPB, true>>(grid, dim3(kThreads), smem, st, p);
}

int launch_gemv_fast_d8x(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem,
                         hipStream_t st) {
#define VQK_CASE(B)                                                        \
    case B:                                                                \
        if (gpb == 1) return go_d8x<B, 1>(p, grid, smem, st);             \
        if (gpb == 4) return go_d8x<B, 4>(p, grid, smem, st);             \
        break;
    switch (bits) {
        VQK_CASE(2) VQK_CASE(3) VQK_CASE(4) VQK_CASE(5) VQK_CASE(6) VQK_CASE(7)
        VQK_CASE(8) VQK_CASE(9) VQK_CASE(10) VQK_CASE(11) VQK_CASE(12) VQK_CASE(13)
        VQK_CASE(14) VQK_CASE(15) VQK_CASE(16)
        default: break;
    }
#undef VQK_CASE
    return set_error(VQK_ENOTIMPL, "no fast wide-x d=8 kernel for bits=%d, %d groups/block", bits, gpb);
}

}  // namespace vqk
