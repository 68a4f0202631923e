// Fast VQ GEMV instances for d=2: every packed width 2..16 (8 and 16 also
// serve unpacked uint8 / uint16 rows), scale groups of 64 or more weights
// (one group spans one or more whole blocks).
#include "vqk_gemv.h"

namespace vqk {

template <int BITS, int GPB>
static int go_d2(const GemvParams &p, dim3 grid, size_t smem, hipStream_t st) {
    return launch_with_lds<k_gemv_fast<2, BITS, GPB>>(grid, dim3(kThreads), smem, st, p);
}

int launch_gemv_fast_d2(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem,
                        hipStream_t st) {
#define VQK_CASE(B)                                                        \
    case B:                                                                \
        if (gpb == 1) return go_d2<B, 1>(p, grid, smem, st);              \
        break;
    switch (bits) {
        VQK_CASE(2) VQK_CASE(3) VQK_CASE(4) VQK_CASE(5) VQK_CASE(6) VQK_CASE(7)
        VQK_CASE(8) VQK_CASE(9) VQK_CASE(10) VQK_CASE(11) VQK_CASE(12) VQK_CASE(13)
        VQK_CASE(14) VQK_CASE(15) VQK_CASE(16)
        default: break;
    }
#undef VQK_CASE
    return set_error(VQK_ENOTIMPL, "no fast d=2 kernel for bits=%d, %d groups/block", bits, gpb);
}

}  // namespace vqk
