// Wide-x fast VQ GEMV instances (x_type flag VQK_X_KEEP): x staged as fp32,
// fp32 products with the widened table entries. d=8: the widths and scale
// groups of the fp16-x instances; d=4: the unpacked uint8 / uint16 rows (the
// reference's float-staged d4 kernel takes unpacked codes only).
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

template <int BITS, int GPB>
static int go_d4x(const GemvParams &p, dim3 grid, size_t smem, hipStream_t st) {
    return launch_with_lds<k_gemv_fast<4, BITS, GPB, true>>(grid, dim3(kThreads), smem, st, p);
}

bool gemv_fast_d4x_has(int bits) { return bits == 8 || bits == 16; }

int launch_gemv_fast_d4x(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem,
                         hipStream_t st) {
    if (bits == 8 && gpb == 1) return go_d4x<8, 1>(p, grid, smem, st);
    if (bits == 8 && gpb == 2) return go_d4x<8, 2>(p, grid, smem, st);
    if (bits == 16 && gpb == 1) return go_d4x<16, 1>(p, grid, smem, st);
    if (bits == 16 && gpb == 2) return go_d4x<16, 2>(p, grid, smem, st);
    return set_error(VQK_ENOTIMPL, "no fast wide-x d=4 kernel for bits=%d, %d groups/block", bits, gpb);
}

}  // namespace vqk
