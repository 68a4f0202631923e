// k_seg_mfma instances for d = 2: every packed width 2..16 (8 / 16 also
// serve unpacked uint8 / uint16 rows) x the scale-group layouts of the GEMV.
#include "vqk_gseg.h"

namespace vqk {

namespace {
template <int BITS, int GPB>
int go(const SegParams &p, dim3 grid, hipStream_t st) {
    constexpr bool CBL = cb_in_lds(2, BITS);
    return launch_with_lds<k_seg_mfma<2, BITS, GPB, CBL>>(grid, dim3(kSegWaves * 64), seg_lds(2, BITS, CBL), st, p);
}
}  // namespace

int launch_seg_d2(const SegParams &p, int bits, int gpb, dim3 grid, hipStream_t st) {
    switch (bits * 16 + gpb) {
        case 33: return go<2, 1>(p, grid, st);
        case 49: return go<3, 1>(p, grid, st);
        case 65: return go<4, 1>(p, grid, st);
        case 81: return go<5, 1>(p, grid, st);
        case 97: return go<6, 1>(p, grid, st);
        case 113: return go<7, 1>(p, grid, st);
        case 129: return go<8, 1>(p, grid, st);
        case 145: return go<9, 1>(p, grid, st);
        case 161: return go<10, 1>(p, grid, st);
        case 177: return go<11, 1>(p, grid, st);
        case 193: return go<12, 1>(p, grid, st);
        case 209: return go<13, 1>(p, grid, st);
        case 225: return go<14, 1>(p, grid, st);
        case 241: return go<15, 1>(p, grid, st);
        case 257: return go<16, 1>(p, grid, st);
        default: return set_error(VQK_ENOTIMPL, "no segment kernel for d=2 bits=%d gpb=%d", bits, gpb);
    }
}

}  // namespace vqk
