// k_seg_mfma instances for d = 4: every packed width 2..16 (8 / 16 also
// serve unpacked uint8 / uint16 rows) x the scale-group layouts of the GEMV.
#include "vqk_gseg.h"

namespace vqk {

namespace {
template <int BITS, int GPB>
int go(const SegParams &p, dim3 grid, hipStream_t st) {
    constexpr bool CBL = cb_in_lds(4, BITS);
    return launch_with_lds<k_seg_mfma<4, BITS, GPB, CBL>>(grid, dim3(kSegWaves * 64), seg_lds(4, BITS, CBL), st, p);
}
}  // namespace

int launch_seg_d4(const SegParams &p, int bits, int gpb, dim3 grid, hipStream_t st) {
    switch (bits * 16 + gpb) {
        case 33: return go<2, 1>(p, grid, st);
        case 34: return go<2, 2>(p, grid, st);
        case 49: return go<3, 1>(p, grid, st);
        case 50: return go<3, 2>(p, grid, st);
        case 65: return go<4, 1>(p, grid, st);
        case 66: return go<4, 2>(p, grid, st);
        case 81: return go<5, 1>(p, grid, st);
        case 82: return go<5, 2>(p, grid, st);
        case 97: return go<6, 1>(p, grid, st);
        case 98: return go<6, 2>(p, grid, st);
        case 113: return go<7, 1>(p, grid, st);
        case 114: return go<7, 2>(p, grid, st);
        case 129: return go<8, 1>(p, grid, st);
        case 130: return go<8, 2>(p, grid, st);
        case 145: return go<9, 1>(p, grid, st);
        case 146: return go<9, 2>(p, grid, st);
        case 161: return go<10, 1>(p, grid, st);
        case 162: return go<10, 2>(p, grid, st);
        case 177: return go<11, 1>(p, grid, st);
        case 178: return go<11, 2>(p, grid, st);
        case 193: return go<12, 1>(p, grid, st);
        case 194: return go<12, 2>(p, grid, st);
        case 209: return go<13, 1>(p, grid, st);
        case 210: return go<13, 2>(p, grid, st);
        case 225: return go<14, 1>(p, grid, st);
        case 226: return go<14, 2>(p, grid, st);
        case 241: return go<15, 1>(p, grid, st);
        case 242: return go<15, 2>(p, grid, st);
        case 257: return go<16, 1>(p, grid, st);
        case 258: return go<16, 2>(p, grid, st);
        default: return set_error(VQK_ENOTIMPL, "no segment kernel for d=4 bits=%d gpb=%d", bits, gpb);
    }
}

}  // namespace vqk
