// k_seg_mfma instances for d = 8: every packed width 2..16 (8 / 16 also
// serve unpacked uint8 / uint16 rows) x the scale-group layouts of the GEMV;
// k_seg_persist for the widths whose table is beyond LDS.
#include "vqk_gseg.h"

namespace vqk {

namespace {
template <int BITS, int GPB>
int go(const SegParams &p, dim3 grid, hipStream_t st) {
    constexpr bool CBL = cb_in_lds(8, BITS);
    return launch_with_lds<k_seg_mfma<8, BITS, GPB, CBL>>(grid, dim3(kSegWaves * 64), seg_lds(8, BITS, CBL), st, p);
}
// the sort's tiles hold up to 4 or up to 8 rows (its choice, read by the
// kernel): LDS for the larger of the two layouts
template <int BITS, int GPB>
int go_persist(const SegParams &p, dim3 grid, hipStream_t st) {
    constexpr size_t a = seg_lds(8, BITS, false, kSegTokNarrow), b = seg_lds(8, BITS, false, kSegTokMid);
    return launch_with_lds<k_seg_persist<BITS, GPB>>(grid, dim3(kPersistWaves * 64), a > b ? a : b,
                                                     st, p);
}
}  // namespace

int launch_seg_persist_d8(const SegParams &p, int bits, int gpb, dim3 grid, hipStream_t st) {
    switch (bits * 16 + gpb) {
        case 209: return go_persist<13, 1>(p, grid, st);
        case 212: return go_persist<13, 4>(p, grid, st);
        case 225: return go_persist<14, 1>(p, grid, st);
        case 228: return go_persist<14, 4>(p, grid, st);
        case 241: return go_persist<15, 1>(p, grid, st);
        case 244: return go_persist<15, 4>(p, grid, st);
        case 257: return go_persist<16, 1>(p, grid, st);
        case 260: return go_persist<16, 4>(p, grid, st);
        default:
            return set_error(VQK_ENOTIMPL, "no persistent segment kernel for d=8 bits=%d gpb=%d",
                             bits, gpb);
    }
}

// Tiles of at most 16 rows (dense rows or a 16-row sort); narrow sorts run
// the persistent kernel (launch_seg_persist_d8).
int launch_seg_d8(const SegParams &p, int bits, int gpb, int tok, dim3 grid, hipStream_t st) {
    if (tok != kSegTok) return set_error(VQK_EINVAL, "segment kernel tiles of %d rows", tok);
    switch (bits * 16 + gpb) {
        case 33: return go<2, 1>(p, grid, st);
        case 36: return go<2, 4>(p, grid, st);
        case 49: return go<3, 1>(p, grid, st);
        case 52: return go<3, 4>(p, grid, st);
        case 65: return go<4, 1>(p, grid, st);
        case 68: return go<4, 4>(p, grid, st);
        case 81: return go<5, 1>(p, grid, st);
        case 84: return go<5, 4>(p, grid, st);
        case 97: return go<6, 1>(p, grid, st);
        case 100: return go<6, 4>(p, grid, st);
        case 113: return go<7, 1>(p, grid, st);
        case 116: return go<7, 4>(p, grid, st);
        case 129: return go<8, 1>(p, grid, st);
        case 132: return go<8, 4>(p, grid, st);
        case 145: return go<9, 1>(p, grid, st);
        case 148: return go<9, 4>(p, grid, st);
        case 161: return go<10, 1>(p, grid, st);
        case 164: return go<10, 4>(p, grid, st);
        case 177: return go<11, 1>(p, grid, st);
        case 180: return go<11, 4>(p, grid, st);
        case 193: return go<12, 1>(p, grid, st);
        case 196: return go<12, 4>(p, grid, st);
        case 209: return go<13, 1>(p, grid, st);
        case 212: return go<13, 4>(p, grid, st);
        case 225: return go<14, 1>(p, grid, st);
        case 228: return go<14, 4>(p, grid, st);
        case 241: return go<15, 1>(p, grid, st);
        case 244: return go<15, 4>(p, grid, st);
        case 257: return go<16, 1>(p, grid, st);
        case 260: return go<16, 4>(p, grid, st);
        default: return set_error(VQK_ENOTIMPL, "no segment kernel for d=8 bits=%d gpb=%d", bits, gpb);
    }
}

}  // namespace vqk
