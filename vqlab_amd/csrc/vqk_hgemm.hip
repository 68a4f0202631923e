// fp16 matrix-core GEMM for the dense prefill path, after the weight has been
// dequantised (bit-exactly) into a workspace panel:
//     y[m, c0 + n] = sum_k A[m, k] * B[n, k]      A = x as fp16 [M, K],
//                                                  B = W panel fp16 [Nc, K]
// Both operands are K-contiguous, which is what v_mfma_f32_32x32x16_f16
// reads per lane (8 consecutive k of one row), so neither is transposed.
//
// Workgroup tile BM x BN x BK with WGM x WGN waves, each wave owning a
// (BM / WGM) x (BN / WGN) block of 32x32 MFMA tiles with fp32 accumulators.
// Tiles of A and B are copied global -> LDS by global_load_lds_dwordx4 (no
// VGPR round trip) into NST stages: the copies of the next NST - 1 k steps
// are in flight while one multiplies.
// An LDS row is BK halves = BK / 8 slots of 16 bytes; slot s of row r is
// stored at slot s ^ swz(r), so the rows one read phase touches at one
// logical slot hit distinct 4-bank groups. The direct-to-LDS copy writes
// consecutive slots per lane, so the swizzle is applied to the GLOBAL
// address each lane fetches.
// Workgroups are numbered so that the 8 XCDs (workgroups are dealt to them
// round-robin) each own a contiguous band of B panels and sweep all row
// tiles of A for each: a B panel is fetched into one XCD's L2 once.
#include "vqk_common.h"
#include "vqk_gemv.h"

namespace vqk {

typedef float f32x16 __attribute__((ext_vector_type(16)));

struct HgemmParams {
    const uint16_t *A;    // [M, K] fp16
    const uint16_t *B;    // [Nc, K] fp16
    void *y;
    int32_t y_type;
    int64_t ldy;          // elements between rows of y
    int64_t ycol0;        // column of y that B's row 0 lands in
    int32_t M, Nc, K;
    int32_t tiles_m, tiles_n;
};

template <int BM, int BN, int WGM, int WGN, int BK, int NST>
__global__ void __launch_bounds__(64 * WGM * WGN) k_hgemm(const HgemmParams p) {
    constexpr int NW = WGM * WGN;                  // waves: WGM along M x WGN along N
    constexpr int WTM = BM / WGM, WTN = BN / WGN;  // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int RB = BK * 2;                     // bytes per LDS row
    constexpr int SLOTS = RB / 16;                 // 16-byte slots per row
    constexpr int RPI = 1024 / RB;                 // rows per 1 KB wave copy
    constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB;
    constexpr int A_INS = A_BYTES / 1024, B_INS = B_BYTES / 1024;   // 1 KB wave copies
    constexpr int NSL = BK / 16;                   // 16-k slices per step
    static_assert(A_INS % NW == 0 && B_INS % NW == 0, "copies must split over the waves");
    static_assert(TM >= 1 && TN >= 1, "wave tile below one 32x32 MFMA tile");
    static_assert(NST >= 3, "the pipeline keeps two stages in flight");
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    // slot swizzle: the 16 (BK 64) or 32 (BK 32) rows an LDS read phase touches
    // at one logical slot land on distinct 4-bank groups
    auto swz = [](int r) { return SLOTS == 8 ? ((r >> 1) & 7) : ((r >> 2) & (SLOTS - 1)); };

    // XCD-aware tile order: workgroup b runs on XCD b % 8
    const int T = p.tiles_m * p.tiles_n;
    int t = int(blockIdx.x);
    if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;
    const int bm = t % p.tiles_m, bn = t / p.tiles_m;
    const int m0 = bm * BM, n0 = bn * BN;

    // per-lane global sources of this wave's copies (row r of a tile, swizzled slot)
    const int crow = lane / SLOTS, cslot = lane % SLOTS;
    const uint16_t *asrc[A_INS / NW];
    const uint16_t *bsrc[B_INS / NW];
#pragma unroll
    for (int j = 0; j < A_INS / NW; ++j) {
        const int r = (wave * (A_INS / NW) + j) * RPI + crow;
        const int gr = min(m0 + r, p.M - 1);
        asrc[j] = p.A + int64_t(gr) * p.K + 8 * (cslot ^ swz(r));
    }
#pragma unroll
    for (int j = 0; j < B_INS / NW; ++j) {
        const int r = (wave * (B_INS / NW) + j) * RPI + crow;
        const int gr = min(n0 + r, p.Nc - 1);
        bsrc[j] = p.B + int64_t(gr) * p.K + 8 * (cslot ^ swz(r));
    }
    constexpr int STAGE = A_BYTES + B_BYTES;
    auto issue = [&](int kt, int buf) {
        uint8_t *abase = smem + buf * STAGE;
        uint8_t *bbase = abase + A_BYTES;
        const int k0 = kt * BK;
#pragma unroll
        for (int j = 0; j < A_INS / NW; ++j)
            __builtin_amdgcn_global_load_lds((global_void *)(asrc[j] + k0),
                                             (lds_void *)(abase + (wave * (A_INS / NW) + j) * 1024),
                                             16, 0, 0);
#pragma unroll
        for (int j = 0; j < B_INS / NW; ++j)
            __builtin_amdgcn_global_load_lds((global_void *)(bsrc[j] + k0),
                                             (lds_void *)(bbase + (wave * (B_INS / NW) + j) * 1024),
                                             16, 0, 0);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x16{};

    // Software pipeline over NST LDS stages (NST - 1 copies in flight), with
    // the operand fragments read one 16-wide k slice ahead of the MFMAs that
    // use them (two register sets). In step k: slices 0..NSL-2 multiply while
    // slices 1..NSL-1 are read; then this wave waits for its stage-(k+1)
    // copies, one barrier makes stage k+1 visible and retires every wave's
    // reads of stage k-1's buffer, the copy of stage k+NST-1 goes into it, and
    // the last slice multiplies while slice 0 of step k+1 is read. A wave's
    // copies complete in issue order, so "at most (NST-3) stages' copies
    // outstanding" means stage k+1 has landed.
    constexpr int PER_STAGE = A_INS / NW + B_INS / NW;
    const int KT = p.K / BK;
    const int lr = lane & 31, lk = lane >> 5;
    auto frags = [&](int stage, int kk, h8 (&af)[TM], h8 (&bf)[TN]) {
        const uint8_t *abase = smem + stage * STAGE;
        const uint8_t *bbase = abase + A_BYTES;
        const int slot = 2 * kk + lk;
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int r = wm * WTM + a * 32 + lr;
            af[a] = *reinterpret_cast<const h8 *>(abase + r * RB + ((slot ^ swz(r)) << 4));
        }
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int r = wn * WTN + b * 32 + lr;
            bf[b] = *reinterpret_cast<const h8 *>(bbase + r * RB + ((slot ^ swz(r)) << 4));
        }
    };
    auto mma = [&](const h8 (&af)[TM], const h8 (&bf)[TN]) {
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
    };
    h8 f0a[TM], f0b[TN], f1a[TM], f1b[TN];
#pragma unroll
    for (int s = 0; s < NST - 1; ++s)
        if (s < KT) issue(s, s);
    if (KT >= NST - 1) wait_vmcnt<(NST - 2) * PER_STAGE>();
    else wait_vmem();
    __builtin_amdgcn_s_barrier();
    frags(0, 0, f0a, f0b);
    for (int kt = 0; kt < KT; ++kt) {
        const int cs = kt % NST;
#pragma unroll
        for (int kk = 1; kk < NSL; ++kk) {
            if (kk & 1) { frags(cs, kk, f1a, f1b); mma(f0a, f0b); }
            else { frags(cs, kk, f0a, f0b); mma(f1a, f1b); }
        }
        if (kt + NST - 2 < KT) wait_vmcnt<(NST - 3) * PER_STAGE>();
        else wait_vmem();
        __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): the last slice of stage k read
        __builtin_amdgcn_s_barrier();
        if (kt + NST - 1 < KT) issue(kt + NST - 1, (kt + NST - 1) % NST);
        static_assert(NSL % 2 == 0, "an even slice count ends on the second register set");
        frags((kt + 1) % NST, 0, f0a, f0b);         // past the last step: unused
        mma(f1a, f1b);
    }
    wait_vmem();

    // C register i of lane l: row 8*(i/4) + 4*(l/32) + i%4, column l%32
#pragma unroll
    for (int a = 0; a < TM; ++a) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = m0 + wm * WTM + a * 32 + (i / 4) * 8 + lk * 4 + (i % 4);
            if (m >= p.M) continue;
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int n = n0 + wn * WTN + b * 32 + lr;
                if (n < p.Nc) store_act(p.y, p.y_type, int64_t(m) * p.ldy + p.ycol0 + n, acc[a][b][i]);
            }
        }
    }
}

// x (any activation type) -> fp16 [N, IN], 8 elements per thread.
__global__ void k_x_to_f16(const void *x, int32_t type, int64_t n8, uint16_t *out) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    *reinterpret_cast<u32x4 *>(out + i * 8) = load8_act(x, type, i * 8);
}

// Tile shapes, measured on MI355X at the dense prefill shapes (M = 2048,
// 5120 x 17408 and 17408 x 5120): 256 x 256 with 8 waves (4 x 2, wave tile
// 64 x 128) and 32-wide k steps in four stages (128 KB of LDS) for large
// outputs -- each operand byte staged feeds twice the MFMA work of a 128-wide
// tile; 128 x 128 with 4 waves and 64-wide steps in three stages otherwise,
// whose 4x more tiles fill the GPU when the output is narrow.
template <int BM, int BN, int WGM, int WGN, int BK, int NST>
static int go_hgemm(HgemmParams p, hipStream_t st) {
    p.tiles_m = int32_t((p.M + BM - 1) / BM);
    p.tiles_n = int32_t((p.Nc + BN - 1) / BN);
    const int64_t T = int64_t(p.tiles_m) * p.tiles_n;
    if (T > INT32_MAX) return set_error(VQK_ENOTIMPL, "GEMM grid too large");
    const size_t lds = size_t(NST) * (BM + BN) * BK * 2;
    return launch_with_lds<k_hgemm<BM, BN, WGM, WGN, BK, NST>>(dim3(unsigned(T)), dim3(64 * WGM * WGN),
                                                              lds, st, p);
}

// y[:, c0 : c0 + Nc] = A . B^T; A [M, K], B [Nc, K] fp16, K % 64 == 0,
// both 16-byte aligned.
int launch_hgemm(const uint16_t *A, const uint16_t *B, void *y, int32_t y_type, int64_t ldy,
                 int64_t ycol0, int64_t M, int64_t Nc, int64_t K, hipStream_t st) {
    HgemmParams p;
    p.A = A;
    p.B = B;
    p.y = y;
    p.y_type = y_type;
    p.ldy = ldy;
    p.ycol0 = ycol0;
    p.M = int32_t(M);
    p.Nc = int32_t(Nc);
    p.K = int32_t(K);
    if (M >= 1024 && Nc >= 1024) return go_hgemm<256, 256, 4, 2, 32, 4>(p, st);
    return go_hgemm<128, 128, 2, 2, 64, 3>(p, st);
}

int launch_x_to_f16(const void *x, int32_t type, int64_t n, uint16_t *out, hipStream_t st) {
    const int64_t n8 = n / 8;
    if (n8 == 0) return VQK_OK;
    hipLaunchKernelGGL(k_x_to_f16, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0, st, x, type,
                       n8, out);
    return hip_status(hipGetLastError(), "x conversion launch");
}

}  // namespace vqk
