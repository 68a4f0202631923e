// Matrix-core GEMM of the dense prefill path, after the weight has been
// dequantised (bit-exactly) into a workspace panel:
//     y[m, c0 + n] = sum_k A[m, k] * B[n, k]      A = x [M, K],
//                                                  B = W panel [Nc, K]
// in fp16 or bf16 operands (OP) with fp32 accumulation, the reference's
// `xf @ w.T.astype(xf.dtype)` (vq_dense.py:288, 294). Both operands are
// K-contiguous, which is what v_mfma_f32_32x32x16_{f16,bf16} reads per lane
// (8 consecutive k of one row), so neither is transposed.
//
// Workgroup tile BM x BN x BK with WGM x WGN waves, each wave owning a
// (BM / WGM) x (BN / WGN) block of 32x32 MFMA tiles with fp32 accumulators.
// A stage of both operand tiles is CH 1 KB chunks (64 lanes x 16 bytes),
// copied global -> LDS by global_load_lds_dwordx4 (no VGPR round trip) and
// dealt to the waves in contiguous runs of CPW; when CH is not a multiple of
// the wave count the last wave repeats the final chunk (same bytes to the
// same place). NST stages: the copies of the next NST - 2 k steps are in
// flight while one multiplies.
// An LDS row is BK elements = BK / 8 slots of 16 bytes; slot s of row r is
// stored at slot s ^ swz(r), so the 16 rows one ds_read_b128 phase touches
// at one logical slot fall on distinct 16-byte bank groups (64 banks). The
// direct-to-LDS copy writes consecutive slots per lane, so the swizzle is
// applied to the GLOBAL address each lane fetches.
// Workgroups are numbered so that the 8 XCDs (workgroups are dealt to them
// round-robin) each own a contiguous band of tiles, row tiles of A fastest:
// a B panel is fetched into one XCD's L2 once.
#pragma once

#include <type_traits>

#include "vqk_common.h"
#include "vqk_gemv.h"

namespace vqk {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));


template <int OP> struct HgemmOp;
template <> struct HgemmOp<kOpF16> {
    typedef h8 frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct HgemmOp<kOpBF16> {
    typedef bf8 frag;
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

struct HgemmParams {
    const uint16_t *A;    // [M, K] fp16 / bf16
    const uint16_t *B;    // [Nc, K] same type
    void *y;
    int32_t y_type;
    int64_t ldy;          // elements between rows of y
    int64_t ycol0;        // column of y that B's row 0 lands in
    int32_t M, Nc, K;
    int32_t tiles_m, tiles_n;
    // split-K tail (ping-pong kernel only): workgroups [0, full) run whole
    // tiles 0 .. full-1; each later workgroup u = b - full runs K slice u % splits
    // of tile full + u / splits into its own fp32 partial part[u] (BM * BN
    // floats in register order), summed by k_gemm_reduce. splits = 0: none.
    int32_t full, splits;
    float *part;
};

template <int OP, int BM, int BN, int WGM, int WGN, int BK, int NST>
__global__ void __launch_bounds__(64 * WGM * WGN) k_hgemm(const HgemmParams p) {
    using Op = HgemmOp<OP>;
    using frag = typename Op::frag;
    constexpr int NW = WGM * WGN;                  // waves: WGM along M x WGN along N
    constexpr int WTM = BM / WGM, WTN = BN / WGN;  // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int RB = BK * 2;                     // bytes per LDS row
    constexpr int SLOTS = RB / 16;                 // 16-byte slots per row
    constexpr int RPI = 1024 / RB;                 // rows per 1 KB chunk
    constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB;
    constexpr int A_INS = A_BYTES / 1024, B_INS = B_BYTES / 1024;
    constexpr int CH = A_INS + B_INS;              // 1 KB chunks per stage
    constexpr int CPW = (CH + NW - 1) / NW;        // chunks per wave
    constexpr int NSL = BK / 16;                   // 16-k slices per step
    static_assert(BM % RPI == 0 && BN % RPI == 0, "tiles are whole chunks");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && TM >= 1 && TN >= 1,
                  "wave tile is whole 32x32 MFMA tiles");
    static_assert(NST >= 3, "the pipeline keeps two stages in flight");
    static_assert(SLOTS == 4 || SLOTS == 8, "BK is 32 or 64");
    static_assert(NSL % 2 == 0, "an even slice count ends on the second register set");
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    auto swz = [](int r) { return SLOTS == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3); };

    // XCD-aware tile order: workgroup b runs on XCD b % 8
    const int T = p.tiles_m * p.tiles_n;
    int t = int(blockIdx.x);
    if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;
    const int bm = t % p.tiles_m, bn = t / p.tiles_m;
    const int m0 = bm * BM, n0 = bn * BN;

    // this wave's chunks: per-lane global source (row clamped into the
    // operand, slot swizzled) and LDS offset within a stage
    const int crow = lane / SLOTS, cslot = lane % SLOTS;
    const uint16_t *src[CPW];
    int dst[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        const int c = min(wave * CPW + j, CH - 1);
        const bool isa = c < A_INS;
        const int r = (isa ? c : c - A_INS) * RPI + crow;
        const int gr = isa ? min(m0 + r, p.M - 1) : min(n0 + r, p.Nc - 1);
        src[j] = (isa ? p.A : p.B) + int64_t(gr) * p.K + 8 * (cslot ^ swz(r));
        dst[j] = c * 1024;
    }
    constexpr int STAGE = A_BYTES + B_BYTES;
    auto issue = [&](int kt, int buf) {
        uint8_t *base = smem + buf * STAGE;
        const int k0 = kt * BK;
#pragma unroll
        for (int j = 0; j < CPW; ++j)
            __builtin_amdgcn_global_load_lds((global_void *)(src[j] + k0), (lds_void *)(base + dst[j]),
                                             16, 0, 0);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x16{};

    // Software pipeline over NST LDS stages, with the operand fragments read
    // one 16-wide k slice ahead of the MFMAs that use them (two register
    // sets). In step k: slices 0..NSL-2 multiply while slices 1..NSL-1 are
    // read; then this wave waits for its stage-(k+1) copies, one barrier makes
    // stage k+1 visible and retires every wave's reads of stage k-1's buffer,
    // the copy of stage k+NST-1 goes into it, and the last slice multiplies
    // while slice 0 of step k+1 is read. A wave's copies complete in issue
    // order, so "at most (NST-3) stages' copies outstanding" means stage k+1
    // has landed. Steps past the end copy the last stage again into a buffer
    // nobody reads any more, so every step issues the same copies, the waits
    // are the same constants and the loop body is one scheduling region, in
    // which each fragment read and each copy is paired with an MFMA.
    const int KT = p.K / BK;
    const int lr = lane & 31, lk = lane >> 5;
    auto frags = [&](int stage, int kk, frag (&af)[TM], frag (&bf)[TN]) {
        const uint8_t *abase = smem + stage * STAGE;
        const uint8_t *bbase = abase + A_BYTES;
        const int slot = 2 * kk + lk;
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int r = wm * WTM + a * 32 + lr;
            af[a] = *reinterpret_cast<const frag *>(abase + r * RB + ((slot ^ swz(r)) << 4));
        }
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int r = wn * WTN + b * 32 + lr;
            bf[b] = *reinterpret_cast<const frag *>(bbase + r * RB + ((slot ^ swz(r)) << 4));
        }
    };
    auto mma = [&](const frag (&af)[TM], const frag (&bf)[TN]) {
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) acc[a][b] = Op::mma(af[a], bf[b], acc[a][b]);
    };
    constexpr int NR = TM + TN, NM = TM * TN;   // fragment reads and MFMAs per slice
    // scheduling groups: one MFMA, then one of `mask` (0x100 LDS read, 0x020
    // global read), n times; the rest of the slice's MFMAs after them
    auto pair_with_mfma = [](auto mask_c, auto n_c) {
        constexpr int mask = decltype(mask_c)::value, n = decltype(n_c)::value;
#pragma unroll
        for (int i = 0; i < n; ++i) {
            if (i < NM) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(mask, 1, 0);
        }
        if (NM > n) __builtin_amdgcn_sched_group_barrier(0x008, NM > n ? NM - n : 0, 0);
    };
    using ic = std::integral_constant<int, 0x100>;
    frag f0a[TM], f0b[TN], f1a[TM], f1b[TN];
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(min(s, KT - 1), s);
    wait_vmcnt<(NST - 2) * CPW>();
    __builtin_amdgcn_s_barrier();
    frags(0, 0, f0a, f0b);
    for (int kt = 0; kt < KT; ++kt) {
        const int cs = kt % NST;
#pragma unroll
        for (int kk = 1; kk < NSL; ++kk) {
            if (kk & 1) { frags(cs, kk, f1a, f1b); mma(f0a, f0b); }
            else { frags(cs, kk, f0a, f0b); mma(f1a, f1b); }
            pair_with_mfma(ic{}, std::integral_constant<int, NR>{});
        }
        wait_vmcnt<(NST - 3) * CPW>();
        __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): the last slice of stage k read
        __builtin_amdgcn_s_barrier();
        issue(min(kt + NST - 1, KT - 1), (kt + NST - 1) % NST);
        frags((kt + 1) % NST, 0, f0a, f0b);         // past the last step: unused
        mma(f1a, f1b);
        pair_with_mfma(std::integral_constant<int, 0x020>{}, std::integral_constant<int, CPW>{});
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

}  // namespace vqk

namespace vqk {

// Ping-pong variant: 8 waves in two groups of four (waves 0-3 and 4-7; wave
// w runs on SIMD w % 4, so every SIMD holds one wave of each group). The
// waves form a WGM x WGN grid over the tile; group g owns grid columns
// [g * WGN / 2, (g + 1) * WGN / 2) when WGN is even, else grid rows
// [g * WGM / 2, ...). A group alternates two phases: LOAD (read every
// fragment of one BK stage from LDS into registers and issue its half of
// the chunks of a later stage) and MMA (all of that stage's MFMAs back to
// back). Group 1 starts one phase late, so on every SIMD one wave issues
// MFMAs while the other loads, and the barrier that ends each phase never
// drains the matrix pipe.
//   phase 2k   : group 0 LOAD stage k,  group 1 MMA stage k-1
//   phase 2k+1 : group 0 MMA stage k,   group 1 LOAD stage k
// Stage k + NST - 1 goes into the buffer of stage k - 1, whose last reads
// (group 1, phase 2k-1) completed before the barrier that ends that phase.
// Stage k + 1 must be visible at phase 2k+2: group 0 waits for its copies at
// the end of its MMA phase 2k+1, group 1 at the end of its LOAD phase 2k+1.
template <int OP, int BM, int BN, int WGM, int WGN, int BK, int NST>
__global__ void __launch_bounds__(512) k_pgemm(const HgemmParams p) {
    using Op = HgemmOp<OP>;
    using frag = typename Op::frag;
    static_assert(WGM * WGN == 8, "eight waves");
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int RB = BK * 2, SLOTS = RB / 16, RPI = 1024 / RB;
    constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB;
    constexpr int A_INS = A_BYTES / 1024, B_INS = B_BYTES / 1024;
    constexpr int CH = A_INS + B_INS;              // 1 KB chunks per stage
    constexpr int CHG = (CH + 1) / 2;              // chunks of group 0 (group 1: the rest)
    constexpr int CPW = (CHG + 3) / 4;             // chunks per wave
    constexpr int NSL = BK / 16;
    constexpr int STAGE = A_BYTES + B_BYTES;
    static_assert(BM % RPI == 0 && BN % RPI == 0, "tiles are whole chunks");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && TM >= 1 && TN >= 1, "whole MFMA tiles");
    static_assert(NST >= 3 && (SLOTS == 4 || SLOTS == 8), "stages / BK");
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = wave >> 2, wg = wave & 3;
    // grid position: group g takes half the columns (WGN even) or half the rows
    int wm, wn;
    if constexpr (WGN % 2 == 0) { wm = wg % WGM; wn = grp * (WGN / 2) + wg / WGM; }
    else { wm = grp * (WGM / 2) + wg / WGN; wn = wg % WGN; }
    auto swz = [](int r) { return SLOTS == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3); };

    // whole tiles in XCD-aware order (workgroup b runs on XCD b % 8), then
    // the split-K units of the remaining tiles
    const int KTA = p.K / BK;                      // k steps of the whole operand
    int t = int(blockIdx.x), k_lo = 0, k_hi = KTA, unit = -1;
    const int F = p.splits ? p.full : p.tiles_m * p.tiles_n;
    if (t < F) {
        if (F % 8 == 0) t = (t % 8) * (F / 8) + t / 8;
    } else {
        unit = t - F;
        t = F + unit / p.splits;
        const int per = (KTA + p.splits - 1) / p.splits;
        k_lo = min(KTA, (unit % p.splits) * per);
        k_hi = min(KTA, k_lo + per);
    }
    const int bm = t % p.tiles_m, bn = t / p.tiles_m;
    const int m0 = bm * BM, n0 = bn * BN;
    if (k_hi <= k_lo) {                            // an empty K slice (the host avoids them)
        float *dstp = p.part + int64_t(unit) * BM * BN;
        for (int e = int(threadIdx.x); e < BM * BN; e += 512) dstp[e] = 0.f;
        return;
    }

    // this wave's chunks (group 0: chunks [0, CHG), group 1: [CHG, CH); a
    // wave past its group's last chunk repeats it)
    const int crow = lane / SLOTS, cslot = lane % SLOTS;
    const int c_lo = grp ? CHG : 0, c_hi = grp ? CH - 1 : CHG - 1;
    const uint16_t *src[CPW];
    int dst[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        const int c = min(c_lo + wg * CPW + j, c_hi);
        const bool isa = c < A_INS;
        const int r = (isa ? c : c - A_INS) * RPI + crow;
        const int gr = isa ? min(m0 + r, p.M - 1) : min(n0 + r, p.Nc - 1);
        src[j] = (isa ? p.A : p.B) + int64_t(gr) * p.K + int64_t(k_lo) * BK + 8 * (cslot ^ swz(r));
        dst[j] = c * 1024;
    }
    const int KT = k_hi - k_lo;                    // k steps of this workgroup (>= 0)
    auto issue = [&](int kt, int buf) {
        uint8_t *base = smem + buf * STAGE;
        const int k0 = max(0, min(kt, KT - 1)) * BK;   // past the end: a copy nobody reads
#pragma unroll
        for (int j = 0; j < CPW; ++j)
            __builtin_amdgcn_global_load_lds((global_void *)(src[j] + k0), (lds_void *)(base + dst[j]),
                                             16, 0, 0);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x16{};

    const int lr = lane & 31, lk = lane >> 5;
    frag fa[NSL][TM], fb[NSL][TN];
    auto load_phase = [&](int kt) {              // every fragment of stage kt
        const uint8_t *abase = smem + (kt % NST) * STAGE;
        const uint8_t *bbase = abase + A_BYTES;
#pragma unroll
        for (int kk = 0; kk < NSL; ++kk) {
            const int slot = 2 * kk + lk;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int r = wm * WTM + a * 32 + lr;
                fa[kk][a] = *reinterpret_cast<const frag *>(abase + r * RB + ((slot ^ swz(r)) << 4));
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int r = wn * WTN + b * 32 + lr;
                fb[kk][b] = *reinterpret_cast<const frag *>(bbase + r * RB + ((slot ^ swz(r)) << 4));
            }
        }
        issue(kt + NST - 1, (kt + NST - 1) % NST);
    };
    auto mma_phase = [&]() {
#pragma unroll
        for (int kk = 0; kk < NSL; ++kk)
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b) acc[a][b] = Op::mma(fa[kk][a], fb[kk][b], acc[a][b]);
    };

#pragma unroll
    for (int s = 0; s < NST - 1; ++s) issue(s, s);
    wait_vmcnt<(NST - 2) * CPW>();                 // this wave's part of stage 0
    __builtin_amdgcn_s_barrier();
    if (grp) __builtin_amdgcn_s_barrier();         // group 1 runs one phase behind
    for (int kt = 0; kt < KT; ++kt) {
        load_phase(kt);
        if (grp) wait_vmcnt<(NST - 2) * CPW>();    // group 1: its part of stage kt+1
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): fragments in registers
        __builtin_amdgcn_s_barrier();
        mma_phase();
        if (!grp) wait_vmcnt<(NST - 2) * CPW>();   // group 0: its part of stage kt+1
        __builtin_amdgcn_s_barrier();
    }
    if (!grp) __builtin_amdgcn_s_barrier();        // pairs group 1's last barrier
    wait_vmem();

    if (unit >= 0) {
        // fp32 partial in register order: element ((((wave*TM + a)*TN + b)*16 + i)*64 + lane)
        float *dstp = p.part + int64_t(unit) * BM * BN;
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    dstp[(((wave * TM + a) * TN + b) * 16 + i) * 64 + lane] = acc[a][b][i];
        return;
    }
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

// Sum of the split-K partials of tile p.full + blockIdx.y in split order (a
// fixed order: the result does not depend on which workgroup finished
// first), stored like k_pgemm's epilogue. Four consecutive elements of the
// register order per thread: four consecutive columns of one row.
template <int BM, int BN, int WGM, int WGN>
__global__ void __launch_bounds__(256) k_gemm_reduce(const HgemmParams p) {
    constexpr int WTM = BM / WGM, WTN = BN / WGN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    const int e = (int(blockIdx.x) * 256 + int(threadIdx.x)) * 4;
    if (e >= BM * BN) return;
    const int tile = p.full + int(blockIdx.y);
    const float *src = p.part + int64_t(blockIdx.y) * p.splits * BM * BN + e;
    float4 v = *reinterpret_cast<const float4 *>(src);
    for (int s = 1; s < p.splits; ++s) {
        const float4 w = *reinterpret_cast<const float4 *>(src + int64_t(s) * BM * BN);
        v.x += w.x; v.y += w.y; v.z += w.z; v.w += w.w;
    }
    const int lane = e % 64, i = (e / 64) % 16, b = (e / 1024) % TN, a = (e / (1024 * TN)) % TM;
    const int wave = e / (1024 * TN * TM);
    const int grp = wave >> 2, wg = wave & 3;
    int wm, wn;
    if constexpr (WGN % 2 == 0) { wm = wg % WGM; wn = grp * (WGN / 2) + wg / WGM; }
    else { wm = grp * (WGM / 2) + wg / WGN; wn = wg % WGN; }
    const int bm = tile % p.tiles_m, bn = tile / p.tiles_m;
    const int m = bm * BM + wm * WTM + a * 32 + (i / 4) * 8 + (lane >> 5) * 4 + (i % 4);
    const int n = bn * BN + wn * WTN + b * 32 + (lane & 31);
    if (m >= p.M) return;
    const float r[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (n + u < p.Nc) store_act(p.y, p.y_type, int64_t(m) * p.ldy + p.ycol0 + n + u, r[u]);
}

}  // namespace vqk
