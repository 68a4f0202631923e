// Fused VQ GEMV kernels: y[n, r] = sum_i x[n / xkrep, i] * W_e(n)[r, i], with
// W decoded on the fly from packed indices, codebook and per-group scales.
//
// Serves the decode regime of VQSwitchLinear (_fused, vq_switch.py:2919-3249,
// kernels such as the d4 device-codebook walk 925-990 and the d8 simd kernels
// 1424-1660) and VQLinear (_dense_fused, 3339-3434). Arithmetic per row, as in
// the reference: x is narrowed to fp16 (vq_switch.py:5306-5308; devx kernels
// 2371-2441), each code's subvector dot <cb[c], x> is accumulated in fp32 per
// scale group, and the group sum is scaled by its fp16 scale into an fp32
// accumulator (vq_switch.py:958-985). Summation order differs from the
// reference's serial walk (lane partials are added by a butterfly), which the
// output tolerance covers.
//
// Fast kernel layout (gfx950, wave64):
//   * one lane owns one 32-code packing block of a row: it loads the block's
//     BITS words (plus its scales) and decodes the 32 codes with shifts fixed
//     at compile time (BITS is a template parameter);
//   * LPR = next_pow2(NB) lanes cover a row, 64 / LPR rows per wave step;
//     a lane keeps the same block index for every row it visits, so its slice
//     of x (32*D fp16 values) is read from LDS once into registers;
//   * the codebook is staged into LDS as a 2^BITS-entry table when that fits
//     kCbLdsMax; a larger table keeps its first kGemvHybBytes in LDS and the
//     codes beyond it gather from L2 / MALL (clamped to K-1), which cuts the
//     L2 requests -- the rate that bounds such tables -- by that fraction;
//   * each wave issues the loads of its next row step before it decodes the
//     current one.
// Shapes outside the fast kernel's reach (ragged NSUB, rows not word
// aligned, NB > 64, unusual scale groups) run on the generic kernel: one
// thread per row, walking its codes.
//
// Wide-x instances (XF, d = 4 and 8, x_type flag VQK_X_KEEP): x is staged
// in LDS as fp32 -- bf16 and fp32 activations exactly -- and each table
// entry's halves are widened to fp32 and multiplied with fp32 FMAs, the
// arithmetic of the reference's float-staged kernels (the d4 `_SRC_FUSED`,
// vq_switch.py:106-150; the d8 ones at 153-237, 1316-1354, 1424-1660) that
// VQ_DECODE_BF16IO feeds bf16 x unrounded (vq_switch.py:4412-4417). Lanes
// read their block's activations from LDS per code (256 fp32 values per
// block would not fit in registers), and a table too large for LDS keeps
// only its first kCbLdsMax bytes there, leaving room for the fp32 row.
#pragma once

#include <mutex>
#include "vqk_common.h"

namespace vqk {

struct GemvParams {
    const void *codes;         // code rows (u32 words when packed)
    int64_t row_words;         // fast path: u32 words per code row
    int64_t code_cols;         // generic path: row stride in code units (words if packed)
    int32_t bits;              // packed width; 0 = unpacked (code_bytes 1 or 2)
    int32_t code_bytes;
    const uint16_t *codebook;  // fp16 [K, D]
    int32_t K;
    const uint16_t *scales;    // fp16, ngrp per code row
    int32_t ngrp, bpg, G;
    const int32_t *row_table;  // [E, OUT] or NULL
    int64_t stored_rows;       // code rows present (bound for device indices)
    const uint32_t *eidx;      // [N] expert per pair, NULL = expert 0
    int32_t E, OUT, IN, NSUB, NB;
    int32_t lpr_log2;          // lanes per row = 1 << lpr_log2
    const void *x;
    int32_t x_type;
    int64_t x_stride;          // elements between token rows
    int32_t pair0, xkrep;      // pair = pair0 + blockIdx.y, token = pair / xkrep
    void *y;
    int32_t y_type;
    int64_t y_stride;          // elements between pair rows of y
    int32_t rows_per_wg, steps;
};

// ---------------------------------------------------------------- helpers
template <int D>
__device__ __forceinline__ float dot_entry(const h2 *cb, uint32_t c, const h2 *x, float acc) {
    if constexpr (D == 2) {
        return __builtin_amdgcn_fdot2(cb[c], x[0], acc, false);
    } else if constexpr (D == 4) {
        const h4 e = reinterpret_cast<const h4 *>(cb)[c];
        acc = __builtin_amdgcn_fdot2(h2{e[0], e[1]}, x[0], acc, false);
        return __builtin_amdgcn_fdot2(h2{e[2], e[3]}, x[1], acc, false);
    } else {
        const h8 e = reinterpret_cast<const h8 *>(cb)[c];
        acc = __builtin_amdgcn_fdot2(h2{e[0], e[1]}, x[0], acc, false);
        acc = __builtin_amdgcn_fdot2(h2{e[2], e[3]}, x[1], acc, false);
        acc = __builtin_amdgcn_fdot2(h2{e[4], e[5]}, x[2], acc, false);
        return __builtin_amdgcn_fdot2(h2{e[6], e[7]}, x[3], acc, false);
    }
}

// Field i (compile-time after unrolling) of a 32-code block held in registers.
template <int BITS>
__device__ __forceinline__ uint32_t block_field(const uint32_t (&w)[BITS], int i) {
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    const int bit = i * BITS, wi = bit >> 5, sh = bit & 31;
    if (sh + BITS <= 32) return (w[wi] >> sh) & MASK;
    return __builtin_amdgcn_alignbit(w[wi + 1 < BITS ? wi + 1 : BITS - 1], w[wi], sh) & MASK;
}

// sum_g s[g] * sum_{codes i of group g} <cb[c_i], x_i> over one block.
template <int D, int BITS, int GPB, bool CBL>
__device__ __forceinline__ float block_dot(const uint32_t (&w)[BITS], const h2 (&xr)[16 * D],
                                           const float (&s)[GPB], const h2 *cb, uint32_t kmax) {
    constexpr int CPG = kBlock / GPB;
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < GPB; ++g) {
        float ga = 0.f;
#pragma unroll
        for (int q = 0; q < CPG; ++q) {
            const int i = g * CPG + q;
            uint32_t c = block_field<BITS>(w, i);
            if (!CBL) c = min(c, kmax);
            ga = dot_entry<D>(cb, c, &xr[i * (D / 2)], ga);
        }
        acc = fmaf(s[g], ga, acc);
    }
    return acc;
}

// One codebook entry (D halves) as a vector, and its dot with D x values.
template <int D> struct EntryT;
template <> struct EntryT<2> { typedef h2 type; };
template <> struct EntryT<4> { typedef h4 type; };
template <> struct EntryT<8> { typedef h8 type; };

template <int D>
__device__ __forceinline__ float dot_vec(typename EntryT<D>::type e, const h2 *x, float acc) {
    if constexpr (D == 2) {
        return __builtin_amdgcn_fdot2(e, x[0], acc, false);
    } else if constexpr (D == 4) {
        acc = __builtin_amdgcn_fdot2(h2{e[0], e[1]}, x[0], acc, false);
        return __builtin_amdgcn_fdot2(h2{e[2], e[3]}, x[1], acc, false);
    } else {
        acc = __builtin_amdgcn_fdot2(h2{e[0], e[1]}, x[0], acc, false);
        acc = __builtin_amdgcn_fdot2(h2{e[2], e[3]}, x[1], acc, false);
        acc = __builtin_amdgcn_fdot2(h2{e[4], e[5]}, x[2], acc, false);
        return __builtin_amdgcn_fdot2(h2{e[6], e[7]}, x[3], acc, false);
    }
}

// block_dot for a table only partly in LDS: entries below `kl` are read from
// the LDS copy `cbl`, the rest from the global table `cbg` (clamped to kmax).
// The two reads run under complementary lane masks into the same registers,
// so each code costs one read and one set of dot products, and the L2 sees
// requests only for the codes beyond the LDS part.
template <int D, int BITS, int GPB>
__device__ __forceinline__ float block_dot_hyb(const uint32_t (&w)[BITS], const h2 (&xr)[16 * D],
                                               const float (&s)[GPB], const h2 *cbl, const h2 *cbg,
                                               uint32_t kl, uint32_t kmax) {
    typedef typename EntryT<D>::type E;
    constexpr int CPG = kBlock / GPB;
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < GPB; ++g) {
        float ga = 0.f;
#pragma unroll
        for (int q = 0; q < CPG; ++q) {
            const int i = g * CPG + q;
            const uint32_t c = block_field<BITS>(w, i);
            // exec-masked reads (measured 3 % faster here than the
            // branch-free pair the segment kernels use)
            E e;
            if (c < kl) e = reinterpret_cast<const E *>(cbl)[c];
            else e = reinterpret_cast<const E *>(cbg)[min(c, kmax)];
            ga = dot_vec<D>(e, &xr[i * (D / 2)], ga);
        }
        acc = fmaf(s[g], ga, acc);
    }
    return acc;
}

// block_dot with the table in LDS and all 32 entry reads issued before the
// first product: at one wave per SIMD nothing else hides their latency.
template <int D, int BITS, int GPB>
__device__ __forceinline__ float block_dot_all(const uint32_t (&w)[BITS], const h2 (&xr)[16 * D],
                                               const float (&s)[GPB], const h2 *cb) {
    typedef typename EntryT<D>::type E;
    constexpr int CPG = kBlock / GPB;
    E e[kBlock];
#pragma unroll
    for (int i = 0; i < kBlock; ++i) e[i] = reinterpret_cast<const E *>(cb)[block_field<BITS>(w, i)];
    __builtin_amdgcn_sched_barrier(0);
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < GPB; ++g) {
        float ga = 0.f;
#pragma unroll
        for (int q = 0; q < CPG; ++q) {
            const int i = g * CPG + q;
            ga = dot_vec<D>(e[i], &xr[i * (D / 2)], ga);
        }
        acc = fmaf(s[g], ga, acc);
    }
    return acc;
}

// block_dot with the table in LDS and the block's 32·D activations read from
// LDS (`xl`) per code instead of held in 16·D registers (d8: 128 registers a
// wave of an 8-wave workgroup cannot spare).
template <int D, int BITS, int GPB>
__device__ __forceinline__ float block_dot_lx(const uint32_t (&w)[BITS], const f16 *xl,
                                              const float (&s)[GPB], const h2 *cb) {
    typedef typename EntryT<D>::type E;
    constexpr int CPG = kBlock / GPB;
    const E *xv = reinterpret_cast<const E *>(__builtin_assume_aligned(xl, 16));
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < GPB; ++g) {
        float ga = 0.f;
#pragma unroll
        for (int q = 0; q < CPG; ++q) {
            const int i = g * CPG + q;
            const E e = reinterpret_cast<const E *>(cb)[block_field<BITS>(w, i)];
            const E x = xv[i];
            h2 xh[D / 2];
#pragma unroll
            for (int k = 0; k < D / 2; ++k) xh[k] = h2{x[2 * k], x[2 * k + 1]};
            ga = dot_vec<D>(e, xh, ga);
        }
        acc = fmaf(s[g], ga, acc);
    }
    return acc;
}

// block_dot_hyb with the block's 32·D activations read from LDS (`xl`) per
// code instead of held in 16·D registers: the registers that frees let two
// waves share a SIMD, each hiding the other's table-read latency.
template <int D, int BITS, int GPB>
__device__ __forceinline__ float block_dot_hyb_lx(const uint32_t (&w)[BITS], const f16 *xl,
                                                  const float (&s)[GPB], const h2 *cbl,
                                                  const h2 *cbg, uint32_t kl, uint32_t kmax) {
    typedef typename EntryT<D>::type E;
    constexpr int CPG = kBlock / GPB;
    const E *xv = reinterpret_cast<const E *>(__builtin_assume_aligned(xl, 16));
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < GPB; ++g) {
        float ga = 0.f;
#pragma unroll
        for (int q = 0; q < CPG; ++q) {
            const int i = g * CPG + q;
            const uint32_t c = block_field<BITS>(w, i);
            E e;
            if (c < kl) e = reinterpret_cast<const E *>(cbl)[c];
            else e = reinterpret_cast<const E *>(cbg)[min(c, kmax)];
            const E x = xv[i];
            h2 xh[D / 2];
#pragma unroll
            for (int k = 0; k < D / 2; ++k) xh[k] = h2{x[2 * k], x[2 * k + 1]};
            ga = dot_vec<D>(e, xh, ga);
        }
        acc = fmaf(s[g], ga, acc);
    }
    return acc;
}

// block_dot of the wide-x instances: the block's 32·D activations as fp32 in
// LDS (`xl`), every entry half widened exactly to fp32. CBL: the whole table
// is in `cbl`; otherwise entries below `kl` come from `cbl`, the rest from
// the global table `cbg` (clamped to kmax).
template <int D, int BITS, int GPB, bool CBL>
__device__ __forceinline__ float block_dot_xf(const uint32_t (&w)[BITS], const float *xl,
                                              const float (&s)[GPB], const h2 *cbl,
                                              const h2 *cbg, uint32_t kl, uint32_t kmax) {
    typedef typename EntryT<D>::type E;
    constexpr int CPG = kBlock / GPB;
    const f32x4 *xv = reinterpret_cast<const f32x4 *>(__builtin_assume_aligned(xl, 16));
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < GPB; ++g) {
        float ga = 0.f;
#pragma unroll
        for (int q = 0; q < CPG; ++q) {
            const int i = g * CPG + q;
            const uint32_t c = block_field<BITS>(w, i);
            E e;
            if constexpr (CBL) {
                e = reinterpret_cast<const E *>(cbl)[c];
            } else {
                if (c < kl) e = reinterpret_cast<const E *>(cbl)[c];
                else e = reinterpret_cast<const E *>(cbg)[min(c, kmax)];
            }
#pragma unroll
            for (int k = 0; k < D / 4; ++k) {
                const f32x4 x = xv[i * (D / 4) + k];
                ga = fmaf(float(e[4 * k]), x.x, ga);
                ga = fmaf(float(e[4 * k + 1]), x.y, ga);
                ga = fmaf(float(e[4 * k + 2]), x.z, ga);
                ga = fmaf(float(e[4 * k + 3]), x.w, ga);
            }
        }
        acc = fmaf(s[g], ga, acc);
    }
    return acc;
}

template <int BITS, int GPB>
__device__ __forceinline__ void load_block(const GemvParams &p, int64_t cr, int blk, int sidx,
                                           uint32_t (&w)[BITS], uint32_t (&s)[GPB]) {
    if (cr >= 0) {
        // streaming loads: config 1 ran 5.86 us per call with them, 6.33 us
        // with plain loads (the fused layer's blocks take plain loads)
        const uint32_t *src = static_cast<const uint32_t *>(p.codes) + cr * p.row_words +
                              int64_t(blk) * BITS;
#pragma unroll
        for (int i = 0; i < BITS; ++i) w[i] = __builtin_nontemporal_load(src + i);
        const uint16_t *sr = p.scales + cr * p.ngrp + sidx;
#pragma unroll
        for (int g = 0; g < GPB; ++g) s[g] = __builtin_nontemporal_load(sr + g);
    } else {
#pragma unroll
        for (int i = 0; i < BITS; ++i) w[i] = 0u;
#pragma unroll
        for (int g = 0; g < GPB; ++g) s[g] = 0u;
    }
}

// Raw fp16 scale bits (as loaded) -> fp32, at their use: converting them in
// the load helper would be the loads' first use and put a wait right behind
// them, serialising the wave's next loads (table copy, next projection).
template <int GPB>
struct ScalesF32 {
    float v[GPB];
    __device__ __forceinline__ explicit ScalesF32(const uint32_t (&r)[GPB]) {
#pragma unroll
        for (int g = 0; g < GPB; ++g) v[g] = h_to_f32(uint16_t(r[g]));
    }
};

typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

// Asynchronous global -> LDS copy of `bytes` (a multiple of 4; src and dst
// 16-byte aligned), then zero-fill up to `total` bytes. The 16-byte pieces go
// through global_load_lds_dwordx4: each wave instruction moves 1 KB straight
// into LDS without passing through VGPRs, so a 32 KB codebook costs one
// memory latency. The caller waits (vmcnt 0) and barriers before reading.
__device__ __forceinline__ void lds_copy_async(const void *src, void *dst, int bytes, int total) {
    const uint8_t *s = static_cast<const uint8_t *>(src);
    uint8_t *d = static_cast<uint8_t *>(dst);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int n16 = bytes >> 4;
    for (int c = wave * kWave; c < n16; c += nw * kWave) {    // c: first piece of a 1 KB chunk
        if (c + lane < n16)
            __builtin_amdgcn_global_load_lds((global_void *)(s + int64_t(c + lane) * 16),
                                             (lds_void *)(d + int64_t(c) * 16), 16, 0, 0);
    }
    for (int i = n16 * 4 + threadIdx.x; i < total / 4; i += blockDim.x)
        reinterpret_cast<uint32_t *>(d)[i] =
            i < bytes / 4 ? reinterpret_cast<const uint32_t *>(s)[i] : 0u;
}

// Codebook -> LDS table of `entries` (>= K) rows of D halves, zero beyond K.
template <int D>
__device__ __forceinline__ void stage_codebook(const uint16_t *cb, int K, int entries, h2 *dst) {
    lds_copy_async(cb, dst, K * D * 2, entries * D * 2);
}

// Same for a table of compile-time size CBN entries staged by the NT threads
// of waves W0 .. W0 + NT/64 - 1: every one of them issues at most
// ceil(CBN*D*2 / (16 * NT)) direct-to-LDS loads (predicated off past K), and
// no global load sits in a loop.
template <int D, int CBN, int NT, int W0 = 0>
__device__ __forceinline__ void stage_codebook_fixed(const uint16_t *cb, int K, h2 *dst) {
    constexpr int PIECES = CBN * D * 2 / 16;                 // 16-byte pieces of the table
    constexpr int ROUNDS = (PIECES + NT - 1) / NT;
    const uint8_t *s = reinterpret_cast<const uint8_t *>(cb);
    uint8_t *d = reinterpret_cast<uint8_t *>(dst);
    const int lane = threadIdx.x & (kWave - 1), wave = int(threadIdx.x >> 6) - W0;
    // whole pieces to copy: all of a table that fits, the first CBN entries
    // of a larger one (ROUNDS * NT may exceed PIECES: never copy past it)
    const int valid = min((K * D * 2) >> 4, PIECES);
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
        const int c = (r * (NT / kWave) + wave) * kWave;     // first piece of this wave's chunk
        if (c + lane < valid)
            __builtin_amdgcn_global_load_lds((global_void *)(s + int64_t(c + lane) * 16),
                                             (lds_void *)(d + int64_t(c) * 16), 16, 0, 0);
    }
    if (valid == PIECES) return;                             // the LDS table is full
    // the sub-16-byte tail of the valid bytes (at most 3 words, one load per
    // thread), then zeros up to the table end
    const int tail_words = ((K * D * 2) >> 2) - valid * 4;
    const int tid = int(threadIdx.x) - W0 * kWave;
    if (tid < tail_words)
        reinterpret_cast<uint32_t *>(d)[valid * 4 + tid] =
            reinterpret_cast<const uint32_t *>(s)[valid * 4 + tid];
    for (int i = valid * 4 + tail_words + tid; i < PIECES * 4; i += NT)
        reinterpret_cast<uint32_t *>(d)[i] = 0u;
}

// Wait for every outstanding vector-memory operation of this wave (the
// asynchronous LDS copies included).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0); }

// Wait until at most N vector-memory operations of this wave are outstanding
// (gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt
// left at their maxima, i.e. not waited for).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Eight activations starting at element i of row `base` -> fp16, as one
// 16-byte value. 16-byte aligned rows only (checked by the caller).
__device__ __forceinline__ u32x4 load8_act(const void *x, int32_t type, int64_t i) {
    if (type == VQK_F32) {
        const u32x4 a = *reinterpret_cast<const u32x4 *>(static_cast<const float *>(x) + i);
        const u32x4 b = *reinterpret_cast<const u32x4 *>(static_cast<const float *>(x) + i + 4);
        u32x4 r;
        r.x = uint32_t(f32_to_h(__uint_as_float(a.x))) | (uint32_t(f32_to_h(__uint_as_float(a.y))) << 16);
        r.y = uint32_t(f32_to_h(__uint_as_float(a.z))) | (uint32_t(f32_to_h(__uint_as_float(a.w))) << 16);
        r.z = uint32_t(f32_to_h(__uint_as_float(b.x))) | (uint32_t(f32_to_h(__uint_as_float(b.y))) << 16);
        r.w = uint32_t(f32_to_h(__uint_as_float(b.z))) | (uint32_t(f32_to_h(__uint_as_float(b.w))) << 16);
        return r;
    }
    u32x4 v = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(x) + i);
    if (type == VQK_BF16) {
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w[k] = uint32_t(f32_to_h(bf16_to_f32(uint16_t(w[k])))) |
                   (uint32_t(f32_to_h(bf16_to_f32(uint16_t(w[k] >> 16)))) << 16);
        v = u32x4{w[0], w[1], w[2], w[3]};
    }
    return v;
}

// One activation row -> fp16 in LDS, blocks of XH values at a padded stride
// XS (halves). Vector path: every thread issues all its 16-byte loads before
// converting any, so the row costs one memory latency.
// Eight fp16 values fp16(silu(g) * u) of fp32 gate / up rows (the SwiGLU
// product the fused layer writes), packed as four words; 32-byte aligned.
__device__ __forceinline__ u32x4 swiglu8(const float *g, const float *u) {
    const u32x4 g0 = reinterpret_cast<const u32x4 *>(g)[0], g1 = reinterpret_cast<const u32x4 *>(g)[1];
    const u32x4 u0 = reinterpret_cast<const u32x4 *>(u)[0], u1 = reinterpret_cast<const u32x4 *>(u)[1];
    const uint32_t gw[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const uint32_t uw[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float gv = __uint_as_float(gw[i]);
        h[i] = f32_to_h(gv / (1.f + __expf(-gv)) * __uint_as_float(uw[i]));
    }
    return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

// `tid0` / `nthr`: the staging threads' first index and count (default: the
// whole workgroup).
template <int XH, int XS>
__device__ __forceinline__ void stage_x(const void *x, int32_t type, int64_t base, int IN, int NB,
                                        f16 *xs, int tid0 = -1, int nthr = 0) {
    const int me = tid0 < 0 ? int(threadIdx.x) : int(threadIdx.x) - tid0;
    const int nt = tid0 < 0 ? int(blockDim.x) : nthr;
    const int esz = type == VQK_F32 ? 4 : 2;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) + uint64_t(base) * esz) & 15) == 0 &&
                     (IN & 7) == 0;
    if (vec) {
        constexpr int U = 4;
        const int ng = NB * XH / 8;                      // 8-value groups incl. zero tail
        for (int g0 = me; g0 < ng; g0 += U * nt) {
            u32x4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int g = g0 + u * nt;
                v[u] = (g < ng && g * 8 < IN) ? load8_act(x, type, base + g * 8) : u32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int g = g0 + u * nt;
                if (g < ng) {
                    const int i = g * 8;
                    *reinterpret_cast<u32x4 *>(xs + (i / XH) * XS + (i % XH)) = v[u];
                }
            }
        }
        return;
    }
    for (int i = me; i < NB * XH; i += nt) {
        const float v = i < IN ? load_act(x, type, base + i) : 0.f;
        xs[(i / XH) * XS + (i % XH)] = f16(v);
    }
}

// Eight activations starting at element i -> fp32, exactly (16-byte aligned
// rows only, checked by the caller).
__device__ __forceinline__ void load8_f32(const void *x, int32_t type, int64_t i, float (&v)[8]) {
    if (type == VQK_F32) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(x) + i);
        const f32x4 b = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(x) + i + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        return;
    }
    const u32x4 u = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(x) + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint16_t lo = uint16_t(w[k]), hi = uint16_t(w[k] >> 16);
        v[2 * k] = type == VQK_BF16 ? bf16_to_f32(lo) : h_to_f32(lo);
        v[2 * k + 1] = type == VQK_BF16 ? bf16_to_f32(hi) : h_to_f32(hi);
    }
}

// One activation row -> fp32 in LDS (the wide-x instances), blocks of XH
// values at a padded stride XS (floats), zero past IN; the loads of a
// thread's groups are all issued before the first store, as in stage_x.
template <int XH, int XS>
__device__ __forceinline__ void stage_xf(const void *x, int32_t type, int64_t base, int IN, int NB,
                                         float *xs) {
    static_assert(XH % 8 == 0 && XS % 4 == 0, "8-value groups stay inside a 16-byte aligned block");
    const int me = threadIdx.x, nt = blockDim.x;
    const int esz = type == VQK_F32 ? 4 : 2;
    const bool vec = ((reinterpret_cast<uintptr_t>(x) + uint64_t(base) * esz) & 15) == 0 &&
                     (IN & 7) == 0;
    if (vec) {
        constexpr int U = 2;
        const int ng = NB * XH / 8;
        for (int g0 = me; g0 < ng; g0 += U * nt) {
            float v[U][8];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int g = g0 + u * nt;
                if (g < ng && g * 8 < IN) {
                    load8_f32(x, type, base + g * 8, v[u]);
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[u][k] = 0.f;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int g = g0 + u * nt;
                if (g < ng) {
                    const int i = g * 8;
                    f32x4 *d = reinterpret_cast<f32x4 *>(xs + (i / XH) * XS + (i % XH));
                    d[0] = f32x4{v[u][0], v[u][1], v[u][2], v[u][3]};
                    d[1] = f32x4{v[u][4], v[u][5], v[u][6], v[u][7]};
                }
            }
        }
        return;
    }
    for (int i = me; i < NB * XH; i += nt)
        xs[(i / XH) * XS + (i % XH)] = i < IN ? load_act(x, type, base + i) : 0.f;
}

// The lane's 32*D staged activations -> 16*D half2 registers. Read as plain
// 32-bit words (the compiler merges them into 128-bit LDS reads):
// bit-casting elements of a u32x4 value miscompiled, every element read as
// element 0.
template <int D>
// `src` is 16-byte aligned at every call (block strides are multiples of 16
// bytes), which lets the reads go out as 16-byte LDS loads: half the
// instructions of 8-byte pairs, and the padded stride keeps them free of
// bank conflicts.
__device__ __forceinline__ void load_xregs(const f16 *src, h2 (&xr)[16 * D]) {
    const uint32_t *s = static_cast<const uint32_t *>(__builtin_assume_aligned(src, 16));
#pragma unroll
    for (int j = 0; j < 16 * D; ++j) xr[j] = __builtin_bit_cast(h2, s[j]);
}

// ------------------------------------------------------------ fast kernel
template <int D, int BITS, int GPB, bool XF = false>
__global__ void __launch_bounds__(kThreads) k_gemv_fast(const GemvParams p) {
    constexpr bool CBL = cb_in_lds(D, BITS);
    // LDS table entries: the whole table, or the first part of it
    constexpr int CBN = CBL ? (1 << BITS) : gemv_hyb_bytes(XF) / (2 * D);
    constexpr int XH = kBlock * D;               // x values per block
    constexpr int XS = XH + (XF ? 4 : 8);        // padded LDS stride: 16 B skew per block
    extern __shared__ __align__(16) uint8_t smem[];
    h2 *cb_lds = reinterpret_cast<h2 *>(smem);
    f16 *xs = reinterpret_cast<f16 *>(smem + CBN * D * 2);
    float *xsf = reinterpret_cast<float *>(smem + CBN * D * 2);

    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
    const int lpr = 1 << p.lpr_log2, rpw = kWave >> p.lpr_log2;
    const int sub = lane >> p.lpr_log2, blk = lane & (lpr - 1);
    const bool on = blk < p.NB;
    const int pair = p.pair0 + int(blockIdx.y);
    const int tok = pair / p.xkrep;
    const uint32_t e = p.eidx ? p.eidx[pair] : 0u;
    const bool e_ok = e < uint32_t(p.E);
    const int r_wg = int(blockIdx.x) * p.rows_per_wg;
    const int sidx = GPB == 1 ? blk / p.bpg : blk * GPB;

    auto row_at = [&](int st) { return r_wg + (st * 4 + wave) * rpw + sub; };
    auto code_row = [&](int st) -> int64_t {
        const int r = row_at(st);
        if (!on || !e_ok || r >= p.OUT) return -1;
        int64_t f = int64_t(e) * p.OUT + r;
        if (p.row_table) f = p.row_table[f];
        return f < p.stored_rows ? f : -1;
    };

    uint32_t w[BITS];
    uint32_t s[GPB];
    int64_t cr = code_row(0);
    load_block<BITS, GPB>(p, cr, blk, sidx, w, s);   // in flight during staging

    stage_codebook_fixed<D, CBN, kThreads>(p.codebook, p.K, cb_lds);
    if constexpr (XF) stage_xf<XH, XS>(p.x, p.x_type, int64_t(tok) * p.x_stride, p.IN, p.NB, xsf);
    else stage_x<XH, XS>(p.x, p.x_type, int64_t(tok) * p.x_stride, p.IN, p.NB, xs);
    wait_vmem();
    __syncthreads();

    h2 xr[16 * D];
    if constexpr (!XF) load_xregs<D>(xs + (on ? blk : 0) * XS, xr);
    const float *xl = xsf + (on ? blk : 0) * XS;
    const h2 *cb = CBL ? cb_lds : reinterpret_cast<const h2 *>(p.codebook);
    const uint32_t kmax = uint32_t(p.K - 1);
    const uint32_t kl = uint32_t(min(p.K, CBN));

    for (int st = 0; st < p.steps; ++st) {
        uint32_t wn[BITS];
        uint32_t sn[GPB];
        const int64_t crn = st + 1 < p.steps ? code_row(st + 1) : -1;
        load_block<BITS, GPB>(p, crn, blk, sidx, wn, sn);
        float v = 0.f;
        const ScalesF32<GPB> fs(s);
        if constexpr (XF) {
            if (cr >= 0)
                v = block_dot_xf<D, BITS, GPB, CBL>(w, xl, fs.v, cb_lds,
                                                    reinterpret_cast<const h2 *>(p.codebook), kl, kmax);
        } else if constexpr (CBL) {
            if (cr >= 0) v = block_dot<D, BITS, GPB, true>(w, xr, fs.v, cb, kmax);
        } else {
            if (cr >= 0) v = block_dot_hyb<D, BITS, GPB>(w, xr, fs.v, cb_lds, cb, kl, kmax);
        }
        v = group_sum(v, lpr);
        const int r = row_at(st);
        if (blk == lpr - 1 && r < p.OUT) store_act(p.y, p.y_type, int64_t(pair) * p.y_stride + r, v);
        cr = crn;
#pragma unroll
        for (int i = 0; i < BITS; ++i) w[i] = wn[i];
#pragma unroll
        for (int g = 0; g < GPB; ++g) s[g] = sn[g];
    }
}

// --------------------------------------------------------- generic kernel
__device__ __forceinline__ uint32_t generic_code(const GemvParams &p, int64_t cr, int j) {
    if (p.bits) {
        const uint32_t *row = static_cast<const uint32_t *>(p.codes) + cr * p.code_cols;
        const int64_t bit = int64_t(j >> 5) * (int64_t(kBlock) * p.bits) + (j & 31) * p.bits;
        const int sh = int(bit & 31);
        uint32_t v = row[bit >> 5] >> sh;
        if (sh + p.bits > 32) v |= row[(bit >> 5) + 1] << (32 - sh);
        return v & ((1u << p.bits) - 1u);
    }
    if (p.code_bytes == 1) return static_cast<const uint8_t *>(p.codes)[cr * p.code_cols + j];
    return static_cast<const uint16_t *>(p.codes)[cr * p.code_cols + j];
}

// One thread per (pair, row); x row staged once per workgroup as plain fp16
// (XF: as fp32, the wide-x arithmetic).
template <int D, bool XF = false>
__global__ void __launch_bounds__(kThreads) k_gemv_generic(const GemvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    f16 *xs = reinterpret_cast<f16 *>(smem);
    float *xsf = reinterpret_cast<float *>(smem);
    const int pair = p.pair0 + int(blockIdx.y);
    const int tok = pair / p.xkrep;
    for (int i = threadIdx.x; i < p.IN; i += blockDim.x) {
        const float v = load_act(p.x, p.x_type, int64_t(tok) * p.x_stride + i);
        if constexpr (XF) xsf[i] = v;
        else xs[i] = f16(v);
    }
    __syncthreads();
    const int r = int(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= p.OUT) return;
    const uint32_t e = p.eidx ? p.eidx[pair] : 0u;
    int64_t cr = -1;
    if (e < uint32_t(p.E)) {
        cr = int64_t(e) * p.OUT + r;
        if (p.row_table) cr = p.row_table[cr];
        if (cr >= p.stored_rows) cr = -1;
    }
    float acc = 0.f;
    if (cr >= 0) {
        const uint16_t *srow = p.scales + cr * p.ngrp;
        float ga = 0.f;
        int gcur = 0;
        for (int j = 0; j < p.NSUB; ++j) {
            const int g = (j * D) / p.G;
            if (g != gcur) {
                acc = fmaf(h_to_f32(srow[gcur]), ga, acc);
                ga = 0.f;
                gcur = g;
            }
            const uint32_t c = min(generic_code(p, cr, j), uint32_t(p.K - 1));
            const uint16_t *ce = p.codebook + int64_t(c) * D;
#pragma unroll
            for (int u = 0; u < D; ++u)
                ga = fmaf(h_to_f32(ce[u]), XF ? xsf[j * D + u] : float(xs[j * D + u]), ga);
        }
        acc = fmaf(h_to_f32(srow[gcur]), ga, acc);
    }
    store_act(p.y, p.y_type, int64_t(pair) * p.y_stride + r, acc);
}

// Per-D launchers of the fast kernel (one translation unit per D).
int launch_gemv_fast_d2(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st);
int launch_gemv_fast_d4(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st);
int launch_gemv_fast_d8(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st);
int launch_gemv_fast_d8x(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st);
int launch_gemv_fast_d4x(const GemvParams &p, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st);
bool gemv_fast_d4x_has(int bits);   // a fast wide-x d=4 instance exists for this width

// Launch helper: raises each kernel instance's dynamic-LDS cap as its launches need more.
template <auto KERN, typename P>
int launch_with_lds(dim3 grid, dim3 block, size_t smem, hipStream_t st, const P &p) {
    // the kernel's dynamic-LDS limit only ever rises, so a later launch asking
    // for more than an earlier one is covered
    static std::mutex mu;
    static size_t raised_to = 64 * 1024;
    if (smem > 64 * 1024) {
        std::lock_guard<std::mutex> lk(mu);
        if (smem > raised_to) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(KERN),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, int(smem));
            if (e != hipSuccess) return hip_status(e, "hipFuncSetAttribute");
            raised_to = smem;
        }
    }
    hipLaunchKernelGGL(KERN, grid, block, smem, st, p);
    return hip_status(hipGetLastError(), "kernel launch");
}

}  // namespace vqk
