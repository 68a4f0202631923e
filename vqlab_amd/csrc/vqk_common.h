// Shared declarations of libvqk: vector types, activation conversions,
// geometry validation and error reporting. Written for gfx950 (CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "vqk.h"

namespace vqk {

typedef _Float16 f16;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;            // CDNA wavefront width
constexpr int kBlock = 32;           // codes per packing block
constexpr int kThreads = 256;        // threads per workgroup of the GEMV kernels
constexpr int kLdsBytes = 160 * 1024; // LDS a gfx950 workgroup may hold
constexpr int kCbLdsMax = 64 * 1024; // largest codebook table staged in LDS (bytes)
constexpr int kGemvHybBytes = 128 * 1024;  // part of a larger table the GEMV keeps in LDS
// Part of a larger table the GEMV keeps in LDS: less for the wide-x
// instances, whose fp32 activation row (up to 64 blocks of 1 KB) needs room.
__host__ __device__ constexpr int gemv_hyb_bytes(bool xf) { return xf ? kCbLdsMax : kGemvHybBytes; }

// Output forms of the weight dequant: fp16 (the bit-exact weight), bf16 (one
// RNE of it) or rows [W_hi | W_lo | W_hi] of 3 * IN bf16 with W_hi + W_lo = W.
enum : int { kDqF16 = 0, kDqBF16 = 1, kDqSplit = 2 };

// Operand types of the matrix-core GEMM of the dense prefill path.
enum : int { kOpF16 = 0, kOpBF16 = 1 };

// A GEMM launch plan: tile shape (index into the launcher's table), whole
// tiles before the split-K tail, K slices per tail tile (0: no tail) and the
// fp32 partials the tail needs.
struct GemmPlan {
    int shape;
    int32_t full, splits;
    size_t part_bytes;
};

// Plan of y = A . B^T with A [M, K], B [Nc, K] on the current device, using
// at most part_room bytes of split-K partials (vqk_hgemm.hip).
GemmPlan plan_gemm(int64_t M, int64_t Nc, int64_t K, size_t part_room);
int launch_hgemm(int op, const GemmPlan &plan, const uint16_t *A, const uint16_t *B, void *y,
                 int32_t y_type, int64_t ldy, int64_t ycol0, int64_t M, int64_t Nc, int64_t K,
                 float *part, hipStream_t st);

// A codebook table of 2^BITS entries of D halves is staged in LDS when it
// fits kCbLdsMax; larger tables are gathered from L2 / MALL.
__host__ __device__ constexpr bool cb_in_lds(int D, int BITS) {
    return (int64_t(1) << BITS) * D * 2 <= kCbLdsMax;
}

// ------------------------------------------------------------ host errors
int set_error(int code, const char *fmt, ...);
int hip_status(hipError_t e, const char *what);

// Validated geometry of one vqk_weights descriptor.
struct Geom {
    int64_t E, OUT, IN, K, NSUB, NB, NGRP, rows;  // rows = code rows stored
    int32_t D, G, BITS;      // BITS = pack_bits, or 8 / 16 for unpacked u8 / u16
    bool packed;
    int64_t row_words;       // u32 words per code row; 0 if rows are not word aligned
    int32_t gpb;             // scale groups per 32-code block (1 if a group spans >= 1 block)
    int32_t bpg;             // blocks per scale group when gpb == 1
    bool fast_ok;            // shape fits the block-per-lane kernels
};

// Validates `w` and fills `g`; returns a VQK_* status and sets the message.
int make_geom(const vqk_weights *w, Geom *g);

// Activation (x / y) element size in bytes for VQK_F16 / VQK_BF16 / VQK_F32.
int act_size(int32_t type);
// Output element size: act_size of an output type that may carry VQK_VIA_F16.
int out_size(int32_t type);

// ------------------------------------------------------ device conversions
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(uint32_t(b) << 16);
}

// Round to nearest even; NaN stays NaN (quieted).
// fp32 -> bf16, round to nearest even, NaN kept NaN with its top payload
// bits and the quiet bit set: gfx950's v_cvt_pk_bf16_f32 (what the compiler
// emits for this cast), which gives exactly the integer formulation
// ((u + 0x7fff + lsb) >> 16; NaN: (u >> 16) | 0x40) on every one of the 2^32
// inputs, denormals included (vqk__test_f32_to_bf16 and its GPU test check
// the special classes).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float h_to_f32(uint16_t h) {
    return float(__builtin_bit_cast(f16, h));
}

__device__ __forceinline__ uint16_t f32_to_h(float f) {
    return __builtin_bit_cast(uint16_t, f16(f));
}

// Element i of a table in global memory, read through the global address
// space: a global_load waits on the vector-memory counter only, where the
// flat_load a generic pointer (e.g. one taken from a parameter struct) gets
// also counts as an LDS access, so every LDS wait after it waits for it.
template <typename T>
__device__ __forceinline__ T load_global(const T *p, int64_t i) {
    return ((const __attribute__((address_space(1))) T *)p)[i];
}

__device__ __forceinline__ float load_act(const void *p, int32_t type, int64_t i) {
    if (type == VQK_F32) return static_cast<const float *>(p)[i];
    uint16_t v = static_cast<const uint16_t *>(p)[i];
    return type == VQK_BF16 ? bf16_to_f32(v) : h_to_f32(v);
}

__device__ __forceinline__ void store_act(void *p, int32_t type, int64_t i, float v) {
    if (type & VQK_VIA_F16) {                // round through fp16 first
        v = h_to_f32(f32_to_h(v));
        type &= ~VQK_VIA_F16;
    }
    if (type == VQK_F32) { static_cast<float *>(p)[i] = v; return; }
    static_cast<uint16_t *>(p)[i] = type == VQK_BF16 ? f32_to_bf16(v) : f32_to_h(v);
}

// ---------------------------------------------------------- wave reductions
// DPP (data-parallel primitives) move values between lanes inside the VALU,
// without the LDS crossbar round trip of ds_bpermute. Lanes whose source is
// masked off keep their own value (old operand = src).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL,
                                                      ROW_MASK, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

// Sum over aligned groups of `width` lanes (a power of two <= 64). The total
// is valid in the LAST lane of each group (every lane of it for width <= 16).
__device__ __forceinline__ float group_sum(float v, int width) {
    if (width >= 2) v += dpp_f<kDppQuadXor1>(v);
    if (width >= 4) v += dpp_f<kDppQuadXor2>(v);
    if (width >= 8) v += dpp_f<kDppRowHalfMirror>(v);
    if (width >= 16) v += dpp_f<kDppRowMirror>(v);
    if (width >= 32) v += dpp_f<kDppRowBcast15, 0xA>(v);
    if (width >= 64) v += dpp_f<kDppRowBcast31, 0xC>(v);
    return v;
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), CTRL, ROW_MASK, 0xf, false));
}

// Unsigned max over the whole wave, returned uniformly.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u<kDppQuadXor1>(v));
    v = max(v, dpp_u<kDppQuadXor2>(v));
    v = max(v, dpp_u<kDppRowHalfMirror>(v));
    v = max(v, dpp_u<kDppRowMirror>(v));
    v = max(v, dpp_u<kDppRowBcast15, 0xA>(v));
    v = max(v, dpp_u<kDppRowBcast31, 0xC>(v));
    return uint32_t(__builtin_amdgcn_readlane(int(v), kWave - 1));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_u<kDppQuadXor1>(v));
    v = min(v, dpp_u<kDppQuadXor2>(v));
    v = min(v, dpp_u<kDppRowHalfMirror>(v));
    v = min(v, dpp_u<kDppRowMirror>(v));
    v = min(v, dpp_u<kDppRowBcast15, 0xA>(v));
    v = min(v, dpp_u<kDppRowBcast31, 0xC>(v));
    return uint32_t(__builtin_amdgcn_readlane(int(v), kWave - 1));
}

// Order-preserving map float -> uint32 (NaN maps below every number, -0 to
// the key of +0, as they compare equal) and back.
// Written as selects (no branches: a routing wave maps its logits with it).
__device__ __forceinline__ uint32_t f32_key(float f) {
    const uint32_t b0 = __float_as_uint(f);
    const uint32_t b = b0 == 0x80000000u ? 0u : b0;
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (b0 & 0x7fffffffu) > 0x7f800000u ? 0u : k;      // NaN: never selected
}
__device__ __forceinline__ float key_f32(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Max / sum of one value per lane over the whole wave, returned uniformly.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppRowMirror>(v));
    v = fmaxf(v, dpp_f<kDppRowBcast15, 0xA>(v));
    v = fmaxf(v, dpp_f<kDppRowBcast31, 0xC>(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), kWave - 1));
}

__device__ __forceinline__ float wave_sum(float v) {
    v = group_sum(v, kWave);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), kWave - 1));
}

}  // namespace vqk
