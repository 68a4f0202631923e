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

constexpr int kWave = 64;            // CDNA wavefront width
constexpr int kBlock = 32;           // codes per packing block
constexpr int kThreads = 256;        // threads per workgroup of the GEMV kernels
constexpr int kCbLdsMax = 64 * 1024; // largest codebook table staged in LDS (bytes)

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

// ------------------------------------------------------ device conversions
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(uint32_t(b) << 16);
}

// Round to nearest even; NaN stays NaN (quieted).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

__device__ __forceinline__ float h_to_f32(uint16_t h) {
    return float(__builtin_bit_cast(f16, h));
}

__device__ __forceinline__ uint16_t f32_to_h(float f) {
    return __builtin_bit_cast(uint16_t, f16(f));
}

__device__ __forceinline__ float load_act(const void *p, int32_t type, int64_t i) {
    if (type == VQK_F32) return static_cast<const float *>(p)[i];
    uint16_t v = static_cast<const uint16_t *>(p)[i];
    return type == VQK_BF16 ? bf16_to_f32(v) : h_to_f32(v);
}

__device__ __forceinline__ void store_act(void *p, int32_t type, int64_t i, float v) {
    if (type == VQK_F32) { static_cast<float *>(p)[i] = v; return; }
    static_cast<uint16_t *>(p)[i] = type == VQK_BF16 ? f32_to_bf16(v) : f32_to_h(v);
}

// Butterfly sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

}  // namespace vqk
