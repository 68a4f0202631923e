/* CPU oracle, C restatement -- TEST INFRASTRUCTURE ONLY.
 *
 * A second, independent restatement of the bit-exact parts of the VQ decode
 * path (the numpy one is oracle/vq_oracle.py). Tests compare the two against
 * each other and against the reference's golden vectors; the product library
 * never links or calls this file.
 *
 * Reference anchors (relative to the reference checkout):
 *   vqo_pack / vqo_unpack      src/vqlab/runtime/vq_pack.py:48-97 (layout 11-27)
 *   vqo_f32_to_f16             IEEE 754 binary16, round to nearest even: the
 *                              single rounding of vq_switch.py:3447-3453
 *   vqo_dequant                vq_switch.py:3484-3492, vq_dense.py:132-137
 *   vqo_gemv_f32               gate/kernel_reference.py:10-23 (fp32 accumulate)
 *
 * fp16 conversion is written from the IEEE 754 definition (no compiler
 * _Float16 support is assumed: gcc 11 on x86 has none).
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

#define VQO_BLOCK 32

int vqo_words_per_row(int nsub, int bits) {
    return (nsub + VQO_BLOCK - 1) / VQO_BLOCK * bits;
}

/* codes: rows x nsub uint16 -> packed: rows x wpr uint32 (tail block zero). */
int vqo_pack(const uint16_t *codes, uint32_t *packed, int64_t rows, int nsub,
             int bits) {
    if (bits < 1 || bits > 16) return -1;
    const int wpr = vqo_words_per_row(nsub, bits);
    for (int64_t r = 0; r < rows; ++r) {
        uint32_t *prow = packed + r * wpr;
        memset(prow, 0, sizeof(uint32_t) * (size_t)wpr);
        for (int j = 0; j < nsub; ++j) {
            uint32_t c = codes[r * nsub + j];
            if (c >> bits) return -2;
            /* absolute bit of field j inside the row */
            int64_t pos = (int64_t)(j / VQO_BLOCK) * VQO_BLOCK * bits
                        + (int64_t)(j % VQO_BLOCK) * bits;
            uint64_t v = (uint64_t)c << (pos & 31);
            prow[pos >> 5] |= (uint32_t)v;
            if ((pos & 31) + bits > 32) prow[(pos >> 5) + 1] |= (uint32_t)(v >> 32);
        }
    }
    return 0;
}

/* packed rows -> uint16 codes (rows x nsub). */
int vqo_unpack(const uint32_t *packed, uint16_t *codes, int64_t rows, int nsub,
               int bits) {
    if (bits < 1 || bits > 16) return -1;
    const int wpr = vqo_words_per_row(nsub, bits);
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t r = 0; r < rows; ++r) {
        const uint32_t *prow = packed + r * wpr;
        for (int j = 0; j < nsub; ++j) {
            int64_t pos = (int64_t)(j / VQO_BLOCK) * VQO_BLOCK * bits
                        + (int64_t)(j % VQO_BLOCK) * bits;
            uint64_t lo = prow[pos >> 5];
            uint64_t hi = ((pos & 31) + bits > 32) ? prow[(pos >> 5) + 1] : 0;
            codes[r * nsub + j] = (uint16_t)(((lo | (hi << 32)) >> (pos & 31)) & mask);
        }
    }
    return 0;
}

float vqo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) { bits = sign; }
        else {                       /* subnormal: m * 2^-24 */
            float f = (float)m * (1.0f / 16777216.0f);
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t vqo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {                          /* inf or NaN */
        if (man == 0) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)(man >> 13);   /* quiet NaN */
    }
    if (exp == 0) return sign;                  /* f32 subnormal: < 2^-126 */
    int32_t E = exp - 127;                      /* unbiased exponent */
    uint32_t m = man | 0x800000u;               /* 24-bit significand */
    if (E > 15) return sign | 0x7c00u;          /* overflow */
    if (E >= -14) {                             /* normal half */
        uint32_t r = ((uint32_t)(E + 15) << 10) | (man >> 13);
        uint32_t rem = man & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1;  /* may carry to inf */
        return sign | (uint16_t)r;
    }
    /* subnormal half: value = m * 2^(E-23); unit 2^-24 -> q = m >> -(E+1) */
    int32_t shift = -(E + 1);                   /* >= 14 */
    if (shift >= 32) return sign;
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return sign | (uint16_t)q;
}

/* codes rows x nsub (uint16), cb K x d fp16 bits, scales rows x (nsub*d/G)
 * fp16 bits -> w rows x (nsub*d) fp16 bits. */
void vqo_dequant(const uint16_t *codes, const uint16_t *cb, int d,
                 const uint16_t *scales, int group, int64_t rows, int nsub,
                 uint16_t *w) {
    const int in = nsub * d, ngrp = in / group;
    for (int64_t r = 0; r < rows; ++r)
        for (int j = 0; j < nsub; ++j)
            for (int u = 0; u < d; ++u) {
                int col = j * d + u;
                float s = vqo_f16_to_f32(scales[r * ngrp + col / group]);
                float c = vqo_f16_to_f32(cb[(int64_t)codes[r * nsub + j] * d + u]);
                w[r * in + col] = vqo_f32_to_f16(s * c);
            }
}

/* y[n, r] = sum_i x[n, i] * W[r, i] with fp32 accumulation, W fp16 bits. */
void vqo_gemv_f32(const float *x, const uint16_t *w, int64_t n, int64_t out,
                  int64_t in, float *y) {
    for (int64_t t = 0; t < n; ++t)
        for (int64_t r = 0; r < out; ++r) {
            float acc = 0.0f;
            for (int64_t i = 0; i < in; ++i)
                acc += x[t * in + i] * vqo_f16_to_f32(w[r * in + i]);
            y[t * out + r] = acc;
        }
}

void vqo_f32_to_f16_array(const float *x, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = vqo_f32_to_f16(x[i]);
}
