// Gather-only decode of VQ-coded embedding tables: VQEmbedding
// (vq_dense.py:444-513) and VQPLEEmbedding (vq_switch.py:5426-5495).
//
//     out[i, j] = out_type( fp16( f32(cb[c(ids[i], j / D)][j % D]) * f32(s[ids[i], j / G]) ) )
//
// Only the gathered rows are decoded, in one launch: a lane produces 8
// consecutive outputs of one row, so a row of IN values is IN / 8 lanes and
// the stores of a wave cover 64 consecutive 16-byte chunks (fp16 / bf16
// output) or 32-byte chunks (fp32). Lookups are tiny (a few rows per token):
// the kernel is bound by one memory latency, not by bandwidth, so it favours
// a single launch and no staging over LDS tables.
//
// Code layouts (per table row):
//   unpacked      uint8 / uint16 [NSUB]
//   block-packed  uint32 words, 32-code blocks of `bits` words (vq_pack.py:11-27)
//   byte stream   uint8 [row_bytes]: code j at bits [j*bits, (j+1)*bits) of the
//                 row, LSB first -- the PLE shard format, read through a
//                 3-byte window at byte (j*bits)/8 (vq_switch.py:5449-5470)
#include "vqk_common.h"
#include "vqk_gemv.h"

namespace vqk {

enum EmbedLayout : int32_t { kEmbU8 = 0, kEmbU16 = 1, kEmbBlocks = 2, kEmbStream = 3 };

struct EmbedArgs {
    const void *codes;
    int64_t code_cols;       // elements of the codes array per row
    int32_t layout, bits;
    const uint16_t *codebook;
    int64_t K;
    int32_t D, G;
    const uint16_t *scales;
    int64_t ngrp;
    int64_t rows;            // table rows (valid ids are [0, rows))
    int64_t IN;
    const void *ids;
    int32_t id64;
    int64_t n;               // ids
    void *out;
    int32_t out_type;
    int32_t vec_ok;          // out is 16-byte aligned and IN % 8 == 0: whole-chunk stores
    int64_t lanes_per_row;   // ceil(IN / 8)
};

__device__ __forceinline__ uint32_t embed_code(const EmbedArgs &a, int64_t row, int64_t c) {
    const uint32_t mask = a.bits >= 32 ? 0xffffffffu : ((1u << a.bits) - 1u);
    switch (a.layout) {
        case kEmbU8:
            return static_cast<const uint8_t *>(a.codes)[row * a.code_cols + c];
        case kEmbU16:
            return static_cast<const uint16_t *>(a.codes)[row * a.code_cols + c];
        case kEmbBlocks: {
            const uint32_t *wr = static_cast<const uint32_t *>(a.codes) + row * a.code_cols +
                                 (c / kBlock) * a.bits;
            const int bit = int(c % kBlock) * a.bits;
            const int w = bit >> 5, sh = bit & 31;
            uint64_t v = wr[w];
            if (sh + a.bits > 32) v |= uint64_t(wr[w + 1]) << 32;   // straddles two words
            return uint32_t(v >> sh) & mask;
        }
        default: {
            const uint8_t *br = static_cast<const uint8_t *>(a.codes) + row * a.code_cols;
            const int64_t bit = c * a.bits, b = bit >> 3;
            uint32_t win = br[b];
            if (b + 1 < a.code_cols) win |= uint32_t(br[b + 1]) << 8;
            if (b + 2 < a.code_cols) win |= uint32_t(br[b + 2]) << 16;
            return (win >> (bit & 7)) & mask;
        }
    }
}

__device__ __forceinline__ uint16_t h_to_bf16(uint16_t h) {
    return f32_to_bf16(h_to_f32(h));   // fp16 -> f32 is exact; one RNE to bf16
}

__global__ void __launch_bounds__(256) k_embed_gather(const EmbedArgs a) {
    const int64_t total = a.n * a.lanes_per_row;
    for (int64_t it = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; it < total;
         it += int64_t(gridDim.x) * blockDim.x) {
        const int64_t i = it / a.lanes_per_row;
        const int64_t j0 = (it % a.lanes_per_row) * 8;
        const int64_t id = a.id64 ? static_cast<const int64_t *>(a.ids)[i]
                                  : int64_t(static_cast<const int32_t *>(a.ids)[i]);
        const bool ok = id >= 0 && id < a.rows;
        uint16_t h[8];
        int64_t cached = -1;
        uint32_t code = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int64_t j = j0 + t;
            h[t] = 0;
            if (!ok || j >= a.IN) continue;   // ids outside the table give rows of +0
            const int64_t c = j / a.D;
            if (c != cached) {
                code = embed_code(a, id, c);
                if (code >= uint32_t(a.K)) code = uint32_t(a.K - 1);   // never read past the table
                cached = c;
            }
            const float s = h_to_f32(a.scales[id * a.ngrp + j / a.G]);
            h[t] = f32_to_h(h_to_f32(a.codebook[int64_t(code) * a.D + (j - c * a.D)]) * s);
        }
        const int64_t o = i * a.IN + j0;
        const bool whole = a.vec_ok != 0;   // chunk is whole and 16/32-byte aligned
        if (a.out_type == VQK_F32) {
            float *dst = static_cast<float *>(a.out) + o;
            if (whole) {
                u32x4 lo = {__float_as_uint(h_to_f32(h[0])), __float_as_uint(h_to_f32(h[1])),
                            __float_as_uint(h_to_f32(h[2])), __float_as_uint(h_to_f32(h[3]))};
                u32x4 hi = {__float_as_uint(h_to_f32(h[4])), __float_as_uint(h_to_f32(h[5])),
                            __float_as_uint(h_to_f32(h[6])), __float_as_uint(h_to_f32(h[7]))};
                reinterpret_cast<u32x4 *>(dst)[0] = lo;
                reinterpret_cast<u32x4 *>(dst)[1] = hi;
            } else {
                for (int t = 0; t < 8 && j0 + t < a.IN; ++t) dst[t] = h_to_f32(h[t]);
            }
        } else {
            if (a.out_type == VQK_BF16) {
#pragma unroll
                for (int t = 0; t < 8; ++t) h[t] = h_to_bf16(h[t]);
            }
            uint16_t *dst = static_cast<uint16_t *>(a.out) + o;
            if (whole) {
                u32x4 v = {uint32_t(h[0]) | (uint32_t(h[1]) << 16), uint32_t(h[2]) | (uint32_t(h[3]) << 16),
                           uint32_t(h[4]) | (uint32_t(h[5]) << 16), uint32_t(h[6]) | (uint32_t(h[7]) << 16)};
                *reinterpret_cast<u32x4 *>(dst) = v;
            } else {
                for (int t = 0; t < 8 && j0 + t < a.IN; ++t) dst[t] = h[t];
            }
        }
    }
}

// Validates an embedding table descriptor (E == 1, OUT = table rows) and
// fills the layout fields of `a`.
static int embed_args(const vqk_weights *w, EmbedArgs *a) {
    if (!w || !w->codes || !w->codebook || !w->scales)
        return set_error(VQK_EINVAL, "embedding: codes, codebook and scales are required");
    if (w->D < 1 || w->D > 16)
        return set_error(VQK_ENOTIMPL, "embedding: subvector dim d=%d outside 1..16", w->D);
    if (w->K < 1 || w->K > 65536)
        return set_error(VQK_EINVAL, "codebook K=%lld outside [1, 65536]", (long long)w->K);
    if (w->k_expect && w->k_expect != w->K)
        return set_error(VQK_ESHARDED, "VQ codebook was sharded; must be replicated (K=%lld, "
                         "expected %lld)", (long long)w->K, (long long)w->k_expect);
    if (w->E != 1 || w->OUT < 1 || w->IN < 1)
        return set_error(VQK_EINVAL, "embedding: expects E=1, rows>=1, IN>=1 (E=%lld OUT=%lld "
                         "IN=%lld)", (long long)w->E, (long long)w->OUT, (long long)w->IN);
    if (w->IN % w->D)
        return set_error(VQK_EINVAL, "IN=%lld is not a multiple of d=%d", (long long)w->IN, w->D);
    if (w->group < 1 || w->IN % w->group)
        return set_error(VQK_EINVAL, "group_size %d does not divide IN=%lld", w->group,
                         (long long)w->IN);
    if (w->row_table)
        return set_error(VQK_ENOTIMPL, "embedding tables have no skipzero row table");
    const int64_t nsub = w->IN / w->D;
    a->codes = w->codes;
    a->code_cols = w->code_cols;
    a->codebook = w->codebook;
    a->K = w->K;
    a->D = w->D;
    a->G = w->group;
    a->scales = w->scales;
    a->ngrp = w->IN / w->group;
    a->rows = w->OUT;
    a->IN = w->IN;
    if (w->pack_bits == 0) {
        if (w->code_type == VQK_U8) {
            if (w->K > 256) return set_error(VQK_EINVAL, "uint8 codes cannot index K=%lld", (long long)w->K);
            a->layout = kEmbU8; a->bits = 8;
        } else if (w->code_type == VQK_U16) {
            a->layout = kEmbU16; a->bits = 16;
        } else {
            return set_error(VQK_EINVAL, "unpacked codes must be uint8 or uint16");
        }
        if (w->code_cols != nsub)
            return set_error(VQK_EINVAL, "codes are %lld cols, expected NSUB=%lld",
                             (long long)w->code_cols, (long long)nsub);
        return VQK_OK;
    }
    if (w->pack_bits < 1 || w->pack_bits > 16)
        return set_error(VQK_ENOTIMPL, "pack_bits=%d: only 0 (unpacked) and 1..16 exist", w->pack_bits);
    if (w->K > (int64_t(1) << w->pack_bits))
        return set_error(VQK_EINVAL, "K=%lld does not fit %d-bit codes", (long long)w->K, w->pack_bits);
    a->bits = w->pack_bits;
    if (w->code_type == VQK_U32) {
        const int64_t wpr = (nsub + kBlock - 1) / kBlock * w->pack_bits;
        if (w->code_cols != wpr)
            return set_error(VQK_EINVAL, "packed codes are %lld words/row, expected %lld",
                             (long long)w->code_cols, (long long)wpr);
        a->layout = kEmbBlocks;
    } else if (w->code_type == VQK_U8) {
        if (w->code_cols * 8 < nsub * w->pack_bits)
            return set_error(VQK_EINVAL, "byte-stream rows of %lld bytes cannot hold %lld %d-bit codes",
                             (long long)w->code_cols, (long long)nsub, w->pack_bits);
        a->layout = kEmbStream;
    } else {
        return set_error(VQK_EINVAL, "packed codes must be uint32 words or a uint8 byte stream");
    }
    return VQK_OK;
}

}  // namespace vqk

using namespace vqk;

extern "C" {

int vqk_embed_gather(const vqk_weights *w, const void *ids, int32_t id_type, int64_t n, void *out,
                     int32_t out_type, void *stream) {
    EmbedArgs a;
    int rc = embed_args(w, &a);
    if (rc) return rc;
    if (id_type != VQK_I32 && id_type != VQK_I64)
        return set_error(VQK_EINVAL, "ids must be int32 or int64 (type %d)", id_type);
    if (out_type != VQK_F16 && out_type != VQK_BF16 && out_type != VQK_F32)
        return set_error(VQK_EINVAL, "output type %d is not fp16 / bf16 / fp32", out_type);
    if (n < 0 || (n > 0 && (!ids || !out)))
        return set_error(VQK_EINVAL, "vqk_embed_gather: bad ids / out");
    if (n == 0) return VQK_OK;
    a.ids = ids;
    a.id64 = id_type == VQK_I64;
    a.n = n;
    a.out = out;
    a.out_type = out_type;
    a.lanes_per_row = (a.IN + 7) / 8;
    a.vec_ok = (a.IN % 8 == 0) && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    const int64_t total = n * a.lanes_per_row;
    const int64_t blocks = (total + 255) / 256;
    const unsigned grid = unsigned(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(k_embed_gather, dim3(grid), dim3(256), 0, hipStream_t(stream), a);
    return hip_status(hipGetLastError(), "embedding gather launch");
}

}  // extern "C"
