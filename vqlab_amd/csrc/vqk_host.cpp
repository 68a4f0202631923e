// Host side of libvqk: error reporting, descriptor validation, code widths,
// host pack/unpack, capability predicates and the skipzero row table.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "vqk_common.h"

namespace vqk {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return VQK_OK;
    return set_error(VQK_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

int act_size(int32_t type) {
    switch (type) {
        case VQK_F16: case VQK_BF16: return 2;
        case VQK_F32: return 4;
        default: return 0;
    }
}

int out_size(int32_t type) {
    return (type & ~int32_t(VQK_VIA_F16 | 0xff)) ? 0 : act_size(type & 0xff);
}

static int64_t wpr_of(int64_t nsub, int bits) { return (nsub + kBlock - 1) / kBlock * bits; }

int make_geom(const vqk_weights *w, Geom *g) {
    memset(g, 0, sizeof *g);
    if (!w || !w->codes || !w->codebook || !w->scales)
        return set_error(VQK_EINVAL, "weights: codes, codebook and scales are required");
    if (w->D != 2 && w->D != 4 && w->D != 8)
        return set_error(VQK_ENOTIMPL,
                         "no fused kernel for subvector dim d=%d; d=2, 4 and 8 are "
                         "implemented and each is dispatched explicitly", w->D);
    if (w->K < 1 || w->K > 65536)
        return set_error(VQK_EINVAL, "codebook K=%lld outside [1, 65536]", (long long)w->K);
    if (w->k_expect && w->k_expect != w->K)
        return set_error(VQK_ESHARDED,
                         "VQ codebook was sharded: K=%lld, expected %lld. The codebook is "
                         "a SHARED lookup table and must be replicated across "
                         "tensor-parallel ranks, not sliced", (long long)w->K,
                         (long long)w->k_expect);
    if (w->E < 1 || w->OUT < 1 || w->IN < 1)
        return set_error(VQK_EINVAL, "bad shape E=%lld OUT=%lld IN=%lld", (long long)w->E,
                         (long long)w->OUT, (long long)w->IN);
    if (w->IN % w->D)
        return set_error(VQK_EINVAL, "IN=%lld is not a multiple of d=%d", (long long)w->IN, w->D);
    if (w->group < 1 || w->IN % w->group)
        return set_error(VQK_EINVAL, "group_size %d does not divide IN=%lld", w->group,
                         (long long)w->IN);
    if (w->group % w->D)
        return set_error(VQK_ENOTIMPL, "group_size %d does not hold whole d=%d subvectors",
                         w->group, w->D);
    g->E = w->E; g->OUT = w->OUT; g->IN = w->IN; g->K = w->K;
    g->D = w->D; g->G = w->group;
    g->NSUB = w->IN / w->D;
    g->NB = (g->NSUB + kBlock - 1) / kBlock;
    g->NGRP = w->IN / w->group;
    if (w->pack_bits == 0) {
        if (w->code_type == VQK_U8) {
            if (w->K > 256)
                return set_error(VQK_EINVAL, "uint8 codes cannot index K=%lld", (long long)w->K);
            g->BITS = 8;
        } else if (w->code_type == VQK_U16) {
            g->BITS = 16;
        } else {
            return set_error(VQK_EINVAL, "unpacked codes must be uint8 or uint16");
        }
        if (w->code_cols != g->NSUB)
            return set_error(VQK_EINVAL, "codes are %lld cols, expected NSUB=%lld for IN=%lld, d=%d",
                             (long long)w->code_cols, (long long)g->NSUB, (long long)w->IN, w->D);
        const int64_t bytes = g->NSUB * (g->BITS / 8);
        g->row_words = (bytes % 4) ? 0 : bytes / 4;
        g->packed = false;
    } else if (w->pack_bits >= 1 && w->pack_bits <= 16) {
        if (w->code_type != VQK_U32)
            return set_error(VQK_EINVAL, "packed codes must be uint32 words");
        if (w->K > (int64_t(1) << w->pack_bits))
            return set_error(VQK_EINVAL, "K=%lld does not fit %d-bit codes", (long long)w->K,
                             w->pack_bits);
        g->BITS = w->pack_bits;
        const int64_t wpr = wpr_of(g->NSUB, g->BITS);
        if (w->code_cols != wpr)
            return set_error(VQK_EINVAL,
                             "packed codes are %lld words/row, expected %lld for IN=%lld, d=%d, bits=%d",
                             (long long)w->code_cols, (long long)wpr, (long long)w->IN, w->D,
                             w->pack_bits);
        g->row_words = wpr;
        g->packed = true;
    } else {
        return set_error(VQK_ENOTIMPL, "pack_bits=%d: only 0 (unpacked) and 1..16 exist",
                         w->pack_bits);
    }
    if (w->row_table) {
        if (w->n_live < 0) return set_error(VQK_EINVAL, "row_table needs n_live >= 0");
        g->rows = w->n_live;
    } else {
        g->rows = g->E * g->OUT;
    }
    const int spg = g->G / g->D;   // codes per scale group
    if (spg <= kBlock && kBlock % spg == 0) { g->gpb = kBlock / spg; g->bpg = 1; }
    else if (spg % kBlock == 0) { g->gpb = 1; g->bpg = spg / kBlock; }
    else { g->gpb = 0; g->bpg = 0; }
    const int gpb_fast = g->D == 4 ? 2 : (g->D == 8 ? 4 : 1);   // group of 64 weights
    g->fast_ok = (g->NSUB % kBlock == 0) && g->row_words > 0 && g->NB <= kWave &&
                 g->BITS >= 2 && (g->gpb == 1 || g->gpb == gpb_fast) &&
                 g->OUT <= INT32_MAX && g->IN <= INT32_MAX &&
                 (reinterpret_cast<uintptr_t>(w->codebook) & 15) == 0;   // async LDS copy
    return VQK_OK;
}

}  // namespace vqk

using namespace vqk;

extern "C" {

const char *vqk_version(void) { return "vqk 0.1 gfx950"; }
const char *vqk_last_error(void) { return g_err; }

int vqk_bits_for_k(int64_t k, int32_t *bits) {
    if (!bits) return set_error(VQK_EINVAL, "bits pointer is NULL");
    int b = 0;
    while ((int64_t(1) << b) < k) ++b;
    if (k < 1 || (int64_t(1) << b) != k)
        return set_error(VQK_EINVAL, "K=%lld is not a power of two", (long long)k);
    *bits = b;
    return VQK_OK;
}

int64_t vqk_words_per_row(int64_t nsub, int32_t bits) {
    if (nsub < 0 || bits < 1 || bits > 32) return -1;
    return wpr_of(nsub, bits);
}

int vqk_pack_bits_for(int64_t k, int64_t nsub, int32_t pack_unaligned, int32_t *bits) {
    int32_t b;
    int rc = vqk_bits_for_k(k, &b);
    if (rc) return rc;
    if ((nsub % kBlock) && !pack_unaligned) b = 0;
    else if (b % 8 == 0) b = 0;
    *bits = b;
    return VQK_OK;
}

int vqk_pack_host(const uint16_t *codes, int64_t rows, int64_t nsub, int32_t bits,
                  uint32_t *packed) {
    if (!codes || !packed || rows < 0 || nsub < 0 || bits < 1 || bits > 16)
        return set_error(VQK_EINVAL, "vqk_pack_host: bad arguments");
    const int64_t wpr = wpr_of(nsub, bits);
    const uint32_t lim = 1u << bits;
    for (int64_t r = 0; r < rows; ++r) {
        uint32_t *out = packed + r * wpr;
        memset(out, 0, sizeof(uint32_t) * size_t(wpr));
        const uint16_t *in = codes + r * nsub;
        for (int64_t j = 0; j < nsub; ++j) {
            const uint32_t c = in[j];
            if (c >= lim) return set_error(VQK_EINVAL, "code exceeds bit width");
            const int64_t bit = (j / kBlock) * kBlock * bits + (j % kBlock) * bits;
            const uint64_t v = uint64_t(c) << (bit & 31);
            out[bit >> 5] |= uint32_t(v);
            if ((bit & 31) + bits > 32) out[(bit >> 5) + 1] |= uint32_t(v >> 32);
        }
    }
    return VQK_OK;
}

int vqk_unpack_host(const uint32_t *packed, int64_t rows, int64_t nsub, int32_t bits,
                    void *codes) {
    if (!codes || !packed || rows < 0 || nsub < 0 || bits < 1 || bits > 16)
        return set_error(VQK_EINVAL, "vqk_unpack_host: bad arguments");
    const int64_t wpr = wpr_of(nsub, bits);
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t r = 0; r < rows; ++r) {
        const uint32_t *in = packed + r * wpr;
        for (int64_t j = 0; j < nsub; ++j) {
            const int64_t bit = (j / kBlock) * kBlock * bits + (j % kBlock) * bits;
            uint64_t v = in[bit >> 5];
            if ((bit & 31) + bits > 32) v |= uint64_t(in[(bit >> 5) + 1]) << 32;
            const uint32_t c = uint32_t(v >> (bit & 31)) & mask;
            if (bits <= 8) static_cast<uint8_t *>(codes)[r * nsub + j] = uint8_t(c);
            else static_cast<uint16_t *>(codes)[r * nsub + j] = uint16_t(c);
        }
    }
    return VQK_OK;
}

int vqk_dense_fits(int64_t K, int64_t IN, int32_t G, int32_t D) {
    return (D == 2 || D == 4 || D == 8) && K >= 1 && K <= 65536 && IN > 0 && G > 0 &&
           IN % D == 0 && IN % G == 0 && G % D == 0;
}

int vqk_wdec_fits(int32_t D, int64_t NSUB, int32_t G, int32_t pack_bits) {
    return (D == 2 || D == 4 || D == 8) && NSUB > 0 && G > 0 && G % D == 0 &&
           pack_bits >= 0 && pack_bits <= 16;
}

int vqk_skipzero_row_table_host(const uint8_t *rowmask, int64_t E, int64_t OUT,
                                int32_t *table, int64_t *n_live) {
    if (!rowmask || !table || E < 0 || OUT < 0)
        return set_error(VQK_EINVAL, "vqk_skipzero_row_table_host: bad arguments");
    const int64_t rb = (OUT + 7) / 8;
    int64_t k = 0;
    for (int64_t e = 0; e < E; ++e)
        for (int64_t r = 0; r < OUT; ++r) {
            const bool live = (rowmask[e * rb + r / 8] >> (r % 8)) & 1u;
            if (k > INT32_MAX) return set_error(VQK_EINVAL, "too many live rows");
            table[e * OUT + r] = live ? int32_t(k++) : -1;
        }
    if (n_live) *n_live = k;
    return VQK_OK;
}

}  // extern "C"
