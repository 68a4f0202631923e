// Index packing and dequantisation kernels (bit-exact paths).
//
//  vqk_pack / vqk_unpack          vq_pack.pack / vq_pack.unpack (vq_pack.py:48-97)
//  vqk_dequant                    wdec_decode (vq_switch.py:3463-3544)
//  vqk_dequant_experts            _decode_chunk / vq_decode (vq_switch.py:2542-2591, 4725-4782)
//
// Layout (vq_pack.py:11-27): each code row is ceil(NSUB/32) blocks of BITS
// uint32 words; code i of a block starts at bit i*BITS of the block, LSB
// first, and may straddle two words of its block. Widths 8 and 16 are
// byte-identical to little-endian uint8 / uint16 arrays.
//
// The dequantised weight is W[r, j*D+u] = fp16(f32(cb[c_rj, u]) * f32(s[r, (j*D+u)/G])):
// the product of two fp16 values is exact in fp32, so the one v_cvt_f16_f32
// (round to nearest even) is the only rounding, as in the reference.
#include "vqk_common.h"

namespace vqk {

// Field j of a packed row, for a runtime width (1..16).
__device__ __forceinline__ uint32_t packed_code(const uint32_t *row, int64_t j, int bits) {
    const int64_t bit = (j >> 5) * (int64_t(kBlock) * bits) + (j & 31) * bits;
    const int sh = int(bit & 31);
    const int64_t wi = bit >> 5;
    uint32_t v = row[wi] >> sh;
    if (sh + bits > 32) v |= row[wi + 1] << (32 - sh);
    return v & ((1u << bits) - 1u);
}

// grid: x covers codes of a row, y strides over rows.
__global__ void __launch_bounds__(256) k_unpack(const uint32_t *packed, int64_t rows, int64_t nsub,
                                                int bits, void *codes) {
    const int64_t wpr = (nsub + kBlock - 1) / kBlock * bits;
    const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (j >= nsub) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const uint32_t c = packed_code(packed + r * wpr, j, bits);
        if (bits <= 8) static_cast<uint8_t *>(codes)[r * nsub + j] = uint8_t(c);
        else static_cast<uint16_t *>(codes)[r * nsub + j] = uint16_t(c);
    }
}

// One thread per output word: gathers the (at most 32/bits + 2) fields that
// overlap word wi of its block. Field bits above `bits` are dropped.
__global__ void __launch_bounds__(256) k_pack(const uint16_t *codes, int64_t rows, int64_t nsub,
                                              int bits, uint32_t *packed) {
    const int64_t wpr = (nsub + kBlock - 1) / kBlock * bits;
    const int64_t w = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (w >= wpr) return;
    const int64_t blk = w / bits;
    const int wi = int(w % bits);
    const int lo = wi * 32;                 // first bit of this word inside the block
    const int i0 = lo / bits;
    const int i1 = min(kBlock - 1, (lo + 31) / bits);
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        uint32_t v = 0;
        for (int i = i0; i <= i1; ++i) {
            const int64_t j = blk * kBlock + i;
            const uint32_t c = j < nsub ? (uint32_t(codes[r * nsub + j]) & mask) : 0u;
            const int p = i * bits;         // field start inside the block
            v |= p >= lo ? (c << (p - lo)) : (c >> (lo - p));
        }
        packed[r * wpr + w] = v;
    }
}

// D halves to dst with one vector store.
template <int D>
__device__ __forceinline__ void store_halves(uint16_t *dst, const uint16_t (&v)[D]) {
    if constexpr (D == 2) {
        *reinterpret_cast<uint32_t *>(dst) = uint32_t(v[0]) | (uint32_t(v[1]) << 16);
    } else if constexpr (D == 4) {
        *reinterpret_cast<u32x2 *>(dst) = u32x2{uint32_t(v[0]) | (uint32_t(v[1]) << 16),
                                               uint32_t(v[2]) | (uint32_t(v[3]) << 16)};
    } else {
        *reinterpret_cast<u32x4 *>(dst) = u32x4{uint32_t(v[0]) | (uint32_t(v[1]) << 16),
                                               uint32_t(v[2]) | (uint32_t(v[3]) << 16),
                                               uint32_t(v[4]) | (uint32_t(v[5]) << 16),
                                               uint32_t(v[6]) | (uint32_t(v[7]) << 16)};
    }
}

struct DequantArgs {
    const void *codes;
    int64_t code_cols;       // u32 words (packed) or codes (unpacked) per code row
    int bits;                // packed width, 0 = unpacked
    int code_bytes;          // 1 or 2 when unpacked
    const uint16_t *codebook;
    int64_t K;
    const uint16_t *scales;
    int64_t ngrp;
    int G;
    const int32_t *row_table;
    const uint32_t *eidx;    // experts of the output chunk (NULL: flat rows)
    int64_t E, stored_rows;  // experts, code rows actually stored (bounds for device indices)
    int64_t OUT, IN, NSUB;
    int64_t r0, rows;        // output rows: flat rows [r0, r0+rows) or ne*OUT
    uint16_t *out;
    int64_t out_ld;          // elements per output row part (>= IN; columns past IN are zeros)
    int mode;                // kDqF16, kDqBF16 or kDqSplit
    int cw_log2;             // code columns per workgroup = 1 << cw_log2 (<= 256)
};

// Code row of output row `orow`, or -1 for a dead skipzero row, an expert id
// outside [0, E) or a corrupt table entry (the row is written as zeros).
__device__ __forceinline__ int64_t dq_code_row(const DequantArgs &a, int64_t orow) {
    int64_t flat;                           // row of the expanded [E*OUT] module
    if (a.eidx) {
        const uint32_t e = a.eidx[orow / a.OUT];
        flat = e < uint64_t(a.E) ? int64_t(e) * a.OUT + orow % a.OUT : -1;
    } else {
        flat = a.r0 + orow;
    }
    int64_t cr = -1;
    if (flat >= 0) cr = a.row_table ? int64_t(a.row_table[flat]) : flat;
    return cr < a.stored_rows ? cr : -1;    // never read past the codes
}

// The D-half table entry `c` as ONE vector load (D * 2 bytes): a gather per
// half would multiply the L2 requests that bound this kernel.
template <int D>
__device__ __forceinline__ void dq_entry(const uint16_t *cb, uint32_t c, uint16_t (&e)[D]) {
    if constexpr (D == 8) {                  // through the global address space
        const u32x4 ev = load_global(reinterpret_cast<const u32x4 *>(cb), int64_t(c));
        __builtin_memcpy(e, &ev, sizeof e);
    } else if constexpr (D == 4) {
        const u32x2 ev = load_global(reinterpret_cast<const u32x2 *>(cb), int64_t(c));
        __builtin_memcpy(e, &ev, sizeof e);
    } else {
        const uint32_t ev = load_global(reinterpret_cast<const uint32_t *>(cb), int64_t(c));
        __builtin_memcpy(e, &ev, sizeof e);
    }
}

// One thread per code column j, kDqRows output rows at a time: a workgroup
// is 2^cw_log2 columns x 256 / 2^cw_log2 row sets (the column count chosen to
// divide the row: config 5's 640 codes per row left a sixth of 256-wide
// workgroups idle), row set q taking rows q + i * GY of a stride of GY sets
// (GY = gridDim.y x row sets per workgroup). Each phase -- code rows, codes,
// scales, table entries, stores -- is issued for all of them before the next
// waits, so a thread has kDqRows code-load -> gather chains in flight instead
// of one (small weights are latency-bound; a large table with random codes is
// bound by the L2's random-read rate instead). Threads past the last code of
// a row zero its padding up to out_ld.
// The code format is a template parameter: with it decided at run time the
// compiler waited for each row's code load before issuing the next row's (one
// HBM round trip per row; config 5: 97-101 us per 17408 x 5120 linear).
constexpr int kDqRows = 4;
enum : int { kCfPacked = 0, kCfU8 = 1, kCfU16 = 2 };
template <int D, int CF>
__global__ void __launch_bounds__(256) k_dequant(DequantArgs a) {
    const int cw = 1 << a.cw_log2;
    const int nrs = int(blockDim.x) >> a.cw_log2, rs = int(threadIdx.x) >> a.cw_log2;
    const int64_t j = int64_t(blockIdx.x) * cw + (int(threadIdx.x) & (cw - 1));
    if (j * D >= a.out_ld) return;
    const bool pad = j >= a.NSUB;
    const int64_t gy = int64_t(gridDim.y) * nrs;
    // where code j sits in a packed row: word wi, shift sh (a field never
    // leaves its 32-code block, so a second word is within the row)
    int64_t wi = 0;
    int sh = 0;
    if (CF == kCfPacked) {
        const int64_t bit = (j >> 5) * (int64_t(kBlock) * a.bits) + (j & 31) * a.bits;
        wi = bit >> 5;
        sh = int(bit & 31);
    }
    const int64_t wi1 = wi + 1 < a.code_cols ? wi + 1 : wi;
    const bool any = a.stored_rows > 0;
    // codes and scales of the kDqRows rows of step o0 (row -1: nothing used).
    // Every row's loads are issued before any is used; a row with no code row
    // reads row 0 (so the loads need no branch) and is zeroed after.
    auto load_step = [&](int64_t o0, int64_t (&cr)[kDqRows], uint32_t (&c)[kDqRows],
                         uint16_t (&sc)[kDqRows]) {
#pragma unroll
        for (int i = 0; i < kDqRows; ++i) {
            const int64_t orow = o0 + i * gy;
            cr[i] = (orow < a.rows && !pad) ? dq_code_row(a, orow) : -1;
        }
        if (!any) {
#pragma unroll
            for (int i = 0; i < kDqRows; ++i) { c[i] = 0u; sc[i] = 0; }
            return;
        }
        uint32_t w0[kDqRows], w1[kDqRows];
#pragma unroll
        for (int i = 0; i < kDqRows; ++i) {
            const int64_t row = cr[i] >= 0 ? cr[i] : 0;
            if (CF == kCfPacked) {
                const uint32_t *r = static_cast<const uint32_t *>(a.codes) + row * a.code_cols;
                w0[i] = r[wi];
                w1[i] = r[wi1];
            } else if (CF == kCfU8) {
                w0[i] = static_cast<const uint8_t *>(a.codes)[row * a.code_cols + j];
            } else {
                w0[i] = static_cast<const uint16_t *>(a.codes)[row * a.code_cols + j];
            }
            // a group boundary can fall inside a subvector only if G % D != 0,
            // which validation refuses; one scale serves all D values
            sc[i] = a.scales[row * a.ngrp + (j * D) / a.G];
        }
#pragma unroll
        for (int i = 0; i < kDqRows; ++i) {
            uint32_t v = w0[i];
            if (CF == kCfPacked) {
                v >>= sh;
                if (sh + a.bits > 32) v |= w1[i] << (32 - sh);
                v &= (1u << a.bits) - 1u;
            }
            c[i] = cr[i] >= 0 ? v : 0u;
            sc[i] = cr[i] >= 0 ? sc[i] : uint16_t(0);
        }
    };
    for (int64_t o0 = int64_t(blockIdx.y) * nrs + rs; o0 < a.rows; o0 += gy * kDqRows) {
        int64_t cr[kDqRows];
        uint32_t c[kDqRows];
        uint16_t sc[kDqRows];
        load_step(o0, cr, c, sc);
#pragma unroll
        for (int i = 0; i < kDqRows; ++i)
            if (c[i] >= uint32_t(a.K)) c[i] = uint32_t(a.K - 1);   // never read past the table
        uint16_t e[kDqRows][D];
#pragma unroll
        for (int i = 0; i < kDqRows; ++i) {
            if (cr[i] >= 0) {
                dq_entry<D>(a.codebook, c[i], e[i]);
            } else {
#pragma unroll
                for (int u = 0; u < D; ++u) e[i][u] = 0;
            }
        }
#pragma unroll
        for (int i = 0; i < kDqRows; ++i) {
            const int64_t orow = o0 + i * gy;
            if (orow >= a.rows) continue;
            // dead skipzero row, expert id outside [0, E) or padding column: +0
            uint16_t vals[D];
            const float s = h_to_f32(sc[i]);
#pragma unroll
            for (int u = 0; u < D; ++u) vals[u] = cr[i] >= 0 ? f32_to_h(s * h_to_f32(e[i][u])) : uint16_t(0);
            if (a.mode == kDqF16) {
                store_halves<D>(a.out + orow * a.out_ld + j * D, vals);
            } else {
                // bf16(the fp16 value): one RNE (fp16 -> f32 is exact)
                uint16_t hi[D];
#pragma unroll
                for (int u = 0; u < D; ++u) hi[u] = f32_to_bf16(h_to_f32(vals[u]));
                if (a.mode == kDqBF16) {
                    store_halves<D>(a.out + orow * a.out_ld + j * D, hi);
                } else {
                    // [W_hi | W_lo | W_hi] rows of 3 * IN: W_lo = W - W_hi has at
                    // most 3 significant bits (a multiple of the fp16 ulp no larger
                    // than half a bf16 ulp), so W_hi + W_lo is the fp16 value exactly
                    uint16_t lo[D];
#pragma unroll
                    for (int u = 0; u < D; ++u) {
                        const float w = h_to_f32(vals[u]), h = bf16_to_f32(hi[u]);
                        lo[u] = (__float_as_uint(h) & 0x7f800000u) == 0x7f800000u ? uint16_t(0)
                                                                                  : f32_to_bf16(w - h);
                    }
                    uint16_t *dst = a.out + orow * 3 * a.out_ld + j * D;
                    store_halves<D>(dst, hi);
                    store_halves<D>(dst + a.out_ld, lo);
                    store_halves<D>(dst + 2 * a.out_ld, hi);
                }
            }
        }
    }
}

// Threads stride over the rows (`rpt` rows each where rows allow): fewer,
// longer-lived waves than one row per thread, whose tiny workgroups cost
// more to dispatch than their single gather.
static dim3 rows_grid(int64_t cols, int64_t rows, int64_t rpt = 1) {
    const int64_t gx = (cols + 255) / 256;
    int64_t gy = (rows + rpt - 1) / rpt;
    gy = gy < 1 ? 1 : (gy > 65535 ? 65535 : gy);
    return dim3(unsigned(gx), unsigned(gy), 1);
}

template <int D>
static void launch_dq(int cf, dim3 grid, hipStream_t st, const DequantArgs &a) {
    if (cf == kCfPacked) hipLaunchKernelGGL((k_dequant<D, kCfPacked>), grid, dim3(256), 0, st, a);
    else if (cf == kCfU8) hipLaunchKernelGGL((k_dequant<D, kCfU8>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_dequant<D, kCfU16>), grid, dim3(256), 0, st, a);
}

static int launch_dequant(const vqk_weights *w, const Geom &g, const uint32_t *eidx, int64_t r0,
                          int64_t rows, uint16_t *out, hipStream_t st, int mode = kDqF16,
                          int64_t out_ld = 0) {
    DequantArgs a;
    a.mode = mode;
    a.out_ld = out_ld > g.IN ? out_ld : g.IN;
    a.codes = w->codes;
    a.code_cols = w->code_cols;
    a.bits = g.packed ? g.BITS : 0;
    a.code_bytes = g.BITS / 8;
    a.codebook = w->codebook;
    a.K = g.K;
    a.scales = w->scales;
    a.ngrp = g.NGRP;
    a.G = g.G;
    a.row_table = w->row_table;
    a.eidx = eidx;
    a.E = g.E;
    a.stored_rows = g.rows;
    a.OUT = g.OUT; a.IN = g.IN; a.NSUB = g.NSUB;
    a.r0 = r0; a.rows = rows;
    a.out = out;
    if (rows == 0) return VQK_OK;
    // the widest of 256 / 128 / 64 columns that leaves the fewest idle lanes
    const int64_t cols = a.out_ld / g.D;
    a.cw_log2 = 8;
    for (int l = 7; l >= 6; --l) {
        const int64_t waste = (cols + (1 << l) - 1) / (1 << l) * (1 << l) - cols;
        const int64_t best = (cols + (1 << a.cw_log2) - 1) / (1 << a.cw_log2) * (1 << a.cw_log2) - cols;
        if (waste < best) a.cw_log2 = l;
    }
    const int64_t nrs = 256 >> a.cw_log2;
    int64_t gy = (rows + kDqRows * nrs - 1) / (kDqRows * nrs);
    gy = gy < 1 ? 1 : (gy > 65535 ? 65535 : gy);
    const dim3 grid(unsigned((cols + (1 << a.cw_log2) - 1) >> a.cw_log2), unsigned(gy), 1);
    const int cf = g.packed ? kCfPacked : (g.BITS == 8 ? kCfU8 : kCfU16);
    if (g.D == 2) launch_dq<2>(cf, grid, st, a);
    else if (g.D == 4) launch_dq<4>(cf, grid, st, a);
    else launch_dq<8>(cf, grid, st, a);
    return hip_status(hipGetLastError(), "dequant launch");
}

// Rows [r0, r0 + rows) of a validated module in `mode`: fp16 (bit-exact), bf16
// (the reference's cast of the fp16 weight to the activation dtype before its
// GEMM, vq_dense.py:288, 294) or the split bf16 rows of the fp32 path; rows
// of ld >= IN elements (per part), zero past IN. ld % D == 0.
int dequant_rows(const vqk_weights *w, int64_t r0, int64_t rows, uint16_t *out, int mode, int64_t ld,
                 hipStream_t st) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (ld % g.D) return set_error(VQK_EINVAL, "dequant row stride %lld", (long long)ld);
    return launch_dequant(w, g, nullptr, r0, rows, out, st, mode, ld);
}

}  // namespace vqk

using namespace vqk;

extern "C" {

int vqk_pack(const uint16_t *codes, int64_t rows, int64_t nsub, int32_t bits, uint32_t *packed,
             void *stream) {
    if (!codes || !packed || rows < 0 || nsub < 0 || bits < 1 || bits > 16)
        return set_error(VQK_EINVAL, "vqk_pack: bad arguments");
    const int64_t wpr = (nsub + kBlock - 1) / kBlock * bits;
    if (rows == 0 || wpr == 0) return VQK_OK;
    hipLaunchKernelGGL(k_pack, rows_grid(wpr, rows), dim3(256), 0, hipStream_t(stream), codes, rows,
                       nsub, int(bits), packed);
    return hip_status(hipGetLastError(), "pack launch");
}

int vqk_unpack(const uint32_t *packed, int64_t rows, int64_t nsub, int32_t bits, void *codes,
               void *stream) {
    if (!codes || !packed || rows < 0 || nsub < 0 || bits < 1 || bits > 16)
        return set_error(VQK_EINVAL, "vqk_unpack: bad arguments");
    if (rows == 0 || nsub == 0) return VQK_OK;
    hipLaunchKernelGGL(k_unpack, rows_grid(nsub, rows), dim3(256), 0, hipStream_t(stream), packed,
                       rows, nsub, int(bits), codes);
    return hip_status(hipGetLastError(), "unpack launch");
}

int vqk_dequant(const vqk_weights *w, int64_t r0, int64_t rows, uint16_t *out, void *stream) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (!out && rows > 0) return set_error(VQK_EINVAL, "vqk_dequant: out is NULL");
    if (r0 < 0 || rows < 0 || r0 + rows > g.E * g.OUT)
        return set_error(VQK_EINVAL, "rows [%lld, %lld) outside the module's %lld rows",
                         (long long)r0, (long long)(r0 + rows), (long long)(g.E * g.OUT));
    return launch_dequant(w, g, nullptr, r0, rows, out, hipStream_t(stream));
}

int vqk_dequant_experts(const vqk_weights *w, const uint32_t *eidx, int64_t ne, uint16_t *out,
                        void *stream) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if ((!out && ne > 0) || (!eidx && ne > 0) || ne < 0)
        return set_error(VQK_EINVAL, "vqk_dequant_experts: bad arguments");
    return launch_dequant(w, g, eidx, 0, ne * g.OUT, out, hipStream_t(stream));
}

}  // extern "C"
