// Register-decode matrix-core kernel for expert segments (and small dense
// batches): y[t, o] = sum_i x[t, i] * W[o, i] for up to 16 tokens t that share
// one expert's weight rows o.
//
// No weight tile passes through LDS. v_mfma_f32_16x16x32_f16 takes its A
// operand as 8 consecutive k values of one row per lane (lane l: row l % 16,
// k group l / 16), which for d = 8 is exactly one codebook entry. So each
// lane owns one 32-code packing block of a weight row (its BITS words and
// scales in registers, as in the GEMV), and per MFMA step decodes the next
// 8 weights straight into its A operand:
//     W[8] = cb[code] * s          (v_pk_mul_f16: the exact product of two fp16
//                                   values rounded once to fp16, i.e. the
//                                   bit-exact dequant fp16(f32(cb) * f32(s)))
// The lane groups g = 0..3 hold blocks 4*sb + g of the same row, and the
// B operand (x) of lane (token t, group g) is read from the matching columns
// of an LDS copy of the tokens' activations, so A and B use the same k
// permutation and the product is the plain dot product.
//
// The codebook table sits in LDS (all of it, or its first 88-128 KB when it
// is larger; those codes beyond it are read from L2), with one zero entry
// past the staged part: lanes without a block (dead skipzero row, past the
// row's end) decode code 0 from it with scale 0, i.e. weights +0.
//
// Workgroup = 8 waves x one row tile of 16 = 128 weight rows (two waves per
// SIMD); one token tile of <= 16 rows (grouped: one tile of an expert segment from the device
// sort, vq_switch.py:4590-4610; dense: 16 consecutive rows of x). The K loop
// walks supersteps of 4 blocks per row (128 * D columns); the x columns of
// the next superstep and the next blocks' words are loaded while the
// current superstep runs, and one barrier per superstep publishes the
// double-buffered x chunk.
#pragma once

#include "vqk_gemv.h"

namespace vqk {

struct SegParams {
    const uint32_t *codes;     // code rows as 32-code blocks of BITS words
    int64_t row_words;         // words per code row (NB * BITS)
    const uint16_t *codebook;  // fp16 [K, D]
    int32_t K;
    const uint16_t *scales;    // fp16, ngrp per code row
    int32_t ngrp, bpg;         // bpg: blocks per scale group when GPB == 1
    const int32_t *row_table;  // [E, OUT] or NULL
    int64_t stored_rows;
    int32_t E, OUT, IN, NB;
    const void *x;
    int32_t x_type, xkrep;
    const float *xg, *xu;      // if xg: x row = fp16(silu(xg) * xu) from fp32 rows of IN
    void *y;
    int32_t y_type;
    int32_t N;                 // dense: rows of x; grouped: pairs
    const int32_t *tmeta;      // grouped: (expert or -1, row_start, nrows) per tile
    const int32_t *ntiles;     // grouped: tiles built by the sort
    const int32_t *order;      // grouped: sorted position -> pair
    int32_t ksplit;            // K slices (blockIdx.z): slice z writes fp32 partials at y + z * ypart
    int64_t ypart;
    int32_t xparts;            // xg / xu given as xparts partial rows, xpstride elements apart
    int64_t xpstride;
};

// Eight fp16 values fp16(silu(g) * u) where g and u are the fixed-order sums
// of `np` fp32 partial rows `stride` elements apart (K-split producers).
__device__ __forceinline__ u32x4 swiglu8_parts(const float *g, const float *u, int np,
                                               int64_t stride) {
    float gv[8], uv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { gv[i] = 0.f; uv[i] = 0.f; }
    for (int q = 0; q < np; ++q) {
        const f32x4 *gq = reinterpret_cast<const f32x4 *>(g + q * stride);
        const f32x4 *uq = reinterpret_cast<const f32x4 *>(u + q * stride);
        const f32x4 g0 = gq[0], g1 = gq[1], u0 = uq[0], u1 = uq[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            gv[i] += g0[i]; gv[4 + i] += g1[i];
            uv[i] += u0[i]; uv[4 + i] += u1[i];
        }
    }
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = f32_to_h(gv[i] / (1.f + __expf(-gv[i])) * uv[i]);
    return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

constexpr int kSegRows = 128;      // weight rows per workgroup
constexpr int kSegTok = 16;        // tokens per tile
// Tiles of at most kSegTokNarrow tokens, for routings that put a few pairs on
// each expert (an MTP verify batch: ~1.25 per expert): the smaller x chunk
// leaves more of the 160 KB to a d8 table too large for LDS.
constexpr int kSegTokNarrow = 4;
// ... or of at most kSegTokMid: a routing that puts several pairs on each of
// fewer experts (an MTP batch drawn with 1..8 tokens per touched expert)
// would split them into two or more 4-row tiles, each decoding the expert's
// weights again. The device sort picks between the two per call (fewer
// decoded rows against the smaller LDS part of the table) and records its
// choice after the tile count; k_seg_persist follows it.
constexpr int kSegTokMid = 8;
// Waves of the persistent kernel's workgroup (one per CU): two per SIMD, so
// one wave's table reads are in flight while the other decodes; an item is
// 32 rows per wave.
constexpr int kPersistWaves = 8;

// Entry D halves of a table (LDS or global) as 8 halves: d8 one entry,
// d4 two, d2 four (the codes of one MFMA step).
template <int D, int BITS>
__device__ __forceinline__ h8 step_entries(const uint32_t (&w)[BITS], int s, const f16 *tab,
                                           uint32_t kmax, bool clamp) {
    if constexpr (D == 8) {
        uint32_t c = block_field<BITS>(w, s);
        if (clamp) c = min(c, kmax);
        return *reinterpret_cast<const h8 *>(tab + c * 8);
    } else if constexpr (D == 4) {
        uint32_t c0 = block_field<BITS>(w, 2 * s), c1 = block_field<BITS>(w, 2 * s + 1);
        if (clamp) { c0 = min(c0, kmax); c1 = min(c1, kmax); }
        const h4 a = *reinterpret_cast<const h4 *>(tab + c0 * 4);
        const h4 b = *reinterpret_cast<const h4 *>(tab + c1 * 4);
        return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    } else {
        uint32_t c[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            c[u] = block_field<BITS>(w, 4 * s + u);
            if (clamp) c[u] = min(c[u], kmax);
        }
        const h2 a = *reinterpret_cast<const h2 *>(tab + c[0] * 2);
        const h2 b = *reinterpret_cast<const h2 *>(tab + c[1] * 2);
        const h2 e = *reinterpret_cast<const h2 *>(tab + c[2] * 2);
        const h2 f = *reinterpret_cast<const h2 *>(tab + c[3] * 2);
        return h8{a[0], a[1], b[0], b[1], e[0], e[1], f[0], f[1]};
    }
}

// The same for a table only partly in LDS: codes below `kl` read the LDS
// copy, the rest the global table (clamped to kmax), under complementary
// lane masks into the same registers.
template <int D>
__device__ __forceinline__ typename EntryT<D>::type hyb_entry(uint32_t c, const f16 *tl, const f16 *tg,
                                                              uint32_t kl, uint32_t kmax) {
    typedef typename EntryT<D>::type E;
    E e;
    // branch-free: both reads for every lane (the other one of entry 0: a
    // broadcast in LDS, one coalesced line in L2), so the unrolled steps'
    // reads are not split into exec-masked blocks and can overlap
    const bool inl = c < kl;
    const E el = reinterpret_cast<const E *>(tl)[inl ? c : 0u];
    const E eg = load_global(reinterpret_cast<const E *>(tg), inl ? 0u : min(c, kmax));
    e = inl ? el : eg;
    return e;
}

template <int D, int BITS>
__device__ __forceinline__ h8 step_entries_hyb(const uint32_t (&w)[BITS], int s, const f16 *tl,
                                               const f16 *tg, uint32_t kl, uint32_t kmax) {
    if constexpr (D == 8) {
        return hyb_entry<8>(block_field<BITS>(w, s), tl, tg, kl, kmax);
    } else if constexpr (D == 4) {
        const h4 a = hyb_entry<4>(block_field<BITS>(w, 2 * s), tl, tg, kl, kmax);
        const h4 b = hyb_entry<4>(block_field<BITS>(w, 2 * s + 1), tl, tg, kl, kmax);
        return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    } else {
        const h2 a = hyb_entry<2>(block_field<BITS>(w, 4 * s), tl, tg, kl, kmax);
        const h2 b = hyb_entry<2>(block_field<BITS>(w, 4 * s + 1), tl, tg, kl, kmax);
        const h2 e = hyb_entry<2>(block_field<BITS>(w, 4 * s + 2), tl, tg, kl, kmax);
        const h2 f = hyb_entry<2>(block_field<BITS>(w, 4 * s + 3), tl, tg, kl, kmax);
        return h8{a[0], a[1], b[0], b[1], e[0], e[1], f[0], f[1]};
    }
}

// LDS entries of a table too large for LDS that the kernel stages: what the
// x chunk (TOK x (128 D + 8) halves) leaves of the 160 KB -- 124 KB of a d8
// table (7936 of K16384's entries; 151 KB, 9664 entries, with 4-token
// tiles; 143 KB, 9152 entries, with 8-token tiles), all of a d4 K16384
// table, 144 KB of a d2 one.
__host__ __device__ constexpr int seg_hyb_entries(int D, int TOK = kSegTok) {
    return (D == 8 ? (TOK == kSegTokNarrow ? 151 : (TOK == kSegTokMid ? 143 : 124)) * 1024
                   : (D == 4 ? 128 * 1024 : 144 * 1024)) / (2 * D);
}


// Waves of k_seg_mfma: 8 x one 16-row tile (two waves per SIMD, so one
// decodes while the other waits on its loads), 128 weight rows per workgroup.
constexpr int kSegWaves = 8;

template <int D, int BITS, int GPB, bool CBL, int TOK = kSegTok>
__global__ void __launch_bounds__(kSegWaves * 64) k_seg_mfma(const SegParams p) {
    constexpr int NT = kSegWaves * 64;          // threads
    constexpr int TN = kSegRows / (16 * kSegWaves);   // 16-row tiles per wave
    constexpr int SPB = 4 * D;                  // MFMA steps per block (8 weights each)
    constexpr int CC = 128 * D;                 // x columns per superstep
    constexpr int XS = CC + 8;                  // LDS row stride of an x chunk (halves)
    constexpr int PIECES = TOK * CC / 8;        // 16-byte pieces per chunk
    constexpr int PPT = PIECES / NT;
    static_assert(PIECES % NT == 0, "chunk must split evenly over the threads");
    // LDS table entries: the whole table, or the first seg_hyb_entries of it
    constexpr int CBN = CBL ? (1 << BITS) : seg_hyb_entries(D, TOK);
    static_assert(TOK == kSegTok || TOK == kSegTokNarrow, "token tile of 16 or 4 rows");
    static_assert(TOK * XS * 2 + (CBN + 1) * D * 2 <= 160 * 1024, "LDS beyond 160 KB");

    extern __shared__ __align__(16) uint8_t smem[];
    f16 *xs = reinterpret_cast<f16 *>(smem);    // [TOK][XS]
    f16 *cbl = xs + TOK * XS;                   // [CBN + 1][D]; entry CBN is zero

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 15, lg = lane >> 4;

    int expert, row0, nrows;
    const bool grouped = p.tmeta != nullptr;
    if (grouped) {
        if (int(blockIdx.y) >= *p.ntiles) return;   // uniform, before any barrier
        const int32_t *tm = p.tmeta + 3 * blockIdx.y;
        expert = tm[0];
        row0 = tm[1];
        nrows = tm[2];
    } else {
        expert = 0;
        row0 = int(blockIdx.y) * TOK;
        nrows = min(TOK, p.N - row0);
    }
    const int o0 = int(blockIdx.x) * kSegRows + wave * 16 * TN;

    {
        const int ent = min(p.K, CBN);
        lds_copy_async(p.codebook, cbl, ent * D * 2, (CBN + 1) * D * 2);
    }

    // ---- this lane's weight rows (one per row tile) and token rows of its x pieces
    int64_t cr[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const int o = o0 + 16 * tn + ln;
        int64_t f = -1;
        if (expert >= 0 && expert < p.E && o < p.OUT) {
            f = int64_t(expert) * p.OUT + o;
            if (p.row_table) f = p.row_table[f];
            if (f < 0 || f >= p.stored_rows) f = -1;
        }
        cr[tn] = f;
    }
    int64_t xoff[PPT];
#pragma unroll
    for (int r = 0; r < PPT; ++r) {
        const int t = (tid + NT * r) / (CC / 8);
        int64_t off = -1;
        if (t < nrows) {
            const int64_t row = grouped ? int64_t(p.order[row0 + t] / p.xkrep) : int64_t(row0 + t);
            off = row * p.IN;
        }
        xoff[r] = off;
    }

    const int NSS = (p.NB + 3) >> 2;
    // K slice of this workgroup: supersteps [sb0, sb1) (all of them unless split)
    const int ks = p.ksplit > 1 ? p.ksplit : 1, per = (NSS + ks - 1) / ks;
    const int sb0 = min(NSS, int(blockIdx.z) * per), sb1 = min(NSS, sb0 + per);
    const uint32_t kmax = uint32_t(p.K - 1);

    auto load_x = [&](int sb, u32x4 (&v)[PPT]) {
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const int col = sb * CC + ((tid + NT * r) % (CC / 8)) * 8;
            const bool ok = xoff[r] >= 0 && col < p.IN;
            if (p.xg) {
                v[r] = !ok ? u32x4{0, 0, 0, 0}
                     : p.xparts > 1 ? swiglu8_parts(p.xg + xoff[r] + col, p.xu + xoff[r] + col,
                                                    p.xparts, p.xpstride)
                                    : swiglu8(p.xg + xoff[r] + col, p.xu + xoff[r] + col);
            } else {
                v[r] = ok ? load8_act(p.x, p.x_type, xoff[r] + col) : u32x4{0, 0, 0, 0};
            }
        }
    };
    auto store_x = [&](const u32x4 (&v)[PPT]) {
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const int pc = tid + NT * r;
            *reinterpret_cast<u32x4 *>(xs + (pc / (CC / 8)) * XS + (pc % (CC / 8)) * 8) = v[r];
        }
    };
    // words and scales of block 4*sb + lg of each row; lanes without one get
    // zero words, zero scales and the zero entry. Plain (cached) loads: a
    // superstep takes 4 blocks of a row (224 bytes at 14 bits), so lines
    // straddle supersteps and a streaming load would fetch them twice.
    auto load_w = [&](int sb, uint32_t (&w)[TN][BITS], h2 (&s)[TN][GPB], bool (&live)[TN]) {
        const int b = 4 * sb + lg;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            live[tn] = cr[tn] >= 0 && b < p.NB;
            if (live[tn]) {
                const uint32_t *src = p.codes + cr[tn] * p.row_words + int64_t(b) * BITS;
#pragma unroll
                for (int i = 0; i < BITS; ++i) w[tn][i] = src[i];
                const uint16_t *sr = p.scales + cr[tn] * p.ngrp + (GPB == 1 ? b / p.bpg : b * GPB);
#pragma unroll
                for (int g = 0; g < GPB; ++g) {
                    const f16 v = __builtin_bit_cast(f16, sr[g]);
                    s[tn][g] = h2{v, v};
                }
            } else {
#pragma unroll
                for (int i = 0; i < BITS; ++i) w[tn][i] = 0u;
#pragma unroll
                for (int g = 0; g < GPB; ++g) s[tn][g] = h2{0, 0};
            }
        }
    };

    f32x4 acc[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tn] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const uint32_t (&w)[TN][BITS], const h2 (&s)[TN][GPB],
                       const bool (&live)[TN]) {
        // MFMA column ln is token ln; with TOK < 16 the columns past the tile
        // repeat its rows and their sums are never stored
        const f16 *xb = xs + (ln & (TOK - 1)) * XS + lg * (32 * D);
        const f16 *tab[TN];
        uint32_t kl[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            tab[tn] = live[tn] ? cbl : cbl + CBN * D;        // dead lanes: code 0 -> zero entry
            kl[tn] = live[tn] ? uint32_t(min(p.K, CBN)) : 1u;
        }
        const f16 *tg = reinterpret_cast<const f16 *>(p.codebook);
#pragma unroll
        for (int st = 0; st < SPB; ++st) {
            const h8 xf = *reinterpret_cast<const h8 *>(xb + 8 * st);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int q = (st * GPB) / (4 * D);
                h8 e;
                if constexpr (CBL) e = step_entries<D, BITS>(w[tn], st, tab[tn], kmax, false);
                else e = step_entries_hyb<D, BITS>(w[tn], st, tab[tn], tg, kl[tn], kmax);
                const h2 sc = s[tn][q];
                const h8 wv = e * h8{sc[0], sc[0], sc[0], sc[0], sc[0], sc[0], sc[0], sc[0]};
                acc[tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv, xf, acc[tn], 0, 0, 0);
            }
        }
    };

    uint32_t w0[TN][BITS], w1[TN][BITS];
    h2 s0[TN][GPB], s1[TN][GPB];
    bool l0[TN], l1[TN];
    u32x4 xr[PPT];

    // One x chunk in LDS (the room a second one would take holds codebook
    // entries instead): the next superstep's x and weights are loaded into
    // registers before the current one multiplies, so their latency stays
    // hidden; the chunk is overwritten between two barriers.
    if (sb0 < sb1) {
        load_x(sb0, xr);
        load_w(sb0, w0, s0, l0);
        store_x(xr);
    }
    wait_vmem();
    __syncthreads();
    for (int sb = sb0; sb < sb1; sb += 2) {
        const bool more1 = sb + 1 < sb1;
        if (more1) {
            load_x(sb + 1, xr);
            load_w(sb + 1, w1, s1, l1);
        }
        compute(w0, s0, l0);
        if (!more1) break;
        __syncthreads();                        // every wave is done with chunk sb
        store_x(xr);
        __syncthreads();                        // chunk sb + 1 is in place
        const bool more2 = sb + 2 < sb1;
        if (more2) {
            load_x(sb + 2, xr);
            load_w(sb + 2, w0, s0, l0);
        }
        compute(w1, s1, l1);
        if (!more2) break;
        __syncthreads();
        store_x(xr);
        __syncthreads();
    }

    // ---- epilogue: lane holds rows 16*tn + 4*lg + i of token ln
    uint64_t alive[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) alive[tn] = __ballot(cr[tn] >= 0);
    const int64_t yoff = ks > 1 ? int64_t(blockIdx.z) * p.ypart : 0;   // K slice's partial
    if (ln < nrows) {
        const int64_t yr = grouped ? int64_t(p.order[row0 + ln]) : int64_t(row0 + ln);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 16 * tn + 4 * lg + i;
                const int o = o0 + r;
                if (o < p.OUT) {
                    const float v = ((alive[tn] >> (r - 16 * tn)) & 1) ? acc[tn][i] : 0.f;
                    store_act(p.y, p.y_type, yoff + yr * p.OUT + o, v);
                }
            }
        }
    }
}

// Persistent form of k_seg_mfma for sorted expert tiles over a d8 table
// beyond LDS (the MTP-verify shape: a few pairs per expert, hundreds of
// experts). One workgroup per CU stages the table's LDS part once and then
// walks its items -- (tile, 128-row block) pairs, item i of workgroup b is
// b + i * gridDim.x -- as one flat sequence of K supersteps. Every step loads
// the next step's weights and x (of the next item when this one ends) before
// it multiplies, so neither the table copy nor an item's first memory latency
// stalls the CU, as they do once per workgroup in k_seg_mfma (for a 1024-wide
// down projection an item is a single superstep). An item's context -- its
// weight rows through the skipzero row table, its token rows through the
// sort order -- is resolved two items ahead and its tile record loaded three
// ahead; each step issues those loads (discarded unless an item ends) so that
// every step sends the same loads and the compiler's load-count waits never
// stall a step on the prefetch issued in it.
template <int BITS, int GPB, int TOK, int NW>
__device__ __forceinline__ void seg_persist_body(const SegParams &p, int ntiles) {
    constexpr int D = 8;
    constexpr int NT = NW * 64;                 // threads
    constexpr int ROWS = NW * 32;               // weight rows per item
    constexpr int TN = 2;                       // 16-row tiles per wave
    constexpr int SPB = 4 * D;                  // MFMA steps per block
    constexpr int CC = 128 * D;                 // x columns per superstep
    constexpr int XS = CC + 8;                  // LDS row stride of the x chunk (halves)
    constexpr int PIECES = TOK * CC / 8;        // 16-byte pieces per chunk
    constexpr int PPT = PIECES / NT;
    static_assert(PIECES % NT == 0, "chunk must split evenly over the threads");
    constexpr int CBN = seg_hyb_entries(D, TOK);
    static_assert(TOK * XS * 2 + (CBN + 1) * D * 2 <= 160 * 1024, "LDS beyond 160 KB");

    extern __shared__ __align__(16) uint8_t smem[];
    f16 *xs = reinterpret_cast<f16 *>(smem);    // [TOK][XS]
    f16 *cbl = xs + TOK * XS;                   // [CBN + 1][D]; entry CBN is zero

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 15, lg = lane >> 4;
    const int nxb = (p.OUT + ROWS - 1) / ROWS;
    const int items = ntiles * nxb;             // uniform
    const int G = int(gridDim.x), i0 = int(blockIdx.x);
    if (i0 >= items) return;                    // uniform, before any barrier
    const int mine = (items - i0 + G - 1) / G;
    const int NSS = (p.NB + 3) >> 2;
    const int steps = mine * NSS;
    const uint32_t kmax = uint32_t(p.K - 1);

    {
        const int ent = min(p.K, CBN);
        lds_copy_async(p.codebook, cbl, ent * D * 2, (CBN + 1) * D * 2);
    }

    struct Meta { int e, row0, nrows, xb; };
    struct Ctx {
        int64_t cr[TN];       // this lane's stored weight row per row tile, or -1
        int64_t xoff[PPT];    // x element offset of each x piece's token row, or -1
        int64_t yrow;         // output row of token ln, or -1
        int o0, nrows;
    };
    // tile record of this workgroup's item m (none past the last: no rows)
    auto meta = [&](int m) {
        Meta r{-1, 0, 0, 0};
        if (m < mine) {
            const int it = i0 + m * G;
            const int32_t *tm = p.tmeta + 3 * (it / nxb);
            r.e = tm[0];
            r.row0 = tm[1];
            r.nrows = tm[2];
            r.xb = it % nxb;
        }
        return r;
    };
    auto resolve = [&](const Meta &m) {
        Ctx c;
        c.o0 = m.xb * ROWS + wave * 32;
        c.nrows = m.nrows;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const int o = c.o0 + 16 * tn + ln;
            int64_t f = -1;
            if (m.e >= 0 && m.e < p.E && o < p.OUT) {
                f = int64_t(m.e) * p.OUT + o;
                if (p.row_table) f = p.row_table[f];
                if (f < 0 || f >= p.stored_rows) f = -1;
            }
            c.cr[tn] = f;
        }
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const int t = (tid + NT * r) / (CC / 8);
            c.xoff[r] = t < m.nrows ? int64_t(p.order[m.row0 + t] / p.xkrep) * p.IN : int64_t(-1);
        }
        c.yrow = ln < m.nrows ? int64_t(p.order[m.row0 + ln]) : int64_t(-1);
        return c;
    };

    auto load_x = [&](const Ctx &c, int sb, u32x4 (&v)[PPT]) {
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const int col = sb * CC + ((tid + NT * r) % (CC / 8)) * 8;
            const bool ok = c.xoff[r] >= 0 && col < p.IN;
            if (p.xg) {
                v[r] = ok ? swiglu8(p.xg + c.xoff[r] + col, p.xu + c.xoff[r] + col) : u32x4{0, 0, 0, 0};
            } else {
                v[r] = ok ? load8_act(p.x, p.x_type, c.xoff[r] + col) : u32x4{0, 0, 0, 0};
            }
        }
    };
    auto store_x = [&](const u32x4 (&v)[PPT]) {
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const int pc = tid + NT * r;
            *reinterpret_cast<u32x4 *>(xs + (pc / (CC / 8)) * XS + (pc % (CC / 8)) * 8) = v[r];
        }
    };
    auto load_w = [&](const Ctx &c, int sb, uint32_t (&w)[TN][BITS], h2 (&s)[TN][GPB],
                      bool (&live)[TN]) {
        const int b = 4 * sb + lg;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            live[tn] = c.cr[tn] >= 0 && b < p.NB;
            if (live[tn]) {
                const uint32_t *src = p.codes + c.cr[tn] * p.row_words + int64_t(b) * BITS;
#pragma unroll
                for (int i = 0; i < BITS; ++i) w[tn][i] = src[i];
                const uint16_t *sr = p.scales + c.cr[tn] * p.ngrp + (GPB == 1 ? b / p.bpg : b * GPB);
#pragma unroll
                for (int g = 0; g < GPB; ++g) {
                    const f16 v = __builtin_bit_cast(f16, sr[g]);
                    s[tn][g] = h2{v, v};
                }
            } else {
#pragma unroll
                for (int i = 0; i < BITS; ++i) w[tn][i] = 0u;
#pragma unroll
                for (int g = 0; g < GPB; ++g) s[tn][g] = h2{0, 0};
            }
        }
    };

    f32x4 acc[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tn] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const uint32_t (&w)[TN][BITS], const h2 (&s)[TN][GPB],
                       const bool (&live)[TN]) {
        // MFMA column ln is token ln; with TOK < 16 the columns past the tile
        // repeat its rows and their sums are never stored
        const f16 *xb = xs + (ln & (TOK - 1)) * XS + lg * (32 * D);
        const f16 *tab[TN];
        uint32_t kl[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            tab[tn] = live[tn] ? cbl : cbl + CBN * D;        // dead lanes: code 0 -> zero entry
            kl[tn] = live[tn] ? uint32_t(min(p.K, CBN)) : 1u;
        }
        const f16 *tg = reinterpret_cast<const f16 *>(p.codebook);
#pragma unroll
        for (int st = 0; st < SPB; ++st) {
            const h8 xf = *reinterpret_cast<const h8 *>(xb + 8 * st);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int q = (st * GPB) / (4 * D);
                const h8 e = step_entries_hyb<D, BITS>(w[tn], st, tab[tn], tg, kl[tn], kmax);
                const h2 sc = s[tn][q];
                const h8 wv = e * h8{sc[0], sc[0], sc[0], sc[0], sc[0], sc[0], sc[0], sc[0]};
                acc[tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv, xf, acc[tn], 0, 0, 0);
            }
        }
    };
    // lane holds rows 16*tn + 4*lg + i of token ln
    auto epilogue = [&](const Ctx &c) {
        uint64_t alive[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) alive[tn] = __ballot(c.cr[tn] >= 0);
        if (ln < c.nrows) {
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 16 * tn + 4 * lg + i;
                    const int o = c.o0 + r;
                    if (o < p.OUT) {
                        const float v = ((alive[tn] >> (r - 16 * tn)) & 1) ? acc[tn][i] : 0.f;
                        store_act(p.y, p.y_type, c.yrow * p.OUT + o, v);
                    }
                }
            }
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tn] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // context pipeline: c0 = item m, c1 = item m + 1 (resolved), m2 = item m + 2
    int m = 0, sb = 0;
    Ctx c0 = resolve(meta(0));
    Ctx c1 = resolve(meta(1));
    Meta m2 = meta(2);

    uint32_t w0[TN][BITS], w1[TN][BITS];
    h2 s0[TN][GPB], s1[TN][GPB];
    bool l0[TN], l1[TN];
    u32x4 xr[PPT];

    load_x(c0, 0, xr);
    load_w(c0, 0, w0, s0, l0);
    store_x(xr);
    wait_vmem();                                // table part and the first chunk
    __syncthreads();

    // one step on buffers (wc, sc, lc), prefetching into (wn, sn, lnx);
    // false after the last step
    auto step = [&](int j, const uint32_t (&wc)[TN][BITS], const h2 (&sc)[TN][GPB],
                    const bool (&lc)[TN], uint32_t (&wn)[TN][BITS], h2 (&sn)[TN][GPB],
                    bool (&lnx)[TN]) {
        const bool last = sb + 1 == NSS;        // this item's last superstep
        const bool more = j + 1 < steps;
        Ctx c2 = c1;
        Meta m3 = m2;
        if (more) {
            c2 = resolve(m2);                   // kept only if this item ends
            m3 = meta(m + 3);
            load_x(last ? c1 : c0, last ? 0 : sb + 1, xr);
            load_w(last ? c1 : c0, last ? 0 : sb + 1, wn, sn, lnx);
        }
        compute(wc, sc, lc);
        if (last) {
            epilogue(c0);
            c0 = c1;
            c1 = c2;
            m2 = m3;
            ++m;
            sb = 0;
        } else {
            ++sb;
        }
        if (!more) return false;
        __syncthreads();                        // every wave is done with this chunk
        store_x(xr);
        __syncthreads();                        // the next chunk is in place
        return true;
    };
    for (int j = 0;; j += 2) {
        if (!step(j, w0, s0, l0, w1, s1, l1)) break;
        if (!step(j + 1, w1, s1, l1, w0, s0, l0)) break;
    }
}

// The persistent kernel over narrow tiles, with the tile size the sort chose
// for this routing: the tile count and that size, read as one 8-byte load
// (ntiles[1]: kSegTokMid, else kSegTokNarrow).
template <int BITS, int GPB, int NW = kPersistWaves>
__global__ void __launch_bounds__(NW * 64) k_seg_persist(const SegParams p) {
    const int2 nt = *reinterpret_cast<const int2 *>(p.ntiles);
    if (nt.y == kSegTokMid) seg_persist_body<BITS, GPB, kSegTokMid, NW>(p, nt.x);
    else seg_persist_body<BITS, GPB, kSegTokNarrow, NW>(p, nt.x);
}

// LDS bytes of k_seg_mfma<D, BITS, GPB, cbl, tok>.
__host__ __device__ constexpr size_t seg_lds(int D, int BITS, bool cbl, int tok = kSegTok) {
    return size_t(tok) * (128 * D + 8) * 2 +
           (size_t(cbl ? (1 << BITS) : seg_hyb_entries(D, tok)) + 1) * D * 2;
}

// Launches k_seg_mfma for geometry-dependent template arguments; returns a
// VQK status (VQK_ENOTIMPL when no instance matches).
int launch_seg_d2(const SegParams &p, int bits, int gpb, dim3 grid, hipStream_t st);
int launch_seg_d4(const SegParams &p, int bits, int gpb, dim3 grid, hipStream_t st);
// Tiles of at most 16 rows (tok == kSegTok; sorted narrow tiles run
// launch_seg_persist_d8).
int launch_seg_d8(const SegParams &p, int bits, int gpb, int tok, dim3 grid, hipStream_t st);
// k_seg_persist (sorted narrow tiles of <= 4 or <= 8 rows as the sort chose,
// d8 tables beyond LDS) on `grid` workgroups.
int launch_seg_persist_d8(const SegParams &p, int bits, int gpb, dim3 grid, hipStream_t st);

}  // namespace vqk
