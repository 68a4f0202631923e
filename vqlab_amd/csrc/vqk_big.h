// GEMV for codebooks larger than LDS (config 3: d8 K16384 = 256 KB).
//
// Gathering each code's entry from L2 costs one random 16-byte request per
// code, and the L2 serves about one such request every three clocks per CU:
// that, not HBM, capped the block-per-lane GEMV at ~0.4 TB/s on these
// tables. Here the table goes through LDS in 128 KB slices instead. A
// workgroup loads ALL its code blocks into registers first (up to S row
// steps per lane), then for each slice: stream the slice into LDS with
// direct-to-LDS copies (full 128-byte lines, ~16 B of L2 traffic per code
// for a two-slice table), and add the contributions of the codes that fall in
// the slice (the others read a zero entry). Per-group sums are linear in the
// codes, so the slices' partial dot products simply add.
//
// One launch serves up to four "segments" (e.g. routed gate, routed up,
// shared gate, shared up) of the same format and input width. Work items are
// (segment, pair, range of rows) in the block-per-lane layout of the fast
// GEMV (LPR lanes per row); each workgroup runs a contiguous range of items
// and takes the slices of an item in an order that starts with the slice the
// previous item left in LDS, so a two-slice table costs one staging per item. The x row
// is staged once into LDS as fp16 — or, for a down projection, built there as
// silu(g) * u from the fp32 gate/up outputs — and each lane keeps its
// 32*D-value slice in registers.
#pragma once

#include "vqk_gemv.h"

namespace vqk {

constexpr int kBigThreads = 256;                 // 4 waves; one workgroup per CU (LDS)
constexpr int kBigSliceBytes = 128 * 1024;       // codebook slice staged per pass
constexpr int kBigSteps = 4;                     // row steps held in registers per lane
constexpr int kBigMaxSeg = 4;

struct BigSeg {
    const uint32_t *codes;     // code rows of 32-code blocks
    int64_t row_words;
    const uint16_t *codebook;  // fp16 [K, D]
    int32_t K;
    const uint16_t *scales;
    int32_t ngrp, bpg;
    const int32_t *row_table;
    int64_t stored_rows;
    int32_t E, OUT;
    const int32_t *eidx;       // expert of each pair (NULL: expert 0)
    int32_t N, xkrep;          // pairs; x row of pair n = n / xkrep
    const void *x;             // activations, x_type
    int32_t x_type;
    const float *xg, *xu;      // if xg: x row = fp16(silu(xg) * xu), fp32 rows
    int64_t x_stride;          // elements between x rows
    void *y;                   // y[n * y_stride + r], y_type
    int32_t y_type;
    int64_t y_stride;
    int32_t wg0, wg_per_pair, rows_per_wg;
};

struct BigParams {
    BigSeg seg[kBigMaxSeg];
    int32_t nseg;
    int32_t IN, NB, lpr_log2, steps;
};

// sum_g s[g] * sum_{codes i of g in the slice} <cb[c_i - base], x_i>; codes
// outside [base, base + cnt) read the zero entry `zero` (branch-free, so the
// gathers of a block can all be in flight together).
// All 32 entry reads are issued before the first product (a scheduling
// barrier keeps the compiler from interleaving them with the dot chain): at
// one wave per SIMD nothing else hides an LDS read's latency, and 32 reads in
// flight per lane run the random gathers near the LDS's rate.
template <int D, int BITS, int GPB>
__device__ __forceinline__ float block_dot_slice(const uint32_t (&w)[BITS], const h2 (&xr)[16 * D],
                                                 const float (&s)[GPB], const h2 *cb,
                                                 uint32_t base, uint32_t cnt, uint32_t zero) {
    typedef typename EntryT<D>::type E;
    constexpr int CPG = kBlock / GPB;
    E e[kBlock];
#pragma unroll
    for (int i = 0; i < kBlock; ++i) {
        uint32_t c = block_field<BITS>(w, i) - base;               // wraps below base
        c = c < cnt ? c : zero;
        e[i] = reinterpret_cast<const E *>(cb)[c];
    }
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

template <int D, int BITS, int GPB>
__global__ void __launch_bounds__(kBigThreads) k_gemv_big(const BigParams p) {
    constexpr int SE = kBigSliceBytes / (2 * D);     // entries per slice
    constexpr int XH = kBlock * D;                   // x values per block
    constexpr int S = kBigSteps;
    constexpr int NWV = kBigThreads / kWave;
    constexpr int CBB = ((SE + 1) * D * 2 + 15) & ~15;              // slice + zero entry, 16-B padded
    extern __shared__ __align__(16) uint8_t smem[];
    h2 *cbl = reinterpret_cast<h2 *>(smem);                          // [SE + 1][D]
    f16 *xs = reinterpret_cast<f16 *>(smem + CBB);                   // [IN]

    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
    const int lpr = 1 << p.lpr_log2, rpw = kWave >> p.lpr_log2;
    const int sub = lane >> p.lpr_log2, blk = lane & (lpr - 1);
    const bool on = blk < p.NB;

    // a contiguous range of work items (segment, pair, row chunk) per
    // workgroup, so consecutive items share a codebook and the slice left in
    // LDS by one item is the first the next one uses
    const int items = p.seg[p.nseg - 1].wg0 + p.seg[p.nseg - 1].N * p.seg[p.nseg - 1].wg_per_pair;
    const int per = (items + int(gridDim.x) - 1) / int(gridDim.x);
    const int it0 = int(blockIdx.x) * per, it1 = min(items, it0 + per);
    const uint16_t *held_cb = nullptr;               // codebook whose slice `held` is in LDS
    int held = -1;
    int prev_x = -1, prev_seg = -1;

    for (int it = it0; it < it1; ++it) {
        int si = 0;
#pragma unroll
        for (int i = 1; i < kBigMaxSeg; ++i)
            if (i < p.nseg && it >= p.seg[i].wg0) si = i;
        const BigSeg &sg = p.seg[si];
        const int local = it - sg.wg0;
        const int n = local / sg.wg_per_pair, chunk = local % sg.wg_per_pair;
        int64_t e = 0;
        if (sg.eidx) {
            const int id = sg.eidx[n];
            e = (id >= 0 && id < sg.E) ? id : -1;
        }
        const int r0 = chunk * sg.rows_per_wg;
        auto row_at = [&](int s) { return r0 + (s * NWV + wave) * rpw + sub; };

        // every code block this lane uses for the item, before anything waits
        uint32_t w[S][BITS];
        uint32_t sc[S][GPB];     // raw fp16 bits: converted at use, so the S loads overlap
        bool live[S];
        const int sidx = GPB == 1 ? blk / sg.bpg : blk * GPB;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int r = row_at(s);
            int64_t cr = -1;
            if (s < p.steps && on && e >= 0 && r < sg.OUT) {
                cr = e * sg.OUT + r;
                if (sg.row_table) cr = sg.row_table[cr];
                if (cr < 0 || cr >= sg.stored_rows) cr = -1;
            }
            live[s] = cr >= 0;
            if (cr >= 0) {
                // plain loads: the vector L1 serves the block loads' repeated
                // segments (config 3 at batch 4: 0.731 -> 0.703 ms)
                const uint32_t *src = sg.codes + cr * sg.row_words + int64_t(blk) * BITS;
#pragma unroll
                for (int i = 0; i < BITS; ++i) w[s][i] = src[i];
                const uint16_t *sr = sg.scales + cr * sg.ngrp + sidx;
#pragma unroll
                for (int g = 0; g < GPB; ++g) sc[s][g] = __builtin_nontemporal_load(sr + g);
            } else {
#pragma unroll
                for (int i = 0; i < BITS; ++i) w[s][i] = 0u;
#pragma unroll
                for (int g = 0; g < GPB; ++g) sc[s][g] = 0u;
            }
        }

        // the pair's x row -> LDS as fp16 (plain, or silu(g) * u), when it changed
        const int xr_id = n / sg.xkrep;
        if (xr_id != prev_x || si != prev_seg) {
            __syncthreads();                             // every wave is done with the old row
            const int64_t xrow = int64_t(xr_id) * sg.x_stride;
            for (int i8 = tid; i8 < p.IN / 8; i8 += kBigThreads) {
                u32x4 v;
                if (sg.xg) {
                    uint16_t h[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float gv = sg.xg[xrow + i8 * 8 + u], uv = sg.xu[xrow + i8 * 8 + u];
                        h[u] = f32_to_h(gv / (1.f + __expf(-gv)) * uv);
                    }
                    v = u32x4{uint32_t(h[0]) | (uint32_t(h[1]) << 16),
                              uint32_t(h[2]) | (uint32_t(h[3]) << 16),
                              uint32_t(h[4]) | (uint32_t(h[5]) << 16),
                              uint32_t(h[6]) | (uint32_t(h[7]) << 16)};
                } else {
                    v = load8_act(sg.x, sg.x_type, xrow + i8 * 8);
                }
                *reinterpret_cast<u32x4 *>(xs + i8 * 8) = v;
            }
            prev_x = xr_id;
            prev_seg = si;
        }

        // slices in an order that starts with the one already in LDS
        const int npass = (sg.K + SE - 1) / SE;
        const int first = (held_cb == sg.codebook && held >= 0 && held < npass) ? held : 0;
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.f;
        h2 xr[16 * D];
        for (int q = 0; q < npass; ++q) {
            const int pass = (first + q) % npass;
            if (held_cb != sg.codebook || held != pass) {
                __syncthreads();                         // every wave is done with the old slice
                const int base = pass * SE;
                lds_copy_async(sg.codebook + int64_t(base) * D, cbl, min(SE, sg.K - base) * D * 2, CBB);
                held_cb = sg.codebook;
                held = pass;
            }
            wait_vmem();
            __syncthreads();
            if (q == 0) load_xregs<D>(xs + (on ? blk : 0) * XH, xr);
            const uint32_t base = uint32_t(pass * SE);
            const uint32_t cnt = uint32_t(min(SE, sg.K - pass * SE));
#pragma unroll
            for (int s = 0; s < S; ++s)
                if (live[s]) acc[s] += block_dot_slice<D, BITS, GPB>(w[s], xr, ScalesF32<GPB>(sc[s]).v, cbl, base, cnt, SE);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (s >= p.steps) break;
            const float v = group_sum(acc[s], lpr);
            const int r = row_at(s);
            if (blk == lpr - 1 && r < sg.OUT)
                store_act(sg.y, sg.y_type, int64_t(n) * sg.y_stride + r, v);
        }
    }
}

__host__ __device__ constexpr size_t big_lds(int D, int64_t IN) {
    return ((size_t(kBigSliceBytes / (2 * D) + 1) * D * 2 + 15) & ~size_t(15)) + size_t(IN) * 2;
}

int launch_gemv_big(const BigParams &p, int D, int bits, int gpb, dim3 grid, hipStream_t st);

// Fills the weight fields of a segment from a validated module.
void big_seg_weights(const vqk_weights *w, const Geom &g, BigSeg *s);

// Rows per work item for OUT rows of NB blocks, total_rows over all items of
// the launch; sets p->lpr_log2 / p->steps. Returns the rows per item.
int big_plan_rows(BigParams *p, int64_t NB, int64_t OUT, int64_t total_rows);

// Workgroups to launch for `items` work items (one per CU at most).
int big_grid(int64_t items);

// True when the sliced-codebook GEMV takes this module (table beyond the
// LDS-resident limit, block-per-lane shape, LDS room for the x row).
bool big_fits(const Geom &g, const vqk_weights *w);

}  // namespace vqk
