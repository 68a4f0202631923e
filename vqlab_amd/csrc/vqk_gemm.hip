// Matrix-core VQ GEMMs: the large-N paths.
//
//   vqk_dense_gemm     _decode_matmul (vq_dense.py:262-312): y = x . W^T, E = 1
//   vqk_grouped_gemm   _gemmseg_prefill (vq_switch.py:4569-4722): routed pairs
//                      count-sorted by expert on device, one tile per <= BM
//                      rows of an expert segment (the reference's tmeta,
//                      vq_switch.py:4590-4610), results in caller order
//
// Each workgroup owns a BM x BN output tile. Per K-step of 64 input columns it
// stages the x rows (fp16) and DECODES the matching 64-column slice of BN
// weight rows into LDS -- W[o, k] = fp16(f32(cb[c]) * f32(s)), the bit-exact
// dequant -- then runs v_mfma_f32_32x32x16_f16 over the two tiles with fp32
// accumulation. No fp16 weight is ever materialised in HBM. Operand layout
// (checked on gfx950): lane l feeds A[l%32][8*(l/32) .. +8] and
// B[8*(l/32) .. +8][l%32]; accumulator register i holds row
// 8*(i/4) + 4*(l/32) + i%4, column l%32.
#include "vqk_gemv.h"
#include "vqk_gseg.h"
#include "vqk_internal.h"

namespace vqk {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;             // input columns per K-step (one 64-weight scale group)
constexpr int kLdsStride = kBK + 8; // halves per staged row (16 B skew)

struct GemmParams {
    const void *codes;
    int64_t code_cols;      // row stride in code units (u32 words when packed)
    int32_t bits;           // packed width, 0 = unpacked
    int32_t code_bytes;     // 1 / 2 when unpacked
    const uint16_t *codebook;
    int32_t K;
    const uint16_t *scales;
    int32_t ngrp, G;
    const int32_t *row_table;
    int64_t stored_rows;
    int32_t E, OUT, IN, NSUB;
    const void *x;
    int32_t x_type, xkrep;
    void *y;
    int32_t y_type;
    int32_t N;              // dense: rows of x; grouped: pairs
    const int32_t *tmeta;   // grouped: [max_tiles, 3] (expert or -1, row_start, nrows)
    const int32_t *ntiles;  // grouped: tiles actually built
    const int32_t *order;   // grouped: sorted position -> pair index
    const uint32_t *eidx;   // grouped: expert of each pair
};

__device__ __forceinline__ uint32_t gemm_code(const GemmParams &p, int64_t cr, int j) {
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

// BM x BN output tile, WM x WN waves, each wave (BM/WM) x (BN/WN) = TM x TN
// MFMA 32x32 tiles. CBL: codebook staged in LDS (K*D*2 bytes, dynamic).
template <int D, bool CBL, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) k_vq_gemm(const GemmParams p) {
    constexpr int NT = 64 * WM * WN;
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
    constexpr int CPR = kBK / D;                      // codes per weight row per K-step
    static_assert(TM >= 1 && TN >= 1, "tile too small for the wave grid");
    extern __shared__ __align__(16) uint8_t smem[];
    f16 *As = reinterpret_cast<f16 *>(smem);                         // [BM][kLdsStride]
    f16 *Bs = As + BM * kLdsStride;                                  // [BN][kLdsStride]
    uint16_t *cbs = reinterpret_cast<uint16_t *>(Bs + BN * kLdsStride);  // [K][D] if CBL

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int o0 = int(blockIdx.x) * BN;

    // ---- the row block of this tile
    int expert, row0, nrows;
    const bool grouped = p.tmeta != nullptr;
    if (grouped) {
        if (int(blockIdx.y) >= *p.ntiles) return;                   // uniform: no barrier passed yet
        const int32_t *tm = p.tmeta + 3 * blockIdx.y;
        expert = tm[0];
        row0 = tm[1];
        nrows = tm[2];
    } else {
        expert = 0;
        row0 = int(blockIdx.y) * BM;
        nrows = min(BM, p.N - row0);
    }
    if constexpr (CBL) {
        lds_copy_async(p.codebook, cbs, p.K * D * 2, p.K * D * 2);
        wait_vmem();
        __syncthreads();
    }
    const uint16_t *cb = CBL ? cbs : p.codebook;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x16{};

    // x row (element offset) of tile row m, or -1
    auto xrow = [&](int m) -> int64_t {
        if (m >= nrows) return -1;
        if (!grouped) return int64_t(row0 + m) * p.IN;
        const int pair = p.order[row0 + m];
        return int64_t(pair / p.xkrep) * p.IN;
    };
    // code row of weight row o of this tile's expert, or -1 (dead / outside)
    auto wrow = [&](int o) -> int64_t {
        if (expert < 0 || o >= p.OUT) return -1;
        int64_t f = int64_t(expert) * p.OUT + o;
        if (p.row_table) f = p.row_table[f];
        return f < p.stored_rows ? f : -1;
    };

    for (int k0 = 0; k0 < p.IN; k0 += kBK) {
        // ---- stage x: BM rows x 64 columns, 8 values per thread per round
        for (int c = tid; c < BM * (kBK / 8); c += NT) {
            const int m = c / (kBK / 8), kc = (c % (kBK / 8)) * 8;
            const int64_t base = xrow(m);
            u32x4 v = {0, 0, 0, 0};
            if (base >= 0) {
                if (k0 + kc + 8 <= p.IN && ((reinterpret_cast<uintptr_t>(p.x) +
                                             uint64_t(base + k0 + kc) * (p.x_type == VQK_F32 ? 4 : 2)) & 15) == 0) {
                    v = load8_act(p.x, p.x_type, base + k0 + kc);
                } else {
                    uint16_t h[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        h[u] = k0 + kc + u < p.IN ? f32_to_h(load_act(p.x, p.x_type, base + k0 + kc + u)) : 0;
                    v = u32x4{uint32_t(h[0]) | (uint32_t(h[1]) << 16), uint32_t(h[2]) | (uint32_t(h[3]) << 16),
                              uint32_t(h[4]) | (uint32_t(h[5]) << 16), uint32_t(h[6]) | (uint32_t(h[7]) << 16)};
                }
            }
            *reinterpret_cast<u32x4 *>(As + m * kLdsStride + kc) = v;
        }
        // ---- decode W: BN rows x CPR codes, D halves each, bit-exact dequant
        for (int c = tid; c < BN * CPR; c += NT) {
            const int r = c / CPR, jj = c % CPR;
            const int j = k0 / D + jj;
            const int64_t cr = wrow(o0 + r);
            uint16_t h[D];
            if (cr >= 0 && j < p.NSUB) {
                const uint32_t code = min(gemm_code(p, cr, j), uint32_t(p.K - 1));
                const float s = h_to_f32(p.scales[cr * p.ngrp + (j * D) / p.G]);
                const uint16_t *e = cb + int64_t(code) * D;
#pragma unroll
                for (int u = 0; u < D; ++u) h[u] = f32_to_h(s * h_to_f32(e[u]));
            } else {
#pragma unroll
                for (int u = 0; u < D; ++u) h[u] = 0;
            }
            f16 *dst = Bs + r * kLdsStride + jj * D;
            if constexpr (D == 2) {
                *reinterpret_cast<uint32_t *>(dst) = uint32_t(h[0]) | (uint32_t(h[1]) << 16);
            } else if constexpr (D == 4) {
                *reinterpret_cast<u32x2 *>(dst) = u32x2{uint32_t(h[0]) | (uint32_t(h[1]) << 16),
                                                         uint32_t(h[2]) | (uint32_t(h[3]) << 16)};
            } else {
                *reinterpret_cast<u32x4 *>(dst) = u32x4{uint32_t(h[0]) | (uint32_t(h[1]) << 16),
                                                         uint32_t(h[2]) | (uint32_t(h[3]) << 16),
                                                         uint32_t(h[4]) | (uint32_t(h[5]) << 16),
                                                         uint32_t(h[6]) | (uint32_t(h[7]) << 16)};
            }
        }
        __syncthreads();
        // ---- matrix cores: 4 sub-steps of 16 columns
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            h8 af[TM], bf[TN];
            const int kof = kk + (lane >> 5) * 8;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int m = (wm * TM + a) * 32 + (lane & 31);
                af[a] = *reinterpret_cast<const h8 *>(As + m * kLdsStride + kof);
            }
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int n = (wn * TN + b) * 32 + (lane & 31);
                bf[b] = *reinterpret_cast<const h8 *>(Bs + n * kLdsStride + kof);
            }
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }

    // ---- epilogue: rows back to caller order
#pragma unroll
    for (int a = 0; a < TM; ++a) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = (wm * TM + a) * 32 + (i / 4) * 8 + (lane >> 5) * 4 + (i % 4);
            if (m >= nrows) continue;
            const int64_t yr = grouped ? int64_t(p.order[row0 + m]) : int64_t(row0 + m);
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int o = o0 + (wn * TN + b) * 32 + (lane & 31);
                if (o < p.OUT) store_act(p.y, p.y_type, yr * p.OUT + o, acc[a][b][i]);
            }
        }
    }
}

// ---------------------------------------------------------------- sorting
// One workgroup: histogram of the pairs' experts (bucket E = ids outside
// [0, E): their rows decode to zero), exclusive scans of the counts and of
// the tile counts, scatter of pair indices into expert order, and one
// (expert, row_start, nrows) record per tile of <= BM rows, experts ascending
// (the reference's tile metadata, vq_switch.py:4590-4610). Within an expert
// the order of pairs follows the atomics; every output row is computed
// independently, so the results do not depend on it.
constexpr int kSortThreads = 1024;

__device__ __forceinline__ void block_exclusive_scan(int *a, int n, int *tmp) {
    // a[0..n) in LDS, n <= 4 * kSortThreads; tmp has kSortThreads ints
    const int tid = threadIdx.x;
    const int per = (n + kSortThreads - 1) / kSortThreads;
    int local = 0;
    for (int i = 0; i < per; ++i) {
        const int k = tid * per + i;
        if (k < n) local += a[k];
    }
    tmp[tid] = local;
    __syncthreads();
    for (int off = 1; off < kSortThreads; off <<= 1) {
        const int v = tid >= off ? tmp[tid - off] : 0;
        __syncthreads();
        tmp[tid] += v;
        __syncthreads();
    }
    int run = tmp[tid] - local;                 // exclusive prefix of this thread's chunk
    for (int i = 0; i < per; ++i) {
        const int k = tid * per + i;
        if (k < n) {
            const int v = a[k];
            a[k] = run;
            run += v;
        }
    }
    __syncthreads();
}

__global__ void __launch_bounds__(kSortThreads) k_group_sort(const uint32_t *eidx, int N, int E,
                                                             int BM, int max_tiles, int32_t *order,
                                                             int32_t *tmeta, int32_t *ntiles) {
    extern __shared__ int sh[];
    const int NBK = E + 1;
    int *cnt = sh;                 // [NBK] counts, then starts
    int *tls = cnt + NBK;          // [NBK] tiles per bucket, then tile starts
    int *cur = tls + NBK;          // [NBK] scatter cursors
    int *tmp = cur + NBK;          // [kSortThreads]
    int *red = tmp + kSortThreads; // [2] tile totals of the two narrow sizes
    const int tid = threadIdx.x;
    for (int b = tid; b < NBK; b += kSortThreads) cnt[b] = 0;
    if (tid < 2) red[tid] = 0;
    __syncthreads();
    for (int n = tid; n < N; n += kSortThreads) {
        const uint32_t e = eidx[n];
        atomicAdd(&cnt[e < uint32_t(E) ? int(e) : E], 1);
    }
    __syncthreads();
    if (BM == kSegTokNarrow) {
        // narrow tiles: 8 rows where that cuts the tile count (every tile
        // decodes its expert's weights once) by more than the ~5 % that the
        // 8-row tile's smaller LDS part of the table costs per tile
        int t4 = 0, t8 = 0;
        for (int b = tid; b < NBK; b += kSortThreads) {
            t4 += (cnt[b] + kSegTokNarrow - 1) / kSegTokNarrow;
            t8 += (cnt[b] + kSegTokMid - 1) / kSegTokMid;
        }
        for (int o = 32; o >= 1; o >>= 1) {     // wave sums, then one add per wave
            t4 += __shfl_xor(t4, o);
            t8 += __shfl_xor(t8, o);
        }
        if ((tid & 63) == 0) {
            atomicAdd(&red[0], t4);
            atomicAdd(&red[1], t8);
        }
        __syncthreads();
        if (21 * red[1] < 20 * red[0]) BM = kSegTokMid;
    }
    for (int b = tid; b < NBK; b += kSortThreads) tls[b] = (cnt[b] + BM - 1) / BM;
    __syncthreads();
    // keep the counts: cur = counts for now
    for (int b = tid; b < NBK; b += kSortThreads) cur[b] = cnt[b];
    __syncthreads();
    block_exclusive_scan(cnt, NBK, tmp);       // cnt -> bucket starts
    block_exclusive_scan(tls, NBK, tmp);       // tls -> tile starts
    for (int b = tid; b < NBK; b += kSortThreads) {
        const int c = cur[b];
        const int nt = (c + BM - 1) / BM;
        for (int t = 0; t < nt; ++t) {
            const int ti = tls[b] + t;
            if (ti < max_tiles) {
                tmeta[3 * ti + 0] = b < E ? b : -1;
                tmeta[3 * ti + 1] = cnt[b] + t * BM;
                tmeta[3 * ti + 2] = min(BM, c - t * BM);
            }
        }
        if (b == NBK - 1) {
            ntiles[0] = min(max_tiles, tls[b] + nt);
            ntiles[1] = BM;                    // the tile rows chosen
        }
    }
    __syncthreads();
    for (int b = tid; b < NBK; b += kSortThreads) cur[b] = cnt[b];
    __syncthreads();
    for (int n = tid; n < N; n += kSortThreads) {
        const uint32_t e = eidx[n];
        const int pos = atomicAdd(&cur[e < uint32_t(E) ? int(e) : E], 1);
        order[pos] = n;
    }
}

// ---------------------------------------------------------------- host
constexpr int kGroupBM = 32, kGroupBN = 128;   // fallback tile kernel (tiles hold <= kSegTok rows)
constexpr int kMaxSortExperts = 4096;
constexpr int kSegDenseMaxN = 64;               // dense rows up to which the segment kernel runs

static size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

// Tiles of <= tok sorted rows: sum over experts of ceil(count / tok) is at
// most ceil(N / tok) + (non-empty buckets).
static int64_t group_max_tiles(int64_t N, int64_t E, int tok) {
    return (N + tok - 1) / tok + (N < E + 1 ? N : E + 1);
}

// The register-decode segment kernel covers whole 32-code blocks per row
// (rows of NB * BITS words), BITS 2..16, the GEMV's scale-group layouts and
// 16-byte aligned codebook and activations.
static bool seg_fits_geom(const Geom &g, const vqk_weights *w) {
    const int gpb_fast = g.D == 4 ? 2 : (g.D == 8 ? 4 : 1);
    return (g.D == 2 || g.D == 4 || g.D == 8) && g.NSUB % kBlock == 0 && g.row_words > 0 &&
           g.row_words == g.NB * g.BITS && g.BITS >= 2 && g.BITS <= 16 &&
           (g.gpb == 1 || g.gpb == gpb_fast) && g.IN <= INT32_MAX && g.OUT <= INT32_MAX &&
           (reinterpret_cast<uintptr_t>(w->codebook) & 15) == 0;
}

static bool seg_fits(const Geom &g, const vqk_weights *w, const void *x) {
    return seg_fits_geom(g, w) && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

static void fill_seg(const vqk_weights *w, const Geom &g, SegParams *p) {
    memset(p, 0, sizeof *p);
    p->codes = static_cast<const uint32_t *>(w->codes);
    p->row_words = g.row_words;
    p->codebook = w->codebook;
    p->K = int32_t(g.K);
    p->scales = w->scales;
    p->ngrp = int32_t(g.NGRP);
    p->bpg = g.bpg;
    p->row_table = w->row_table;
    p->stored_rows = g.rows;
    p->E = int32_t(g.E);
    p->OUT = int32_t(g.OUT);
    p->IN = int32_t(g.IN);
    p->NB = int32_t(g.NB);
}

// Dense large-N path (vqk_hgemm.hip): W dequantised panel by panel into the
// workspace in the GEMM's operand type, then the matrix-core GEMM.
int launch_x_stage(const void *x, int32_t x_type, int64_t N, int64_t IN, int64_t ld, uint16_t *out,
                   hipStream_t st);
int dequant_rows(const vqk_weights *w, int64_t r0, int64_t rows, uint16_t *out, int mode, int64_t ld,
                 hipStream_t st);
constexpr int64_t kPanelMin = 128;   // weight rows of the smallest panel
constexpr int64_t kGemmK = 64;       // the GEMM's k step: operand rows are padded to a multiple

static int64_t pad_k(const Geom &g) { return (g.IN + kGemmK - 1) / kGemmK * kGemmK; }

// Workspace of the decode-then-GEMM path for N rows: the larger of
//   fp16 / bf16 x: the whole weight as one panel of padded rows, plus a copy
//                  of x when IN is not a multiple of the k step, plus the
//                  split-K partials of the whole-weight GEMM's plan;
//   fp32 x:        x split into bf16 rows [x_hi | x_hi | x_lo], plus the
//                  smallest panel of split weight rows.
// A smaller workspace (>= the copy of x + 128 weight rows) runs in panels.
static size_t dense_ws_bytes(const Geom &g, int64_t N) {
    const size_t kp = size_t(pad_k(g));
    const size_t xcopy = g.IN % kGemmK ? al256(size_t(N) * kp * 2) : 0;
    const size_t half = xcopy + al256(size_t(g.OUT) * kp * 2) +
                        al256(plan_gemm(N, g.OUT, int64_t(kp), SIZE_MAX).part_bytes);
    const size_t f32 = al256(size_t(N) * 3 * kp * 2) + size_t(kPanelMin) * 3 * kp * 2;
    return half > f32 ? half : f32;
}

// The reference's `xf @ w.T.astype(xf.dtype)` (vq_dense.py:288, 294): fp16 x
// multiplies the bit-exact fp16 weight, bf16 x its bf16 rounding (one RNE),
// each in its own type with fp32 accumulation; fp32 x goes through the split
// form (k_x_stage). Operand rows are padded with zeros to the GEMM's k step;
// x is staged into the workspace when it is fp32, misaligned or padded.
// Panels of whole 128-row multiples when the workspace is smaller than the
// weight.
static int dense_decode_gemm(const vqk_weights *w, const Geom &g, const void *x, int32_t x_type,
                             int64_t N, void *y, int32_t y_type, void *workspace, size_t ws_bytes,
                             hipStream_t st) {
    const int64_t kp = pad_k(g);
    const int parts = x_type == VQK_F32 ? 3 : 1;
    const size_t row_b = size_t(parts * kp) * 2;
    const bool stage = x_type == VQK_F32 || kp != g.IN || (reinterpret_cast<uintptr_t>(x) & 15);
    const size_t xb = stage ? al256(size_t(N) * row_b) : 0;
    if (!workspace || ws_bytes < xb + kPanelMin * row_b)
        return set_error(VQK_ENOSPACE, "dense GEMM workspace %zu B < %zu B (%s%lld weight rows)",
                         ws_bytes, xb + kPanelMin * row_b, stage ? "staged x + " : "",
                         (long long)kPanelMin);
    if (reinterpret_cast<uintptr_t>(workspace) & 15)
        return set_error(VQK_EINVAL, "dense GEMM workspace must be 16-byte aligned");
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    const uint16_t *a = static_cast<const uint16_t *>(x);
    int rc;
    if (stage) {
        uint16_t *xs = reinterpret_cast<uint16_t *>(ws);
        if ((rc = launch_x_stage(x, x_type, N, g.IN, kp, xs, st))) return rc;
        a = xs;
    }
    const int op = x_type == VQK_F16 ? kOpF16 : kOpBF16;
    const int mode = x_type == VQK_F16 ? kDqF16 : (x_type == VQK_BF16 ? kDqBF16 : kDqSplit);
    uint16_t *panel = reinterpret_cast<uint16_t *>(ws + xb);
    int64_t prow = int64_t((ws_bytes - xb) / row_b);
    prow = prow >= g.OUT ? g.OUT : prow / kPanelMin * kPanelMin;
    for (int64_t r0 = 0; r0 < g.OUT; r0 += prow) {
        const int64_t rows = g.OUT - r0 < prow ? g.OUT - r0 : prow;
        // split-K partials go in whatever the panel leaves of the workspace
        const size_t used = xb + al256(size_t(rows) * row_b);
        const GemmPlan plan = plan_gemm(N, rows, parts * kp, used < ws_bytes ? ws_bytes - used : 0);
        float *part = plan.splits ? reinterpret_cast<float *>(ws + used) : nullptr;
        if ((rc = dequant_rows(w, r0, rows, panel, mode, kp, st))) return rc;
        if ((rc = launch_hgemm(op, plan, a, panel, y, y_type, g.OUT, r0, N, rows, parts * kp, part, st)))
            return rc;
    }
    return VQK_OK;
}

// tok: the most rows a tile holds (16, or 4 from a narrow sort).
static int launch_seg(const SegParams &p, const Geom &g, int tok, dim3 grid, hipStream_t st) {
    switch (g.D) {
        case 2: return launch_seg_d2(p, g.BITS, g.gpb, grid, st);
        case 4: return launch_seg_d4(p, g.BITS, g.gpb, grid, st);
        default: return launch_seg_d8(p, g.BITS, g.gpb, tok, grid, st);
    }
}

static int fill_gemm(const vqk_weights *w, const Geom &g, GemmParams *p) {
    memset(p, 0, sizeof *p);
    p->codes = w->codes;
    p->code_cols = w->code_cols;
    p->bits = g.packed ? g.BITS : 0;
    p->code_bytes = g.packed ? 4 : g.BITS / 8;
    p->codebook = w->codebook;
    p->K = int32_t(g.K);
    p->scales = w->scales;
    p->ngrp = int32_t(g.NGRP);
    p->G = g.G;
    p->row_table = w->row_table;
    p->stored_rows = g.rows;
    p->E = int32_t(g.E);
    p->OUT = int32_t(g.OUT);
    p->IN = int32_t(g.IN);
    p->NSUB = int32_t(g.NSUB);
    if (g.OUT > INT32_MAX || g.IN > INT32_MAX) return set_error(VQK_ENOTIMPL, "shape too large");
    return VQK_OK;
}

template <int D, bool CBL, int BM, int BN, int WM, int WN>
static int go_gemm(const GemmParams &p, dim3 grid, size_t smem, hipStream_t st) {
    return launch_with_lds<k_vq_gemm<D, CBL, BM, BN, WM, WN>>(grid, dim3(64 * WM * WN), smem, st, p);
}

template <int BM, int BN, int WM, int WN>
static int launch_gemm(const GemmParams &p, const Geom &g, dim3 grid, hipStream_t st) {
    const bool cbl = g.K * g.D * 2 <= kCbLdsMax &&
                     (reinterpret_cast<uintptr_t>(p.codebook) & 15) == 0 && (g.K * g.D * 2) % 4 == 0;
    const size_t smem = size_t(BM + BN) * kLdsStride * 2 + (cbl ? size_t(g.K) * g.D * 2 : 0);
    switch (g.D) {
        case 2: return cbl ? go_gemm<2, true, BM, BN, WM, WN>(p, grid, smem, st)
                           : go_gemm<2, false, BM, BN, WM, WN>(p, grid, smem, st);
        case 4: return cbl ? go_gemm<4, true, BM, BN, WM, WN>(p, grid, smem, st)
                           : go_gemm<4, false, BM, BN, WM, WN>(p, grid, smem, st);
        default: return cbl ? go_gemm<8, true, BM, BN, WM, WN>(p, grid, smem, st)
                            : go_gemm<8, false, BM, BN, WM, WN>(p, grid, smem, st);
    }
}

// Types always; x and y only when there are rows (an empty call touches
// neither, so NULL -- an empty tensor's pointer -- is accepted then).
static int check_acts(const void *x, int32_t x_type, const void *y, int32_t y_type, int64_t rows) {
    if (!act_size(x_type) || !out_size(y_type))
        return set_error(VQK_EINVAL, "x/y type must be VQK_F16, VQK_BF16 or VQK_F32");
    if ((!x || !y) && rows > 0) return set_error(VQK_EINVAL, "x and y are required");
    return VQK_OK;
}

// ---- pieces of the grouped path for callers that sort one routing and run
// several projections over it (the batched MoE layer)
static size_t sort_order_bytes(int64_t N) { return al256(sizeof(int32_t) * size_t(N)); }
static size_t sort_meta_bytes(int64_t N, int64_t E) {     // room for either tile size
    return al256(sizeof(int32_t) * 3 * size_t(group_max_tiles(N, E, kSegTokNarrow)));
}

size_t seg_sort_bytes(int64_t N, int64_t E) {
    return sort_order_bytes(N) + sort_meta_bytes(N, E) + 256;
}

bool seg_ok(const vqk_weights *w, int64_t N) {
    Geom g;
    if (make_geom(w, &g)) return false;
    return seg_fits_geom(g, w) && g.E <= kMaxSortExperts &&
           group_max_tiles(N, g.E, kSegTokNarrow) <= 65535 && N <= INT32_MAX / 2;
}

int seg_ksplit(const vqk_weights *w, int64_t N) {
    Geom g;
    if (make_geom(w, &g)) return 1;
    const int64_t nss = (g.NB + 3) / 4;
    const int64_t wgs = ((g.OUT + kSegRows - 1) / kSegRows) * ((N + kSegTok - 1) / kSegTok);
    int64_t ks = wgs > 0 ? big_grid(int64_t(1) << 30) / wgs : 1;
    ks = ks < 1 ? 1 : (ks > nss ? nss : ks);
    return int(ks > 4 ? 4 : ks);
}

int seg_tile_rows(const vqk_weights *w, int64_t N, int64_t E) {
    Geom g;
    if (make_geom(w, &g)) return kSegTok;
    return (g.D == 8 && !cb_in_lds(8, g.BITS) && N <= 2 * E) ? kSegTokNarrow : kSegTok;
}

int seg_sort(const uint32_t *eidx, int64_t N, int64_t E, int tok, void *ws, hipStream_t st) {
    if (N == 0) return VQK_OK;
    if (tok != kSegTok && tok != kSegTokNarrow)
        return set_error(VQK_EINVAL, "sort tiles of %d rows (16 or %d)", tok, kSegTokNarrow);
    uint8_t *b = static_cast<uint8_t *>(ws);
    const int64_t mt = group_max_tiles(N, E, tok);
    int32_t *order = reinterpret_cast<int32_t *>(b);
    int32_t *tmeta = reinterpret_cast<int32_t *>(b + sort_order_bytes(N));
    int32_t *ntiles = reinterpret_cast<int32_t *>(b + sort_order_bytes(N) + sort_meta_bytes(N, E));
    const size_t sort_lds = sizeof(int) * (3 * size_t(E + 1) + kSortThreads + 2);
    hipLaunchKernelGGL(k_group_sort, dim3(1), dim3(kSortThreads), sort_lds, st, eidx, int(N), int(E),
                       tok, int(mt), order, tmeta, ntiles);
    return hip_status(hipGetLastError(), "group sort launch");
}

int seg_run(const vqk_weights *w, const SegCall &c, const void *sort_ws, hipStream_t st) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (c.N == 0) return VQK_OK;
    SegParams sp;
    fill_seg(w, g, &sp);
    sp.x = c.x;
    sp.x_type = c.x_type;
    sp.xg = c.xg;
    sp.xu = c.xu;
    sp.xkrep = int32_t(c.xkrep);
    sp.y = c.y;
    sp.y_type = c.y_type;
    sp.N = int32_t(c.N);
    if (c.xparts > 1) {
        if (!c.xg) return set_error(VQK_EINVAL, "x partials need fp32 gate / up rows");
        sp.xparts = c.xparts;
        sp.xpstride = c.N * g.IN;
    }
    const int ks = c.ksplit > 1 ? c.ksplit : 1;
    if (ks > 1) {
        if (sort_ws || c.y_type != VQK_F32 || ks > 64)
            return set_error(VQK_EINVAL, "K split needs dense rows, fp32 output, <= 64 slices");
        sp.ksplit = ks;
        sp.ypart = c.N * g.OUT;
    }
    int64_t tiles = (c.N + kSegTok - 1) / kSegTok;
    int tok = kSegTok;
    if (sort_ws) {
        tok = c.tok ? c.tok : kSegTok;
        if (tok != kSegTok && tok != kSegTokNarrow)
            return set_error(VQK_EINVAL, "sorted tiles of %d rows (16 or %d)", tok, kSegTokNarrow);
        const uint8_t *b = static_cast<const uint8_t *>(sort_ws);
        sp.order = reinterpret_cast<const int32_t *>(b);
        sp.tmeta = reinterpret_cast<const int32_t *>(b + sort_order_bytes(c.N));
        sp.ntiles = reinterpret_cast<const int32_t *>(b + sort_order_bytes(c.N) + sort_meta_bytes(c.N, g.E));
        tiles = group_max_tiles(c.N, g.E, tok);
    }
    const int64_t nxb = (g.OUT + kSegRows - 1) / kSegRows;
    const int64_t nxp = (g.OUT + kPersistWaves * 32 - 1) / (kPersistWaves * 32);
    if (sort_ws && tok == kSegTokNarrow && g.D == 8 && !cb_in_lds(8, g.BITS)) {
        // one workgroup per CU walking (tile, row block) items: the table
        // part is staged once per CU, not once per item. The sort chose 4- or
        // 8-row tiles; the kernel reads its choice.
        const dim3 grid(unsigned(big_grid(nxp * tiles)), 1, 1);
        return launch_seg_persist_d8(sp, g.BITS, g.gpb, grid, st);
    }
    // the 16-row kernel: dense rows, or sorted tiles of any size (<= 16 rows)
    const dim3 grid{unsigned(nxb), unsigned(tiles), unsigned(ks)};
    return launch_seg(sp, g, kSegTok, grid, st);
}

}  // namespace vqk

using namespace vqk;

extern "C" {

int vqk_gemmseg_fits(int32_t D, int64_t K, int32_t G, int32_t pack_bits, int64_t IN) {
    return (D == 2 || D == 4 || D == 8) && K >= 1 && K <= 65536 && G > 0 && G % D == 0 &&
           IN > 0 && IN % G == 0 && IN % D == 0 && pack_bits >= 0 && pack_bits <= 16;
}

int vqk_dense_gemm_workspace(const vqk_weights *w, int64_t N, size_t *bytes) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (!bytes || N < 0) return set_error(VQK_EINVAL, "bad arguments");
    // up to 64 rows the segment kernel decodes in registers and needs none
    const bool seg = N <= kSegDenseMaxN && seg_fits_geom(g, w);
    *bytes = (!seg && N > 0) ? dense_ws_bytes(g, N) : 0;
    return VQK_OK;
}

int vqk_dense_gemm(const vqk_weights *w, const void *x, int32_t x_type, int64_t N, void *y,
                   int32_t y_type, void *workspace, size_t ws_bytes, void *stream) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (g.E != 1) return set_error(VQK_EINVAL, "dense GEMM takes one linear (E=1), got E=%lld",
                                   (long long)g.E);
    if ((rc = check_acts(x, x_type, y, y_type, N))) return rc;
    if (N < 0 || N > INT32_MAX) return set_error(VQK_EINVAL, "N=%lld", (long long)N);
    if (N == 0) return VQK_OK;
    if (N <= kSegDenseMaxN && seg_fits(g, w, x)) {
        SegParams sp;
        fill_seg(w, g, &sp);
        sp.x = x;
        sp.x_type = x_type;
        sp.xkrep = 1;
        sp.y = y;
        sp.y_type = y_type;
        sp.N = int32_t(N);
        const dim3 grid(unsigned((g.OUT + kSegRows - 1) / kSegRows),
                        unsigned((N + kSegTok - 1) / kSegTok), 1);
        return launch_seg(sp, g, kSegTok, grid, hipStream_t(stream));
    }
    if (g.OUT > INT32_MAX || 3 * pad_k(g) > INT32_MAX)
        return set_error(VQK_ENOTIMPL, "dense GEMM shape OUT %lld IN %lld", (long long)g.OUT,
                         (long long)g.IN);
    return dense_decode_gemm(w, g, x, x_type, N, y, y_type, workspace, ws_bytes, hipStream_t(stream));
}

int vqk_grouped_gemm_workspace(const vqk_weights *w, int64_t N, size_t *bytes) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if (!bytes || N < 0) return set_error(VQK_EINVAL, "bad arguments");
    *bytes = seg_sort_bytes(N, g.E);
    return VQK_OK;
}

int vqk_grouped_gemm(const vqk_weights *w, const void *x, int32_t x_type, int64_t T,
                     const uint32_t *eidx, int64_t N, int64_t xkrep, void *y, int32_t y_type,
                     void *workspace, size_t ws_bytes, void *stream) {
    Geom g;
    int rc = make_geom(w, &g);
    if (rc) return rc;
    if ((rc = check_acts(x, x_type, y, y_type, N))) return rc;
    if (!eidx && N > 0) return set_error(VQK_EINVAL, "eidx is required");
    if (N < 0 || T < 0 || xkrep < 1 || N != T * xkrep)
        return set_error(VQK_EINVAL, "pairs N=%lld must equal tokens T=%lld x xkrep=%lld",
                         (long long)N, (long long)T, (long long)xkrep);
    if (N > INT32_MAX / 2) return set_error(VQK_ENOTIMPL, "N=%lld pairs is too many", (long long)N);
    if (g.E > kMaxSortExperts)
        return set_error(VQK_ENOTIMPL, "grouped GEMM sorts at most %d experts", kMaxSortExperts);
    if (N == 0) return VQK_OK;
    size_t need = 0;
    vqk_grouped_gemm_workspace(w, N, &need);
    if (!workspace || ws_bytes < need)
        return set_error(VQK_ENOSPACE, "workspace %zu B < %zu B", ws_bytes, need);
    if (reinterpret_cast<uintptr_t>(workspace) & 15)
        return set_error(VQK_EINVAL, "grouped GEMM workspace must be 16-byte aligned");
    const bool seg = seg_fits(g, w, x);
    const int tok = seg ? seg_tile_rows(w, N, g.E) : kSegTok;
    const int64_t mt = group_max_tiles(N, g.E, tok);
    if (mt > 65535) return set_error(VQK_ENOTIMPL, "%lld tiles exceed one launch", (long long)mt);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    int32_t *order = reinterpret_cast<int32_t *>(ws);
    int32_t *tmeta = reinterpret_cast<int32_t *>(ws + sort_order_bytes(N));
    int32_t *ntiles = reinterpret_cast<int32_t *>(ws + sort_order_bytes(N) + sort_meta_bytes(N, g.E));
    hipStream_t st = hipStream_t(stream);
    if ((rc = seg_sort(eidx, N, g.E, tok, ws, st))) return rc;
    if (seg) {
        const SegCall c{x, x_type, nullptr, nullptr, xkrep, y, y_type, N, tok};
        return seg_run(w, c, ws, st);
    }
    GemmParams p;
    if ((rc = fill_gemm(w, g, &p))) return rc;
    p.x = x;
    p.x_type = x_type;
    p.xkrep = int32_t(xkrep);
    p.y = y;
    p.y_type = y_type;
    p.N = int32_t(N);
    p.tmeta = tmeta;
    p.ntiles = ntiles;
    p.order = order;
    p.eidx = eidx;
    const dim3 grid(unsigned((g.OUT + kGroupBN - 1) / kGroupBN), unsigned(mt), 1);
    return launch_gemm<kGroupBM, kGroupBN, 1, 4>(p, g, grid, st);
}

}  // extern "C"
