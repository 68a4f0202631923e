// Fused MoE decode layer: routing + SwitchGLU + combine in one launch
// (k_moe_layer1: batch 1, tables in LDS) or two kernels.
//
// Reference: mlx-lm's SparseMoeBlock / SwitchGLU around VQSwitchLinear,
// restated in bench/decode_ladder.py:107-119 (softmax(fp32) -> top-k ->
// renormalise -> up/gate -> SiLU(gate)*up -> down -> sum_j w_j y_j) and
// tests/test_qwen3_5_parity.py:180-205 (+ sigmoid(shared_gate . x) * shared(x)).
//
//   k_moe_up    grid (row tiles of I, T * P), P = top_k + shared pairs per token.
//               Wave 0 computes its token's routing from the logits (no
//               extra launch, no host sync) while the other waves stage both
//               codebooks and x; then waves 0-3 decode the tile's gate rows
//               and waves 4-7 the same rows of up, and the workgroup writes
//               h = silu(g) * u as fp16 into the workspace. Workgroup
//               (0, pair 0) of each token also writes the routing.
//   k_moe_down  grid (row tiles of H, T). Lanes are (pair j, block b) of one
//               token, so a wave covers whole output rows across all the
//               token's experts; each lane scales its partial by the router
//               weight and the butterfly reduction IS the combine -- no
//               atomics, deterministic.
//   k_moe_layer1 both in one grid: the k_moe_up workgroups, then down
//               workgroups that route for themselves, fetch their weights and
//               table entries early and take the SwiGLU rows as tagged words.
#include <atomic>
#include <mutex>

#include "vqk_gemv.h"
#include "vqk_internal.h"
#include "vqk_big.h"

namespace vqk {

constexpr int kMaxExperts = 1024;
constexpr int kMaxSlots = kMaxExperts / kWave;   // logits per lane
constexpr int kMaxTopK = 64;
// (token, expert) pairs from which a layer call runs as grouped GEMMs: at
// least this many, and at least one per expert on average (fewer leave most
// expert tiles with a single pair, where the GEMV paths measured faster:
// config-3 layer, T = 16 -> 160 pairs over 512 experts: 698 us sliced GEMV
// against 745 us grouped; T = 64: 2583 us against 1588 us)
constexpr int64_t kMoeGroupedMinPairs = 64;

struct MoeW {            // one projection of the layer, as the kernels see it
    const uint32_t *codes;
    const uint16_t *codebook;
    const uint16_t *scales;
    const int32_t *row_table;
    int64_t row_words;
    int64_t stored_rows;
    int32_t K;
};

struct MoeParams {
    MoeW gate, up, down, sgate, sup, sdown;   // s* = shared expert (E == 1)
    int32_t shared;                           // 1 if the shared expert exists
    int32_t E, top_k, norm;
    int32_t H, I;                             // hidden (x, y) and intermediate widths
    int32_t NB1, NB2;                         // blocks per row: gate/up (H) and down (I)
    int32_t ngrp1, ngrp2, bpg1, bpg2;
    int32_t lpr1_log2, lpr2_log2;
    int32_t rows_per_wg1, steps1, rows_per_wg2, steps2;
    int32_t T, P;
    const void *x;
    int32_t x_type;
    const float *logits;
    const void *sg_vec;
    int32_t sg_type;
    void *y;
    int32_t y_type;
    int32_t *ids;        // workspace [T, top_k]
    float *wts;          // workspace [T, top_k]
    float *sg;           // workspace [T]
    uint16_t *h;         // workspace [T, P, I] fp16
    float *gbuf, *ubuf;  // split gate/up phase: workspace [T, P, I] fp32 each, else NULL
    int32_t *ids_out;    // optional user copies
    float *wts_out;
    // one-launch layer (k_moe_layer1): call number, error word, per-workgroup
    // stamps and tagged SwiGLU words in the workspace header; gate/up
    // workgroups and their row tiles per pair, down row tiles per token; the
    // bound of every wait
    uint64_t *l1_epoch, *l1_err, *l1_stamp, *l1_hw;
    int32_t l1_g1, l1_gx1, l1_gx2;
    int32_t l1_spins;
};

// ------------------------------------------------------------ routing
// Keys of one lane in descending order, equal keys by lower index: Batcher's
// odd-even merge sort network over NS (a power of two) slots, fully unrolled.
template <int NS>
__device__ __forceinline__ void sort_keys_desc(uint32_t (&key)[NS], uint32_t (&idx)[NS]) {
#pragma unroll
    for (int p = 1; p < NS; p <<= 1)
#pragma unroll
        for (int k = p; k >= 1; k >>= 1)
#pragma unroll
            for (int j = k % p; j + k < NS; j += 2 * k)
#pragma unroll
                for (int i = 0; i < k && i + j + k < NS; ++i)
                    if ((i + j) / (2 * p) == (i + j + k) / (2 * p)) {
                        const int a = i + j, b = i + j + k;
                        const bool sw = key[b] > key[a] || (key[b] == key[a] && idx[b] < idx[a]);
                        const uint32_t ka = key[a], ia = idx[a];
                        key[a] = sw ? key[b] : ka;
                        idx[a] = sw ? idx[b] : ia;
                        key[b] = sw ? ka : key[b];
                        idx[b] = sw ? ia : idx[b];
                    }
}

// LDS of one routing wave: the candidates' 64-bit ranking keys and the
// selections in order.
constexpr int kFastTopK = 16;            // largest k of the threshold-and-rank top-k
struct RouteScratch {
    uint64_t cand[kWave];
    uint32_t sel_idx[kFastTopK];
    uint32_t sel_key[kFastTopK];
};

// Routing of one token by one wave, in two halves: route_pick finds the
// selections (the expert of the workgroup's own pair first of all),
// route_weights turns them into router weights (softmax over all experts, or
// renormalised over the selections). Lanes hold NS logits each (lane l:
// experts s * 64 + l).
struct RoutePick {
    int e_want;          // expert of pair `want` (wave-uniform), -1 if none
    int midx;            // sequential path: lane r < k holds selection r
    uint32_t mykey;
    bool ranked;         // selections in RouteScratch::sel_idx / sel_key
};

// Threshold-and-rank selection (k <= 16). The lanes form G >= k groups (8
// lanes for k <= 8, else 4); the smallest group maximum tau is at most the
// k-th largest key (the G group maxima are G distinct keys >= tau), so every
// selection is among the keys >= tau -- about 20 of 256 for random logits.
// Those candidates are compacted into LDS as (key << 32 | ~index), which
// orders them exactly as the selection does (larger key first, lower index on
// ties), and each takes its rank by counting the candidates above it; ranks
// below k are the selections, written in order, and the pair's own expert
// comes straight from the lane that holds rank `want` (no LDS round trip).
// Returns false when tau is the key of a NaN or padding slot, or more than 64
// keys are >= tau; the caller then takes the sequential selection.
template <int NS>
__device__ __forceinline__ bool topk_rank(const uint32_t (&key)[NS], int k, int want, RouteScratch *rs,
                                          int *e_want) {
    const int lane = threadIdx.x & (kWave - 1);
    uint32_t gm = key[0];
#pragma unroll
    for (int s = 1; s < NS; ++s) gm = max(gm, key[s]);
    gm = max(gm, dpp_u<kDppQuadXor1>(gm));
    gm = max(gm, dpp_u<kDppQuadXor2>(gm));
    if (k <= 8) gm = max(gm, dpp_u<kDppRowHalfMirror>(gm));
    const uint32_t tau = wave_min_u32(gm);
    if (tau == 0u) return false;
    uint64_t bal[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) bal[s] = __ballot(key[s] >= tau);
    int c = 0;                                          // candidates so far (wave-uniform)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int pos = c + int(__builtin_amdgcn_mbcnt_hi(uint32_t(bal[s] >> 32),
                                                           __builtin_amdgcn_mbcnt_lo(uint32_t(bal[s]), 0u)));
        if (key[s] >= tau && pos < kWave)
            rs->cand[pos] = (uint64_t(key[s]) << 32) | uint64_t(~uint32_t(s * kWave + lane));
        c += __popcll(bal[s]);
    }
    if (c > kWave) return false;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // slots past c hold 0 (route_pick clears them before the candidates land)
    const uint64_t mine = rs->cand[lane];
    int rank = 0;
    {
        uint64_t v[16];                                 // the first 16 in one round trip
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = rs->cand[u];
#pragma unroll
        for (int u = 0; u < 16; ++u) rank += v[u] > mine ? 1 : 0;
    }
    for (int j0 = 16; j0 < c; j0 += 8) {
        uint64_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = rs->cand[j0 + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) rank += v[u] > mine ? 1 : 0;
    }
    const bool sel = lane < c && rank < k;
    if (sel) {
        rs->sel_idx[rank] = ~uint32_t(mine);
        rs->sel_key[rank] = uint32_t(mine >> 32);
    }
    int e_w = -1;
    if (want >= 0 && want < k) {
        const uint64_t b = __ballot(sel && rank == want);
        if (b) e_w = __builtin_amdgcn_readlane(int(~uint32_t(mine)), __ffsll((unsigned long long)b) - 1);
    }
    *e_want = e_w;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    return true;
}

// Selections of one token's logits (fp32). Argmax is exact: logits become
// order-preserving integer keys (key[], kept for route_weights). The
// selections come from topk_rank, or (k > 16, NaN-heavy or degenerate
// logits) from k sequential selections over each lane's keys sorted once,
// each a DPP max over the lanes' head keys; the lane holding it (on a tie
// between lanes, the one whose head has the lowest index) pops its head.
// Either way ties go to the lower expert id (stable descending order); NaN
// logits sort below -inf and are never chosen while k <= number of finite
// logits. The loads take clamped indices and no branch.
template <int NS>
__device__ __forceinline__ void route_pick(const float *lg, int E, int k, int want, RouteScratch *rs,
                                           uint32_t (&key)[NS], RoutePick &rp) {
    const int lane = threadIdx.x & (kWave - 1);
    float raw[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) raw[s] = lg[min(s * kWave + lane, E - 1)];
    rs->cand[lane] = 0;                                 // LDS writes of a wave land in order
    wait_vmem();                                        // the logits are this wave's only loads
#pragma unroll
    for (int s = 0; s < NS; ++s) key[s] = s * kWave + lane < E ? f32_key(raw[s]) : 0u;
    rp.midx = -1;
    rp.mykey = 0u;
    rp.ranked = k <= kFastTopK && topk_rank<NS>(key, k, want, rs, &rp.e_want);
    if (rp.ranked) return;
    // sequential selections over a sorted copy; lane r keeps selection r
    uint32_t sk[NS], si[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        sk[s] = key[s];
        si[s] = uint32_t(s * kWave + lane);
    }
    sort_keys_desc<NS>(sk, si);
    int e_w = -1;
    for (int r = 0; r < k; ++r) {
        const uint32_t best = wave_max_u32(sk[0]);
        int bi = -1;
        if (best) {
            const uint64_t hit = __ballot(sk[0] == best);
            int wl;
            if ((hit & (hit - 1)) == 0) {
                wl = __ffsll((unsigned long long)hit) - 1;
            } else {                                     // tie between lanes: lowest index
                const uint32_t mi = wave_min_u32(sk[0] == best ? si[0] : 0xffffffffu);
                wl = int(mi & (kWave - 1));
            }
            bi = __builtin_amdgcn_readlane(int(si[0]), wl);
            if (lane == wl) {
#pragma unroll
                for (int s = 0; s + 1 < NS; ++s) {
                    sk[s] = sk[s + 1];
                    si[s] = si[s + 1];
                }
                sk[NS - 1] = 0u;
            }
        }
        if (r == want) e_w = bi;
        if (lane == r) { rp.midx = bi; rp.mykey = bi >= 0 ? best : 0u; }
    }
    rp.e_want = e_w;
}

// Router weights of the selections (fp32, like the reference's precise
// softmax): lane r < k gets selection r in (*my_idx, *my_w). The largest
// logit, the softmax's shift, is the first selection's.
template <int NS>
__device__ __forceinline__ void route_weights(const uint32_t (&key)[NS], int k, int norm, RouteScratch *rs,
                                              const RoutePick &rp, int *my_idx, float *my_w) {
    const int lane = threadIdx.x & (kWave - 1);
    int midx = rp.midx;
    uint32_t mykey = rp.mykey;
    if (rp.ranked && lane < k) {
        midx = int(rs->sel_idx[lane]);
        mykey = rs->sel_key[lane];
    }
    const float m = key_f32(uint32_t(__builtin_amdgcn_readlane(int(mykey), 0)));
    const float pr = (lane < k && mykey) ? __expf(key_f32(mykey) - m) : 0.f;
    float w;
    if (norm) {
        const float psel = wave_sum(pr);
        w = psel > 0.f ? pr * (1.f / psel) : 0.f;
    } else {
        float lsum = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s)
            if (key[s]) lsum += __expf(key_f32(key[s]) - m);
        w = pr * (1.f / wave_sum(lsum));
    }
    *my_idx = lane < k ? midx : -1;
    *my_w = w;
}

// Both halves: every lane returns the expert of pair `want` (or -1) in
// *e_want; lane r < k holds selection r in (*my_idx, *my_w).
template <int NS>
__device__ __forceinline__ void route_wave(const float *lg, int E, int k, int norm, int want,
                                           RouteScratch *rs, int *e_want, int *my_idx, float *my_w) {
    uint32_t key[NS];
    RoutePick rp;
    route_pick<NS>(lg, E, k, want, rs, key, rp);
    route_weights<NS>(key, k, norm, rs, rp, my_idx, my_w);
    *e_want = rp.e_want;
}

// One instance for E <= 64 * NS (the one-launch layer: its code stays small;
// slots past E hold key 0, so the selections and weights are route()'s).
template <int NS>
__device__ __forceinline__ void route_upto(const float *lg, int E, int k, int norm, int want,
                                           RouteScratch *rs, int *e_want, int *my_idx, float *my_w) {
    route_wave<NS>(lg, E, k, norm, want, rs, e_want, my_idx, my_w);
}

__device__ __forceinline__ void route(const float *lg, int E, int k, int norm, int want,
                                      RouteScratch *rs, int *e_want, int *my_idx, float *my_w) {
    const int ns = (E + kWave - 1) / kWave;              // wave-uniform
    if (ns <= 1) route_wave<1>(lg, E, k, norm, want, rs, e_want, my_idx, my_w);
    else if (ns <= 2) route_wave<2>(lg, E, k, norm, want, rs, e_want, my_idx, my_w);
    else if (ns <= 4) route_wave<4>(lg, E, k, norm, want, rs, e_want, my_idx, my_w);
    else if (ns <= 8) route_wave<8>(lg, E, k, norm, want, rs, e_want, my_idx, my_w);
    else route_wave<16>(lg, E, k, norm, want, rs, e_want, my_idx, my_w);
}

__device__ __forceinline__ float silu(float g) { return g / (1.f + __expf(-g)); }

// Eight activations of a 16-bit type (raw words) as fp32: exact widening.
__device__ __forceinline__ float act16_f32(uint32_t w, int k, int32_t type) {
    const uint16_t h = uint16_t(k ? (w >> 16) : w);
    return type == VQK_BF16 ? bf16_to_f32(h) : h_to_f32(h);
}

// sum_i x[t, i] * sg_vec[i] over the wave (every lane gets it): the shared
// expert's gate logit. 16-bit x and gate vector, 16-byte aligned: each lane
// issues the 16-byte loads of up to 8 chunks of 8 before it multiplies, so
// the dot costs one memory latency per 4096 values; other layouts take the
// element loop.
__device__ __forceinline__ float shared_gate_dot(const void *x, int32_t x_type, const void *sg_vec,
                                                int32_t sg_type, int H, int t) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t xb = int64_t(t) * H;
    const bool vec = x_type != VQK_F32 && sg_type != VQK_F32 && (H % 8) == 0 &&
                     ((reinterpret_cast<uintptr_t>(x) + uint64_t(xb) * 2) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(sg_vec) & 15) == 0;
    float acc = 0.f;
    if (vec) {
        constexpr int U = 8;
        const int nc = H / 8;
        const uint16_t *xr = static_cast<const uint16_t *>(x) + xb;
        const uint16_t *gr = static_cast<const uint16_t *>(sg_vec);
        for (int c0 = 0; c0 < nc; c0 += U * kWave) {
            u32x4 xv[U], gv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + lane + u * kWave;
                xv[u] = c < nc ? *reinterpret_cast<const u32x4 *>(xr + int64_t(c) * 8) : u32x4{0, 0, 0, 0};
                gv[u] = c < nc ? *reinterpret_cast<const u32x4 *>(gr + int64_t(c) * 8) : u32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t xw[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
                const uint32_t gw[4] = {gv[u].x, gv[u].y, gv[u].z, gv[u].w};
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    acc = fmaf(act16_f32(xw[k >> 1], k & 1, x_type), act16_f32(gw[k >> 1], k & 1, sg_type), acc);
            }
        }
    } else {
        for (int i = lane; i < H; i += kWave)
            acc += load_act(x, x_type, xb + i) * load_act(sg_vec, sg_type, i);
    }
    return wave_sum(acc);
}

// One lane's code block and its scales' raw fp16 bits; the scales become
// fp32 at their use (ScalesF32), so the wave's next loads (the up projection
// after the gate, the table copy after the down weights) issue at once.
// The code words are plain (cached) loads: lanes' blocks lie BITS words apart,
// so each of the block's BITS/4 vector loads touches every 64-byte segment of
// the row; the vector L1 serves the repeats, where streaming loads sent each
// one to L2 again (config 3: 48.6 -> 44.7 us per layer; config 2 unchanged).
template <int BITS, int GPB>
__device__ __forceinline__ void moe_load(const MoeW &w, int64_t cr, int blk, int sidx, int ngrp,
                                         uint32_t (&wd)[BITS], uint32_t (&s)[GPB]) {
    if (cr >= 0) {
        const uint32_t *src = w.codes + cr * w.row_words + int64_t(blk) * BITS;
#pragma unroll
        for (int i = 0; i < BITS; ++i) wd[i] = src[i];
        const uint16_t *sr = w.scales + cr * ngrp + sidx;
#pragma unroll
        for (int g = 0; g < GPB; ++g) s[g] = __builtin_nontemporal_load(sr + g);
    } else {
#pragma unroll
        for (int i = 0; i < BITS; ++i) wd[i] = 0u;
#pragma unroll
        for (int g = 0; g < GPB; ++g) s[g] = 0u;
    }
}

__device__ __forceinline__ int64_t moe_row(const MoeW &w, int64_t e, int OUT, int r) {
    int64_t f = e * OUT + r;
    if (w.row_table) f = w.row_table[f];
    return f < w.stored_rows ? f : -1;
}

// ------------------------------------------------------------ K1: gate/up
// LDS of the gate/up phase: two codebook tables, then x at the padded stride.
// Tables beyond the LDS-resident limit keep their first entries in LDS
// (64 KB per gate/up table, 112 KB of the routed down table) and gather the
// rest from L2: fewer L2 requests per code, the rate that bounds these kernels.
constexpr int kHybUpBytes = 64 * 1024;
constexpr int kHybDownBytes = 112 * 1024;
// Larger LDS parts when the workgroup's activations leave room (the host
// checks): every entry moved into LDS is an L2 request per code saved.
// 136 KB leaves room for 11 pairs' SwiGLU rows of a d8 row (config 3: 10 routed +
// the shared expert); the down kernel has no routing block in LDS (config 3:
// 132 KB -> 136 KB, 44.70 -> 44.44 us per layer).
constexpr int kHybDownWideBytes = 136 * 1024;
// Waves of the workgroups with the larger LDS parts (one workgroup per CU),
// which read x from LDS: two per SIMD, so one wave decodes while the other
// waits on its table reads (12 for gate / up measured no faster, 16 for down
// slower: it spills).
constexpr int kWideWavesUp = 8, kWideWavesDown = 8;
__host__ __device__ constexpr int moe_waves_up(bool wide) { return wide ? kWideWavesUp : kThreads / kWave; }
__host__ __device__ constexpr int moe_waves_down(bool wide) {
    return wide ? kWideWavesDown : kThreads / kWave;
}

// Entries of one gate/up table held in LDS, and of the routed down table.
template <int D, int BITS>
__host__ __device__ constexpr int up_cbn() {
    return cb_in_lds(D, BITS) ? (1 << BITS) : kHybUpBytes / (2 * D);
}
template <int D, int BITS, bool W = false>
__host__ __device__ constexpr int down_cbn() {
    return cb_in_lds(D, BITS) ? (1 << BITS) : (W ? kHybDownWideBytes : kHybDownBytes) / (2 * D);
}

// Routing of the workgroup's token as wave 0 computed it (LDS).
struct RouteLds {
    RouteScratch rs;           // the routing wave's scratch
    int route;                 // expert of this workgroup's pair
    uint32_t call;             // one-launch layer: the call number
};

// ------------------------------------------------ one-launch layer hand-off
// Every layer workspace starts with a header at fixed offsets, the same for
// every geometry, path and T, that only one-launch calls write: the call
// number n, a sticky error word, one stamp per workgroup and the hand-off
// words. The SwiGLU rows travel as 64-bit words: two fp16 values below a
// 32-bit tag of (n, w), w the word's index in the header's word region. The
// tag has its top bit set, and its low 31 bits are one-to-one in n mod 2^31
// for a fixed w (an odd multiple of n, then an invertible xorshift-multiply
// mix of 31-bit values). So a zeroed word (a header that starts zeroed) never
// passes, and a word that any earlier one-launch call left at index w -- of
// this geometry or another, on this workspace -- carries an earlier call
// number and never passes, unless it was left exactly a multiple of 2^31
// calls ago and no call since wrote index w. One 64-bit load both checks a
// word and delivers it.
// Every wait is bounded by MoeParams::l1_spins rounds (kL1Spins, ~45 ms, by
// default). A word that does not arrive in time enters the down dot products
// as NaN -- every output row that would have used it comes out NaN -- and
// sets kL1ErrPoll in the error word; workgroup 0, if a stamp does not
// arrive, sets kL1ErrStamp and leaves the call number as it is. Once the
// error word is set, the down workgroups of every later call on that
// workspace take every word as missing without waiting (NaN rows), until
// the header is zeroed again (vqk_moe_layer_reset); vqk_moe_layer_status
// reports it.
constexpr int kL1Spins = 1 << 16;        // default bound of every wait (~45 ms)
constexpr int kL1Slots = 4;              // logits per lane of its routing: E <= 256
constexpr uint64_t kL1ErrPoll = 1, kL1ErrStamp = 2;
// header layout (bytes): call number, error word, stamps, words
constexpr size_t kHdrEpoch = 0, kHdrError = 8, kHdrStamps = 256;
constexpr int kL1MaxWg = 1024;           // workgroups of a one-launch grid
constexpr int kL1MaxWords = 4096;        // hand-off words: P * I / 2 (d4: P * NB2 <= 64 -> 4096)
constexpr size_t kHdrWords = kHdrStamps + 8 * size_t(kL1MaxWg);
constexpr size_t kHdrBytes = VQK_MOE_HEADER_BYTES;
static_assert(kHdrWords % 256 == 0 && kHdrWords + 8 * size_t(kL1MaxWords) <= kHdrBytes,
              "the one-launch header must hold its stamps and words");
__device__ __forceinline__ uint32_t l1_tag(uint32_t n, uint32_t w) {
    constexpr uint32_t M = 0x7fffffffu;
    uint32_t v = (n * 0x9E3779B1u + w * 0x85EBCA6Bu + 0x6A09E667u) & M;
    v ^= v >> 16;
    v = (v * 0x7FEB352Du) & M;
    v ^= v >> 15;
    v = (v * 0x846CA68Bu) & M;
    v ^= v >> 16;
    return v | 0x80000000u;
}
// A workgroup's stamp once it has read call number n.
__device__ __forceinline__ uint64_t l1_stamp(uint32_t n) { return (uint64_t(~n) << 32) | n; }
__device__ __forceinline__ uint64_t l1_load(const uint64_t *a) {
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void l1_store(uint64_t *a, uint64_t v) {
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Down-phase state a workgroup prepares before it needs the SwiGLU input:
// its lane's code row, block words and scales for the first row step.
template <int BITS, int GPB>
struct DownState {
    uint32_t a[BITS];
    uint32_t s[GPB];     // raw fp16 bits
    int64_t cr, e;
    float wj;
};

// K1: routing + gate/up + SwiGLU for pair blockIdx.y, row tile blockIdx.x, with
// both tables in LDS. Eight waves: waves 0-3 decode the tile's gate rows,
// waves 4-7 the same rows of up (one block per lane each), and the two halves
// meet in LDS for silu(g) * u. With one projection per wave each lane decodes
// 32 codes instead of 64 and two waves share a SIMD, so one decodes while the
// other waits on its table reads (config 2: 12.35 -> 11.88 us per layer).
// The body, shared with the one-launch layer (TAG: the SwiGLU rows go out as
// tagged words, and the workgroup records the call number it read).
template <int D, int BITS, int GPB, bool TAG>
__device__ __forceinline__ void up_fused(const MoeParams &p, uint8_t *smem, RouteLds &rl, int bx,
                                         int pair) {
    constexpr int CBN = up_cbn<D, BITS>();         // entries of each table in LDS
    constexpr int XH = kBlock * D, XS = XH + 8;
    h2 *cbg_lds = reinterpret_cast<h2 *>(smem);
    h2 *cbu_lds = reinterpret_cast<h2 *>(smem + CBN * D * 2);
    f16 *xs = reinterpret_cast<f16 *>(smem + 2 * CBN * D * 2);
    // the tile's gate values, then its up values (fp32), after x
    float *vl = reinterpret_cast<float *>(smem + 2 * CBN * D * 2 + ((p.NB1 * XS * 2 + 15) & ~15));

    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
    const int proj = wave >> 2, rw = wave & 3;     // projection (0 gate, 1 up), row wave
    const int lpr = 1 << p.lpr1_log2, rpw = kWave >> p.lpr1_log2;
    const int sub = lane >> p.lpr1_log2, blk = lane & (lpr - 1);
    const bool on = blk < p.NB1;
    const int t = pair / p.P, j = pair % p.P;
    const bool is_shared = j >= p.top_k;
    const MoeW &wg = is_shared ? p.sgate : p.gate;
    const MoeW &wu = is_shared ? p.sup : p.up;
    const float *lg = p.logits + int64_t(t) * p.E;

    // Wave 0 loads the logits and picks the experts, with no other load in
    // flight (a wave's loads complete in order, so anything queued ahead of
    // the logits would delay the routing); waves 1-7 meanwhile stage x and
    // then stream the two codebooks into LDS (x first: its conversion waits
    // on its loads, which land in issue order, so behind the table copies it
    // waited for them too; config 2: 11.76 -> 11.60 us). One barrier
    // publishes the expert id, then every wave issues its weight loads
    // (nothing else is outstanding, so the barrier's wait never drains weight
    // loads). The routing and the table copies end within ~0.2 us of each
    // other; the router weights computed after the decode loop instead (off
    // the barrier's path) measured 0.04 us faster for ~25 more registers.
    int my_idx = -1;
    float my_w = 0.f;
    uint64_t ev = 0;
    if (wave == 0) {
        int e_pair;
        if constexpr (TAG)
            route_upto<kL1Slots>(lg, p.E, p.top_k, p.norm, is_shared ? -1 : j, &rl.rs, &e_pair, &my_idx, &my_w);
        else
            route(lg, p.E, p.top_k, p.norm, is_shared ? -1 : j, &rl.rs, &e_pair, &my_idx, &my_w);
        if (lane == 0) rl.route = e_pair;
    } else {
        constexpr int NT = 2 * kThreads - kWave;
        if (TAG && tid == kWave) ev = l1_load(p.l1_epoch);
        stage_x<XH, XS>(p.x, p.x_type, int64_t(t) * p.H, p.H, p.NB1, xs, kWave, NT);
        stage_codebook_fixed<D, CBN, NT, 1>(wg.codebook, wg.K, cbg_lds);
        stage_codebook_fixed<D, CBN, NT, 1>(wu.codebook, wu.K, cbu_lds);
    }
    wait_vmem();
    if (TAG && tid == kWave) {
        rl.call = uint32_t(ev);
        l1_store(p.l1_stamp + bx + pair * p.l1_gx1, l1_stamp(uint32_t(ev)));
    }
    __syncthreads();

    // a NaN logit can leave a selection empty: such a pair reads nothing
    const int e_pair = rl.route;
    const int64_t e = is_shared ? 0 : ((e_pair >= 0 && e_pair < p.E) ? e_pair : -1);
    const int sidx = GPB == 1 ? blk / p.bpg1 : blk * GPB;
    const int r_wg = bx * p.rows_per_wg1;
    auto row_at = [&](int st) { return r_wg + (st * 4 + rw) * rpw + sub; };
    const MoeW &w = proj ? wu : wg;
    // (this exact form measured 0.2 us per layer faster than the same
    // steps written with a row lambda and a hoisted table bound)
    uint32_t a[BITS];
    uint32_t sc[GPB];
    int64_t cr;
    {
        const int r = row_at(0);
        cr = (on && e >= 0 && r < p.I) ? moe_row(w, e, p.I, r) : -1;
        moe_load<BITS, GPB>(w, cr, blk, sidx, p.ngrp1, a, sc);
    }
    // d8 reads x from LDS per code: its 128 x registers do not fit beside the
    // rest at two waves per SIMD (nor, in the one-launch layer, any x at four)
    constexpr bool XL = D == 8 || TAG;
    const f16 *xl = xs + (on ? blk : 0) * XS;
    h2 xr[XL ? 1 : 16 * D];
    if constexpr (!XL) load_xregs<D>(xl, xr);
    const h2 *cb = proj ? cbu_lds : cbg_lds;
    for (int st = 0; st < p.steps1; ++st) {
        uint32_t n[BITS];
        uint32_t ns[GPB];
        int64_t cn = -1;
        if (st + 1 < p.steps1) {
            const int r = row_at(st + 1);
            cn = (on && e >= 0 && r < p.I) ? moe_row(w, e, p.I, r) : -1;
        }
        moe_load<BITS, GPB>(w, cn, blk, sidx, p.ngrp1, n, ns);
        float v = 0.f;
        const ScalesF32<GPB> fs(sc);
        if constexpr (XL) {
            if (cr >= 0) v = block_dot_lx<D, BITS, GPB>(a, xl, fs.v, cb);
        } else {
            if (cr >= 0) v = block_dot<D, BITS, GPB, true>(a, xr, fs.v, cb, uint32_t(w.K - 1));
        }
        v = group_sum(v, lpr);
        const int r = row_at(st);
        if (blk == lpr - 1 && r < p.I) vl[proj * p.rows_per_wg1 + (r - r_wg)] = v;
        cr = cn;
#pragma unroll
        for (int i = 0; i < BITS; ++i) a[i] = n[i];
#pragma unroll
        for (int g = 0; g < GPB; ++g) sc[g] = ns[g];
    }
    // routing / shared-gate outputs, once per token, after the weight loads:
    // before the barrier, waiting for these stores delayed this workgroup's
    // weights by a round trip, and with them the end of the kernel
    // (config 2: 11.89 -> 11.75 us per layer)
    if (bx == 0 && j == 0 && wave == 0) {
        if (my_idx < 0 || my_idx >= p.E) my_idx = -1;
        if (lane < p.top_k) {
            p.ids[t * p.top_k + lane] = my_idx;
            p.wts[t * p.top_k + lane] = my_w;
            if (p.ids_out) p.ids_out[t * p.top_k + lane] = my_idx;
            if (p.wts_out) p.wts_out[t * p.top_k + lane] = my_w;
        }
        if (p.shared) {
            const float acc = shared_gate_dot(p.x, p.x_type, p.sg_vec, p.sg_type, p.H, t);
            if (lane == 0) p.sg[t] = 1.f / (1.f + __expf(-acc));
        }
    }
    __syncthreads();
    if constexpr (TAG) {
        // rows in pairs (r_wg and I are even): word w = (row of the token's
        // P * I values) / 2, written through to device scope
        const uint32_t n = rl.call;
        const int64_t w0 = ((int64_t(t) * p.P + j) * p.I + r_wg) >> 1;
        for (int i = tid; 2 * i < p.rows_per_wg1; i += 2 * kThreads) {
            const int r = r_wg + 2 * i;
            if (r < p.I) {
                const uint32_t lo = f32_to_h(silu(vl[2 * i]) * vl[p.rows_per_wg1 + 2 * i]);
                const uint32_t hi = f32_to_h(silu(vl[2 * i + 1]) * vl[p.rows_per_wg1 + 2 * i + 1]);
                const uint32_t w = uint32_t(w0 + i);
                l1_store(p.l1_hw + w, (uint64_t(l1_tag(n, w)) << 32) | (hi << 16) | lo);
            }
        }
    } else {
        uint16_t *hrow = p.h + (int64_t(t) * p.P + j) * p.I;
        for (int i = tid; i < p.rows_per_wg1; i += 2 * kThreads) {
            const int r = r_wg + i;
            if (r < p.I) hrow[r] = f32_to_h(silu(vl[i]) * vl[p.rows_per_wg1 + i]);
        }
    }
}

template <int D, int BITS, int GPB>
__global__ void __launch_bounds__(2 * kThreads) k_moe_up(const MoeParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ RouteLds rl;
    up_fused<D, BITS, GPB, false>(p, smem, rl, int(blockIdx.x), int(blockIdx.y));
}

// K1 for tables beyond LDS: one projection per workgroup (blockIdx.z: 0 gate,
// 1 up), so its table gets the LDS of two (the first kHybSplitBytes of it)
// and more of the codes read LDS instead of L2 -- the request rate that
// bounds these tables. The rows go out as fp32; K2 builds silu(g) * u from
// them as it stages its input.
constexpr int kHybSplitBytes = 128 * 1024;
constexpr int kHybSplitWideBytes = 150 * 1024;   // when x leaves room (the host checks)

template <int D, int BITS, int GPB, bool W = false>
__global__ void __launch_bounds__(moe_waves_up(W) * kWave) k_moe_up_split(const MoeParams p) {
    constexpr int CBN = (W ? kHybSplitWideBytes : kHybSplitBytes) / (2 * D);
    constexpr int NWV = moe_waves_up(W);
    constexpr int XH = kBlock * D, XS = XH + 8;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ RouteLds rl;
    h2 *cb_lds = reinterpret_cast<h2 *>(smem);
    f16 *xs = reinterpret_cast<f16 *>(smem + CBN * D * 2);

    const int bx = int(blockIdx.x), pair = int(blockIdx.y), proj = int(blockIdx.z);
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
    const int lpr = 1 << p.lpr1_log2, rpw = kWave >> p.lpr1_log2;
    const int sub = lane >> p.lpr1_log2, blk = lane & (lpr - 1);
    const bool on = blk < p.NB1;
    const int t = pair / p.P, j = pair % p.P;
    const bool is_shared = j >= p.top_k;
    const MoeW &w = proj == 0 ? (is_shared ? p.sgate : p.gate) : (is_shared ? p.sup : p.up);
    const float *lg = p.logits + int64_t(t) * p.E;

    // wave 0 routes with nothing else in flight; the other waves stage the table and x
    int my_idx = -1;
    float my_w = 0.f;
    if (wave == 0) {
        int e_pair;
        route(lg, p.E, p.top_k, p.norm, is_shared ? -1 : j, &rl.rs, &e_pair, &my_idx, &my_w);
        if (lane == 0) rl.route = e_pair;
    } else {
        constexpr int NT = NWV * kWave - kWave;
        stage_codebook_fixed<D, CBN, NT, 1>(w.codebook, w.K, cb_lds);
        stage_x<XH, XS>(p.x, p.x_type, int64_t(t) * p.H, p.H, p.NB1, xs, kWave, NT);
    }
    wait_vmem();
    __syncthreads();

    const int e_pair = rl.route;
    const int64_t e = is_shared ? 0 : ((e_pair >= 0 && e_pair < p.E) ? e_pair : -1);
    const int sidx = GPB == 1 ? blk / p.bpg1 : blk * GPB;
    const int r_wg = bx * p.rows_per_wg1;
    auto row_at = [&](int st) { return r_wg + (st * NWV + wave) * rpw + sub; };
    auto code_row = [&](int st) -> int64_t {
        const int r = row_at(st);
        return (on && e >= 0 && r < p.I) ? moe_row(w, e, p.I, r) : -1;
    };

    uint32_t a[BITS];
    uint32_t sc[GPB];
    int64_t cr = code_row(0);
    moe_load<BITS, GPB>(w, cr, blk, sidx, p.ngrp1, a, sc);
    // 8-wave (wide) instances read x from LDS per code; the others hold it
    h2 xr[W ? 1 : 16 * D];
    const f16 *xl = xs + (on ? blk : 0) * XS;
    if constexpr (!W) load_xregs<D>(xl, xr);
    const h2 *cbg = reinterpret_cast<const h2 *>(w.codebook);
    const uint32_t kl = uint32_t(min(w.K, CBN));
    float *out = (proj == 0 ? p.gbuf : p.ubuf) + (int64_t(t) * p.P + j) * p.I;
    for (int st = 0; st < p.steps1; ++st) {
        uint32_t n[BITS];
        uint32_t ns[GPB];
        const int64_t crn = st + 1 < p.steps1 ? code_row(st + 1) : -1;
        moe_load<BITS, GPB>(w, crn, blk, sidx, p.ngrp1, n, ns);
        float v = 0.f;
        const ScalesF32<GPB> fs(sc);
        if constexpr (W) {
            if (cr >= 0) v = block_dot_hyb_lx<D, BITS, GPB>(a, xl, fs.v, cb_lds, cbg, kl, uint32_t(w.K - 1));
        } else {
            if (cr >= 0) v = block_dot_hyb<D, BITS, GPB>(a, xr, fs.v, cb_lds, cbg, kl, uint32_t(w.K - 1));
        }
        v = group_sum(v, lpr);
        const int r = row_at(st);
        if (blk == lpr - 1 && r < p.I) out[r] = v;
        cr = crn;
#pragma unroll
        for (int i = 0; i < BITS; ++i) a[i] = n[i];
#pragma unroll
        for (int g = 0; g < GPB; ++g) sc[g] = ns[g];
    }
    // routing / shared-gate outputs, once per token, after the weight loads
    if (bx == 0 && j == 0 && proj == 0 && wave == 0) {
        if (my_idx < 0 || my_idx >= p.E) my_idx = -1;
        if (lane < p.top_k) {
            p.ids[t * p.top_k + lane] = my_idx;
            p.wts[t * p.top_k + lane] = my_w;
            if (p.ids_out) p.ids_out[t * p.top_k + lane] = my_idx;
            if (p.wts_out) p.wts_out[t * p.top_k + lane] = my_w;
        }
        if (p.shared) {
            const float acc = shared_gate_dot(p.x, p.x_type, p.sg_vec, p.sg_type, p.H, t);
            if (lane == 0) p.sg[t] = 1.f / (1.f + __expf(-acc));
        }
    }
}

// ------------------------------------------------------------ K2: down + combine
// Lane geometry of the down phase: lanes are (pair j, block) of one row,
// LPR2 = next_pow2(P * NB2) lanes per row.
struct DownLane {
    int lpr, rpw, sub, v, j, blk;
    bool on, is_shared;
    __device__ DownLane(const MoeParams &p) {
        const int lane = threadIdx.x & (kWave - 1);
        lpr = 1 << p.lpr2_log2;
        rpw = kWave >> p.lpr2_log2;
        sub = lane >> p.lpr2_log2;
        v = lane & (lpr - 1);
        j = v / p.NB2;
        blk = v % p.NB2;
        on = j < p.P;
        is_shared = on && j >= p.top_k;
    }
};

// Expert, router weight and first-step weights of this lane's pair for row
// tile `bx`; `eid(j)` / `wt(j)` give the routing and `sgv()` the shared
// expert's gate (workspace or LDS).
template <int BITS, int GPB, typename EID, typename WT, typename SGV>
__device__ __forceinline__ void down_prep(const MoeParams &p, int bx, int t, const DownLane &dl,
                                          EID eid, WT wt, SGV sgv, DownState<BITS, GPB> &ds) {
    const int wave = threadIdx.x >> 6;
    const MoeW &wd = dl.is_shared ? p.sdown : p.down;
    ds.e = -1;
    ds.wj = 0.f;
    if (dl.on) {
        if (dl.is_shared) { ds.e = 0; ds.wj = sgv(); }
        else {
            const int id = eid(dl.j);
            ds.e = (id >= 0 && id < p.E) ? id : -1;
            ds.wj = wt(dl.j);
        }
    }
    const int sidx = GPB == 1 ? dl.blk / p.bpg2 : dl.blk * GPB;
    const int r = bx * p.rows_per_wg2 + wave * dl.rpw + dl.sub;
    ds.cr = (ds.e >= 0 && r < p.H) ? moe_row(wd, ds.e, p.H, r) : -1;
    moe_load<BITS, GPB>(wd, ds.cr, dl.blk, sidx, p.ngrp2, ds.a, ds.s);
}

// Routed down table (all of it, or its first CBN entries) and, when the
// whole table fits, the shared expert's; a partly staged routed table leaves
// the shared expert's to L2.
template <int D, int CBN, bool CBL, int NTH = kThreads>
__device__ __forceinline__ void down_stage_cb(const MoeParams &p, uint8_t *smem) {
    stage_codebook_fixed<D, CBN, NTH>(p.down.codebook, p.down.K, reinterpret_cast<h2 *>(smem));
    if (CBL && p.shared)
        stage_codebook_fixed<D, CBN, NTH>(p.sdown.codebook, p.sdown.K,
                                          reinterpret_cast<h2 *>(smem + CBN * D * 2));
}

// First round of the token's SwiGLU rows in registers: kHFirst 16-byte
// chunks per thread, loaded with clamped indices and no branch, so a wait for
// a load issued before them counts exactly these. With fp32 gate / up rows
// (split phase) the loads read the start of those rows and go unused.
constexpr int kHFirst = 4;
struct HFirst {
    u32x4 v[kHFirst];
};

__device__ __forceinline__ void h_first_load(const MoeParams &p, int t, HFirst &hf) {
    const int ng = p.P * (p.I / 8);
    const uint16_t *src = p.gbuf ? reinterpret_cast<const uint16_t *>(p.gbuf) + int64_t(t) * p.P * p.I * 2
                                 : p.h + int64_t(t) * p.P * p.I;
#pragma unroll
    for (int u = 0; u < kHFirst; ++u) {
        const int g = min(int(threadIdx.x) + u * int(blockDim.x), ng - 1);
        hf.v[u] = *reinterpret_cast<const u32x4 *>(src + int64_t(g) * 8);
    }
}

// The token's P SwiGLU rows (fp16) -> LDS at the padded block stride; the
// first kHFirst chunks per thread of fp16 rows come from `hf`. With fp32
// gate / up rows (split phase) they are built as fp16(silu(g) * u) here.
template <int D>
__device__ __forceinline__ void down_stage_h(const MoeParams &p, int t, f16 *xs, const HFirst &hf) {
    constexpr int XH = kBlock * D, XS = XH + 8;
    const int tid = threadIdx.x;
    const uint16_t *hsrc = p.h + int64_t(t) * p.P * p.I;
    const int64_t f0 = int64_t(t) * p.P * p.I;   // split phase: fp32 g / u rows
    const int gpr = p.I / 8;                     // 8-value groups per row
    const int ng = p.P * gpr;
    constexpr int U = 8;
    int gs = tid;
    if (!p.gbuf) {
#pragma unroll
        for (int u = 0; u < kHFirst; ++u) {
            const int g = tid + u * int(blockDim.x);
            if (g < ng) {
                const int jj = g / gpr, col = (g % gpr) * 8;
                const int b = jj * p.NB2 + col / XH;
                *reinterpret_cast<u32x4 *>(xs + b * XS + col % XH) = hf.v[u];
            }
        }
        gs = tid + kHFirst * int(blockDim.x);
    }
    for (int g0 = gs; g0 < ng; g0 += U * blockDim.x) {
        u32x4 hv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int g = g0 + u * blockDim.x;
            if (p.gbuf)
                hv[u] = g < ng ? swiglu8(p.gbuf + f0 + int64_t(g) * 8, p.ubuf + f0 + int64_t(g) * 8)
                               : u32x4{0, 0, 0, 0};
            else
                hv[u] = g < ng ? *reinterpret_cast<const u32x4 *>(hsrc + int64_t(g) * 8)
                               : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int g = g0 + u * blockDim.x;
            if (g < ng) {
                const int jj = g / gpr, col = (g % gpr) * 8;
                const int b = jj * p.NB2 + col / XH;
                *reinterpret_cast<u32x4 *>(xs + b * XS + col % XH) = hv[u];
            }
        }
    }
}

// The decode half of down_run, once the SwiGLU rows are in LDS: the down
// projection of the workgroup's rows, scaled per pair by its router weight
// and combined over the wave (the DPP row reduction is the sum).
template <int D, int BITS, int GPB, bool W = false>
__device__ __forceinline__ void down_decode(const MoeParams &p, int bx, int t, uint8_t *smem,
                                            const DownLane &dl, DownState<BITS, GPB> &ds) {
    constexpr bool CBL = cb_in_lds(D, BITS);
    constexpr int CBN = down_cbn<D, BITS, W>();
    constexpr int XH = kBlock * D, XS = XH + 8;
    h2 *cbd_lds = reinterpret_cast<h2 *>(smem);
    h2 *cbs_lds = reinterpret_cast<h2 *>(smem + CBN * D * 2);
    f16 *xs = reinterpret_cast<f16 *>(smem + ((CBL && p.shared) ? 2 : 1) * CBN * D * 2);
    const int tid = threadIdx.x, wave = tid >> 6;
    const MoeW &wd = dl.is_shared ? p.sdown : p.down;

    h2 xr[W ? 1 : 16 * D];                  // wide (8-wave) instances read x from LDS
    const f16 *xl = xs + (dl.on ? dl.j * p.NB2 + dl.blk : 0) * XS;
    if constexpr (!W) load_xregs<D>(xl, xr);
    const h2 *cb = CBL ? (dl.is_shared ? cbs_lds : cbd_lds)
                       : reinterpret_cast<const h2 *>(wd.codebook);
    const uint32_t kmax = uint32_t(wd.K - 1);
    const uint32_t kl = dl.is_shared ? 0u : uint32_t(min(wd.K, CBN));     // partly staged: routed only
    const int sidx = GPB == 1 ? dl.blk / p.bpg2 : dl.blk * GPB;
    const int r_wg = bx * p.rows_per_wg2;
    auto row_at = [&](int st) { return r_wg + (st * moe_waves_down(W) + wave) * dl.rpw + dl.sub; };
    auto code_row = [&](int st) -> int64_t {
        const int r = row_at(st);
        return (ds.e >= 0 && r < p.H) ? moe_row(wd, ds.e, p.H, r) : -1;
    };

    for (int st = 0; st < p.steps2; ++st) {
        uint32_t n[BITS];
        uint32_t ns[GPB];
        const int64_t crn = st + 1 < p.steps2 ? code_row(st + 1) : -1;
        moe_load<BITS, GPB>(wd, crn, dl.blk, sidx, p.ngrp2, n, ns);
        float acc = 0.f;
        const ScalesF32<GPB> fs(ds.s);
        if constexpr (CBL) {
            // all of the block's table reads first (four waves, one per SIMD):
            // 11.91 -> 11.88 us per config-2 layer
            if (ds.cr >= 0) acc = ds.wj * block_dot_all<D, BITS, GPB>(ds.a, xr, fs.v, cb);
        } else if constexpr (W) {
            if (ds.cr >= 0) acc = ds.wj * block_dot_hyb_lx<D, BITS, GPB>(ds.a, xl, fs.v, cbd_lds, cb, kl, kmax);
        } else {
            if (ds.cr >= 0) acc = ds.wj * block_dot_hyb<D, BITS, GPB>(ds.a, xr, fs.v, cbd_lds, cb, kl, kmax);
        }
        acc = group_sum(acc, dl.lpr);
        const int r = row_at(st);
        if (dl.v == dl.lpr - 1 && r < p.H) store_act(p.y, p.y_type, int64_t(t) * p.H + r, acc);
        ds.cr = crn;
#pragma unroll
        for (int i = 0; i < BITS; ++i) ds.a[i] = n[i];
#pragma unroll
        for (int g = 0; g < GPB; ++g) ds.s[g] = ns[g];
    }
}

// The token's P SwiGLU rows (fp16) -> LDS at the padded block stride, then
// the down projection of the workgroup's rows, scaled per pair by its router
// weight and combined over the wave (the DPP row reduction is the sum). The
// first kHFirst chunks per thread of fp16 rows come from `hf`.
template <int D, int BITS, int GPB, bool W = false>
__device__ __forceinline__ void down_run(const MoeParams &p, int bx, int t, uint8_t *smem,
                                         const DownLane &dl, DownState<BITS, GPB> &ds,
                                         const HFirst &hf) {
    constexpr bool CBL = cb_in_lds(D, BITS);
    constexpr int CBN = down_cbn<D, BITS, W>();
    f16 *xs = reinterpret_cast<f16 *>(smem + ((CBL && p.shared) ? 2 : 1) * CBN * D * 2);
    down_stage_h<D>(p, t, xs, hf);
    wait_vmem();
    __syncthreads();
    down_decode<D, BITS, GPB, W>(p, bx, t, smem, dl, ds);
}

template <int D, int BITS, int GPB, bool W = false>
__global__ void __launch_bounds__(moe_waves_down(W) * kWave) k_moe_down(const MoeParams p) {
    constexpr int CBN = down_cbn<D, BITS, W>();
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = int(blockIdx.y);
    const DownLane dl(p);
    // Load order (a wave's vector-memory loads complete in issue order): the
    // routing first, since the weight addresses wait on it; then the first
    // round of the SwiGLU rows, which waits on nothing; then, once the
    // routing is in, the weights and the table copy. The routing loads take a
    // clamped pair index and the h loads no branch, so the wait before the
    // weight loads holds only for the routing.
    const int jc = min(dl.j, p.top_k - 1);
    int id = p.ids[t * p.top_k + jc];
    float wt = p.wts[t * p.top_k + jc];
    HFirst hf;
    h_first_load(p, t, hf);
    if (!dl.on || dl.is_shared) {
        id = -1;
        wt = 0.f;
    }
    DownState<BITS, GPB> ds;
    down_prep<BITS, GPB>(p, int(blockIdx.x), t, dl, [&](int) { return id; },
                         [&](int) { return wt; }, [&] { return p.sg[t]; }, ds);
    down_stage_cb<D, CBN, cb_in_lds(D, BITS), moe_waves_down(W) * kWave>(p, smem);
    down_run<D, BITS, GPB, W>(p, int(blockIdx.x), t, smem, dl, ds, hf);
}

// ------------------------------------------------------------ one launch
// Both phases of a layer in one launch, for tables that fit LDS (with a
// shared expert: its down table beside the routed one, its gate taken by each
// down workgroup's routing wave) and a grid that is resident at once (two
// workgroups per CU):
// workgroups [0, G1) run the gate/up phase as k_moe_up does, and
// [G1, G1 + G2) the down phase of one row tile of one token. A down
// workgroup routes its token itself (the same routine, hence the same
// experts and weights), stages its table, loads its weights and looks up its
// block's table entries while the gate/up phase runs, then polls the tagged
// SwiGLU words of its token and finishes k_moe_down's arithmetic (same order,
// same bits) with the dot products. So the layer costs one kernel boundary,
// and the down weights' latency and table gathers overlap the gate/up phase
// instead of following the routing read of a second launch.
// The call number n lives in the workspace header: every workgroup reads it
// at its start and then writes its stamp; workgroup 0, once every stamp shows
// n, writes n + 1 for the next call, which starts after this launch ends.
// Gate/up workgroups never wait on anything and are dispatched first (lower
// ids); the down workgroups and workgroup 0 wait on them, each wait bounded
// (l1_spins). A wait that gives up is reported, never computed through: the
// missing words enter as NaN and the header's error word is set.
struct L1Lds {
    RouteLds rl;
    int ids[kMaxTopK];
    float wts[kMaxTopK];
    float sg;            // down workgroups: the shared expert's gate (layers with one)
    uint64_t call_bad;   // down workgroups: call number | (error word set at the start) << 32
};
// Waves of a down workgroup that decode rows (all of them stage, route and
// poll): eight, i.e. 16 rows per workgroup and 128 down workgroups at
// config 2. With the table entries looked up before the SwiGLU words arrive,
// the decode after them is short, and fewer workgroups polling the words
// shorten the hand-off: four decoding waves over 256 workgroups measured
// 10.33 us per config-2 layer against 10.0 for eight over 128.
constexpr int kL1DownWaves = 8;

template <int D, int BITS, int GPB, bool SH>
__device__ __forceinline__ void l1_down(const MoeParams &p, uint8_t *smem, L1Lds &ll, int cbi) {
    constexpr int CBN = 1 << BITS;                 // the whole table (the host checks it fits)
    constexpr int XH = kBlock * D, XS = XH + 8;
    constexpr int NT = 2 * kThreads;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
    const int bx = cbi % p.l1_gx2, t = cbi / p.l1_gx2;
    // LDS: the routed down table, the SwiGLU rows at a fixed offset (their
    // reads and writes after the hand-off keep constant address offsets),
    // then a shared expert's down table; the instance without a shared
    // expert (SH false) carries none of its code (a runtime flag cost 0.03-0.05
    // us per config-2 layer)
    f16 *xs = reinterpret_cast<f16 *>(smem + CBN * D * 2);
    const int sh_off = CBN * D * 2 + p.P * p.NB2 * XS * 2;
    // the last wave routes (the gate/up workgroup beside it on the CU routes
    // on its wave 0, and two routing waves on one SIMD slow both: 9.99 ->
    // 9.83 us per config-2 layer) and, with a shared expert, takes its gate
    // with the routine the gate/up workgroup 0 uses (the same bits); the
    // others stage the down tables (routed, then shared)
    uint64_t ev = 0, er = 0;
    if (wave == NT / kWave - 1) {
        int e_pair, my_idx = -1;
        float my_w = 0.f;
        route_upto<kL1Slots>(p.logits + int64_t(t) * p.E, p.E, p.top_k, p.norm, -1, &ll.rl.rs, &e_pair, &my_idx,
                             &my_w);
        if (lane < p.top_k) {
            ll.ids[lane] = (my_idx >= 0 && my_idx < p.E) ? my_idx : -1;
            ll.wts[lane] = my_w;
        }
        if constexpr (SH) {
            const float acc = shared_gate_dot(p.x, p.x_type, p.sg_vec, p.sg_type, p.H, t);
            if (lane == 0) ll.sg = 1.f / (1.f + __expf(-acc));
        }
    } else {
        if (tid == 0) {
            ev = l1_load(p.l1_epoch);
            er = l1_load(p.l1_err);
        }
        stage_codebook_fixed<D, CBN, NT - kWave, 0>(p.down.codebook, p.down.K, reinterpret_cast<h2 *>(smem));
        if constexpr (SH)
            stage_codebook_fixed<D, CBN, NT - kWave, 0>(p.sdown.codebook, p.sdown.K,
                                                        reinterpret_cast<h2 *>(smem + sh_off));
    }
    wait_vmem();
    if (tid == 0) {
        ll.call_bad = (uint64_t(er != 0) << 32) | uint32_t(ev);
        l1_store(p.l1_stamp + p.l1_g1 + cbi, l1_stamp(uint32_t(ev)));
    }
    __syncthreads();
    const DownLane dl(p);
    DownState<BITS, GPB> ds;
    const bool dec = wave < kL1DownWaves;
    if (dec) {
        down_prep<BITS, GPB>(p, bx, t, dl, [&](int j) { return ll.ids[j]; }, [&](int j) { return ll.wts[j]; },
                             [&] { return ll.sg; }, ds);
        // the weights land here, before the polls: left to itself the
        // compiler sinks these loads past the poll loop and the barrier (it is
        // short of registers), which put a whole memory latency between the
        // SwiGLU words' arrival and the decode
#pragma unroll
        for (int i = 0; i < BITS; ++i) asm volatile("" ::"v"(ds.a[i]));
#pragma unroll
        for (int g = 0; g < GPB; ++g) asm volatile("" ::"v"(ds.s[g]));
    }
    // The block's 32 table entries, looked up while the gate/up phase still
    // runs: the LDS gathers (bank-conflicted random reads, the decode's
    // largest cost) leave only the dot products with x for after the SwiGLU
    // words arrive. Held in registers (pinned, or the compiler would sink
    // the reads past the polls).
    typedef typename EntryT<D>::type Ent;
    struct EntW { uint32_t w[D / 2]; };
    EntW ent[kBlock];
    {
        const Ent *cbe = reinterpret_cast<const Ent *>(smem + ((SH && dl.is_shared) ? sh_off : 0));
        const bool live = dec && ds.cr >= 0;
#pragma unroll
        for (int i = 0; i < kBlock; ++i) {
            ent[i] = __builtin_bit_cast(EntW, cbe[live ? block_field<BITS>(ds.a, i) : 0u]);
#pragma unroll
            for (int k2 = 0; k2 < D / 2; ++k2) asm volatile("" : "+v"(ent[i].w[k2]));
        }
    }
    // the token's SwiGLU words: each thread polls up to four at a time until
    // their tags are the call's, then writes their halves into LDS. A word
    // still missing once l1_spins rounds have passed (or at once, after an
    // earlier call's error) enters as two fp16 NaNs, so every row whose dot
    // products would have used it comes out NaN, and its thread sets the
    // error word. (A workgroup-wide give-up flag in LDS, set before the
    // barrier, cost 0.15 us per config-2 layer.)
    const uint64_t cb = ll.call_bad;               // one LDS read ahead of the polls
    const uint32_t n = uint32_t(cb);
    const bool skip = (cb >> 32) != 0;
    const int bound = skip ? 0 : p.l1_spins;
    const int nwd = p.P * p.I / 2;
    const int64_t w0 = int64_t(t) * nwd;
    for (int g0 = tid; g0 < nwd; g0 += 4 * NT) {
        uint64_t v[4] = {0, 0, 0, 0};
        uint32_t need = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (g0 + u * NT < nwd) need |= 1u << u;
        for (int spin = 0; need && spin < bound; ++spin) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if ((need >> u) & 1u) v[u] = l1_load(p.l1_hw + w0 + g0 + u * NT);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (((need >> u) & 1u) &&
                    uint32_t(v[u] >> 32) == l1_tag(n, uint32_t(w0 + g0 + u * NT)))
                    need &= ~(1u << u);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int g = g0 + u * NT;
            if (g < nwd) {
                const int jj = (2 * g) / p.I, col = (2 * g) % p.I;
                const int b = jj * p.NB2 + col / XH;
                *reinterpret_cast<uint32_t *>(xs + b * XS + col % XH) =
                    ((need >> u) & 1u) ? 0x7E007E00u : uint32_t(v[u]);
            }
        }
        if (need && !skip)
            __hip_atomic_fetch_or(p.l1_err, kL1ErrPoll, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (dec) {
        // the block's dot products with its x chunk, in block_dot_lx's order
        constexpr int CPG = kBlock / GPB;
        const Ent *xv = reinterpret_cast<const Ent *>(xs + (dl.on ? dl.j * p.NB2 + dl.blk : 0) * XS);
        float acc = 0.f;
        if (ds.cr >= 0) {
            const ScalesF32<GPB> fs(ds.s);
            float bsum = 0.f;
#pragma unroll
            for (int g = 0; g < GPB; ++g) {
                float ga = 0.f;
#pragma unroll
                for (int q = 0; q < CPG; ++q) {
                    const int i = g * CPG + q;
                    const Ent x = xv[i];
                    h2 xh[D / 2];
#pragma unroll
                    for (int k2 = 0; k2 < D / 2; ++k2) xh[k2] = h2{x[2 * k2], x[2 * k2 + 1]};
                    ga = dot_vec<D>(__builtin_bit_cast(Ent, ent[i]), xh, ga);
                }
                bsum = fmaf(fs.v[g], ga, bsum);
            }
            acc = ds.wj * bsum;
        }
        acc = group_sum(acc, dl.lpr);
        const int r = bx * p.rows_per_wg2 + wave * dl.rpw + dl.sub;
        if (dl.v == dl.lpr - 1 && r < p.H)
            store_act(p.y, p.y_type, int64_t(t) * p.H + r, acc);
    }
}

template <int D, int BITS, int GPB, bool SH>
__global__ void __launch_bounds__(2 * kThreads, 4) k_moe_layer1(const MoeParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ L1Lds ll;
    const int b = int(blockIdx.x);
    if (b < p.l1_g1) {
        const int bx = b % p.l1_gx1, pair = b / p.l1_gx1;
        up_fused<D, BITS, GPB, true>(p, smem, ll.rl, bx, pair);
        if (b == 0) {
            // every workgroup has read the call number once its stamp shows
            // it: advance it for the next call (or, if a stamp never came,
            // report that and leave it)
            const uint32_t n = ll.rl.call;
            const int nwg = p.l1_g1 + p.l1_gx2 * p.T;
            int miss = 0;
            for (int i = int(threadIdx.x); i < nwg; i += 2 * kThreads) {
                int spin = 0;
                while (l1_load(p.l1_stamp + i) != l1_stamp(n))
                    if (++spin >= p.l1_spins) {
                        miss = 1;
                        break;
                    }
            }
            const bool lost = __syncthreads_or(miss) != 0;
            if (threadIdx.x == 0) {
                if (lost)
                    __hip_atomic_fetch_or(p.l1_err, kL1ErrStamp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else
                    l1_store(p.l1_epoch, uint64_t(n + 1u));
            }
        }
    } else {
        l1_down<D, BITS, GPB, SH>(p, smem, ll, b - p.l1_g1);
    }
}

// ------------------------------------------------ codebooks beyond LDS
// For tables the block-per-lane kernels would gather from L2 (config 3:
// d8 K16384), the layer is composed of four launches: routing (one wave per
// token), the sliced-codebook GEMV over routed + shared gate/up, the same
// over routed + shared down with silu(g) * u built as its input, and the
// weighted combine.
__global__ void __launch_bounds__(kWave) k_route_tokens(const MoeParams p) {
    __shared__ RouteScratch rs;
    const int t = int(blockIdx.x), lane = int(threadIdx.x);
    int e_pair, my_idx = -1;
    float my_w = 0.f;
    route(p.logits + int64_t(t) * p.E, p.E, p.top_k, p.norm, -1, &rs, &e_pair, &my_idx, &my_w);
    if (my_idx < 0 || my_idx >= p.E) my_idx = -1;
    if (lane < p.top_k) {
        p.ids[t * p.top_k + lane] = my_idx;
        p.wts[t * p.top_k + lane] = my_w;
        if (p.ids_out) p.ids_out[t * p.top_k + lane] = my_idx;
        if (p.wts_out) p.wts_out[t * p.top_k + lane] = my_w;
    }
    if (p.shared) {
        const float acc = shared_gate_dot(p.x, p.x_type, p.sg_vec, p.sg_type, p.H, t);
        if (lane == 0) p.sg[t] = 1.f / (1.f + __expf(-acc));
    }
}

// y[t, r] = sum_j w[t, j] * yd[t * k + j, r] + sg[t] * ysh[t, r]
__global__ void __launch_bounds__(256) k_moe_combine(const MoeParams p, const float *yd,
                                                     const float *ysh) {
    const int t = int(blockIdx.y);
    const int r = int(blockIdx.x) * 256 + int(threadIdx.x);
    if (r >= p.H) return;
    float acc = 0.f;
    for (int j = 0; j < p.top_k; ++j)
        acc += p.wts[t * p.top_k + j] * yd[(int64_t(t) * p.top_k + j) * p.H + r];
    if (p.shared) acc += p.sg[t] * ysh[int64_t(t) * p.H + r];
    store_act(p.y, p.y_type, int64_t(t) * p.H + r, acc);
}

// ------------------------------------------------------------ host side
static size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }

// Offsets in a layer workspace. Every layout starts with the one-launch
// header (kHdrBytes: call number, error word, stamps, hand-off words), so no
// other path, geometry or T ever writes into it.
struct MoeLayout {
    size_t ids, wts, sg, h, total;
    size_t g, u, sgg, sgu, yd, ysh;      // composed paths (sliced-codebook GEMV, grouped GEMM)
    size_t sort;                         // grouped path: pair order and tile records
    size_t gs, us;                       // fused path, split K1: fp32 gate / up rows
};

// Paths of the layer: the two fused decode kernels, the sliced-codebook GEMV
// composition (codebooks beyond LDS, batch >= 2), the grouped-GEMM
// composition (many pairs).
enum MoePath { kMoeFused = 0, kMoeBig = 1, kMoeGrouped = 2 };

static MoeLayout moe_layout(int64_t T, int k, int P, int64_t I, int64_t H, int path, int64_t E,
                            bool split) {
    MoeLayout L;
    L.ids = kHdrBytes;
    L.wts = align_up(L.ids + sizeof(int32_t) * T * k);
    L.sg = align_up(L.wts + sizeof(float) * T * k);
    L.h = align_up(L.sg + sizeof(float) * T);
    L.total = align_up(L.h + (path == kMoeFused && !split ? 2 * size_t(T) * P * I : 0));
    L.g = L.u = L.sgg = L.sgu = L.yd = L.ysh = L.sort = L.gs = L.us = 0;
    if (path == kMoeFused && split) {
        L.gs = L.total;
        L.us = align_up(L.gs + 4 * size_t(T) * P * I);
        L.total = align_up(L.us + 4 * size_t(T) * P * I);
    }
    if (path != kMoeFused) {
        // grouped: the shared gate / up rows as up to 4 K-slice partials
        const size_t nsh = path == kMoeGrouped ? 4 : 1;
        L.g = L.total;
        L.u = align_up(L.g + 4 * size_t(T) * k * I);
        L.sgg = align_up(L.u + 4 * size_t(T) * k * I);
        L.sgu = align_up(L.sgg + 4 * nsh * size_t(T) * I);
        L.yd = align_up(L.sgu + 4 * nsh * size_t(T) * I);
        L.ysh = align_up(L.yd + 4 * size_t(T) * k * H);
        L.total = align_up(L.ysh + 4 * size_t(T) * H);
    }
    if (path == kMoeGrouped) {
        L.sort = L.total;
        L.total = align_up(L.sort + seg_sort_bytes(T * k, E));
    }
    return L;
}

static bool same_format(const Geom &a, const Geom &b) {
    return a.D == b.D && a.BITS == b.BITS && a.packed == b.packed && a.G == b.G &&
           a.OUT == b.OUT && a.IN == b.IN && a.gpb == b.gpb && a.bpg == b.bpg;
}

static void fill_moew(const vqk_weights *w, const Geom &g, MoeW *m) {
    m->codes = static_cast<const uint32_t *>(w->codes);
    m->codebook = w->codebook;
    m->scales = w->scales;
    m->row_table = w->row_table;
    m->row_words = g.row_words;
    m->stored_rows = g.rows;
    m->K = int32_t(g.K);
}

struct MoePlan {
    Geom g1, g2;
    MoeParams p;
    MoeLayout lay;
    size_t smem1, smem2;
    dim3 grid1, grid2;
    int path;                 // MoePath
    bool split;               // fused path, tables beyond LDS: one projection per K1 workgroup
    bool wide1, wide2;        // the larger LDS parts of a partly staged table fit
    bool l1;                  // fused path as one launch (k_moe_layer1)
    size_t smem_l1;
    int l1_nwg;               // its workgroups
};

// Test hooks (vqk__test_*, not part of include/vqk.h): the bound of the
// one-launch layer's waits, and a switch that keeps every call on the other
// paths, so tests can force a give-up and compare the two forms.
static std::atomic<int> g_l1_spins{kL1Spins};
static std::atomic<int> g_l1_mode{0};        // 0 = one launch where it applies, 1 = never

// Widths of the one-launch layer's instances: tables of 256 to 4096 entries
// at d 2 and 4, with their scale-group blocking.
static bool l1_instance(int d, int bits, int gpb) {
    return ((d == 2 && gpb == 1) || (d == 4 && gpb == 2)) && bits >= 8 && bits <= 12;
}

static int lg2(int64_t v) {
    int l = 0;
    while ((int64_t(1) << l) < v) ++l;
    return l;
}

static int moe_plan(const vqk_moe_desc *m, int64_t T, MoePlan *pl) {
    if (!m || !m->gate || !m->up || !m->down)
        return set_error(VQK_EINVAL, "moe layer: gate, up and down are required");
    Geom gg, gu, gd;
    int rc;
    if ((rc = make_geom(m->gate, &gg)) || (rc = make_geom(m->up, &gu)) || (rc = make_geom(m->down, &gd)))
        return rc;
    if (!same_format(gg, gu) || gg.E != gu.E)
        return set_error(VQK_ENOTIMPL, "fused layer: gate and up must share one format");
    if (gd.E != gg.E || gd.OUT != gg.IN || gd.IN != gg.OUT)
        return set_error(VQK_EINVAL, "fused layer: down must be [E, H, I] for gate/up [E, I, H]");
    const bool shared = m->sh_gate != nullptr;
    if (shared) {
        Geom sg1, su1, sd1;
        if (!m->sh_up || !m->sh_down || !m->sh_gate_vec)
            return set_error(VQK_EINVAL, "shared expert needs gate, up, down and the gate vector");
        if ((rc = make_geom(m->sh_gate, &sg1)) || (rc = make_geom(m->sh_up, &su1)) ||
            (rc = make_geom(m->sh_down, &sd1)))
            return rc;
        if (sg1.E != 1 || su1.E != 1 || sd1.E != 1)
            return set_error(VQK_EINVAL, "shared expert projections have E=1");
        if (!same_format(sg1, gg) || !same_format(su1, gg) || !same_format(sd1, gd))
            return set_error(VQK_ENOTIMPL, "fused layer: shared expert must share the routed formats");
        if (!sg1.fast_ok || !su1.fast_ok || !sd1.fast_ok)
            return set_error(VQK_ENOTIMPL, "fused layer: shared expert outside the fast kernels");
        if (!act_size(m->sh_gate_vec_type)) return set_error(VQK_EINVAL, "bad shared gate vector type");
    }
    const int64_t E = gg.E;
    const int k = m->top_k;
    if (E > kMaxExperts) return set_error(VQK_ENOTIMPL, "fused layer: E=%lld > %d", (long long)E, kMaxExperts);
    if (k < 1 || k > E || k > kMaxTopK) return set_error(VQK_EINVAL, "top_k=%d outside [1, min(E, %d)]", k, kMaxTopK);
    if (!gg.fast_ok || !gu.fast_ok || !gd.fast_ok)
        return set_error(VQK_ENOTIMPL, "fused layer: shape outside the fast kernels (ragged / NB > 64)");
    const int P = k + (shared ? 1 : 0);
    if (P * gd.NB > kWave)
        return set_error(VQK_ENOTIMPL, "fused layer: %d pairs x %lld blocks exceed one wave", P,
                         (long long)gd.NB);
    if (T < 0 || T > 65535) return set_error(VQK_EINVAL, "T=%lld", (long long)T);
    pl->g1 = gg;
    pl->g2 = gd;
    MoeParams &p = pl->p;
    memset(&p, 0, sizeof p);
    fill_moew(m->gate, gg, &p.gate);
    fill_moew(m->up, gu, &p.up);
    fill_moew(m->down, gd, &p.down);
    if (shared) {
        Geom a;
        make_geom(m->sh_gate, &a); fill_moew(m->sh_gate, a, &p.sgate);
        make_geom(m->sh_up, &a);   fill_moew(m->sh_up, a, &p.sup);
        make_geom(m->sh_down, &a); fill_moew(m->sh_down, a, &p.sdown);
    } else {
        p.sgate = p.gate; p.sup = p.up; p.sdown = p.down;
    }
    p.shared = shared;
    p.E = int32_t(E);
    p.top_k = k;
    p.norm = m->norm_topk ? 1 : 0;
    p.H = int32_t(gg.IN);
    p.I = int32_t(gg.OUT);
    p.NB1 = int32_t(gg.NB);
    p.NB2 = int32_t(gd.NB);
    p.ngrp1 = int32_t(gg.NGRP);
    p.ngrp2 = int32_t(gd.NGRP);
    p.bpg1 = gg.bpg;
    p.bpg2 = gd.bpg;
    p.lpr1_log2 = lg2(gg.NB);
    p.lpr2_log2 = lg2(int64_t(P) * gd.NB);
    p.T = int32_t(T);
    p.P = P;
    p.sg_vec = m->sh_gate_vec;
    p.sg_type = m->sh_gate_vec_type;
    const bool full1 = cb_in_lds(gg.D, gg.BITS), full2 = cb_in_lds(gd.D, gd.BITS);
    pl->split = !full1;
    const size_t cb1 = full1 ? (size_t(1) << gg.BITS) * gg.D * 2 : size_t(kHybUpBytes);
    const size_t cb2 = full2 ? (size_t(1) << gd.BITS) * gd.D * 2 : size_t(kHybDownBytes);
    const size_t xs1 = size_t(gg.NB) * (kBlock * gg.D + 8) * 2;
    const size_t xs2 = size_t(P) * gd.NB * (kBlock * gd.D + 8) * 2;
    // LDS a workgroup may take, kept clear of the 160 KB by the gate/up
    // kernels' static routing block (and slack for alignment); the down kernel
    // has no static LDS
    const size_t lds_room = 160 * 1024 - sizeof(RouteLds) - 256;
    const size_t lds_room2 = 160 * 1024 - 256;
    pl->wide1 = pl->split && gg.K * gg.D * 2 > kHybSplitBytes && kHybSplitWideBytes + xs1 <= lds_room;
    pl->wide2 = !full2 && gd.K * gd.D * 2 > kHybDownBytes && kHybDownWideBytes + xs2 <= lds_room2;
    pl->smem1 = (pl->split ? size_t(pl->wide1 ? kHybSplitWideBytes : kHybSplitBytes) : 2 * cb1) + xs1;
    pl->smem2 = ((shared && full2) ? 2 : 1) * (pl->wide2 ? size_t(kHybDownWideBytes) : cb2) + xs2;
    // Row steps per workgroup: about 2048 row steps per launch spread over the
    // grid; a workgroup whose LDS leaves room for no second one on a CU gets
    // enough steps that the grid fits the CUs in one round (each round would
    // repeat the routing, the table copy and the first weight latency).
    const int64_t target = 2048, ncu = big_grid(int64_t(1) << 30);
    auto plan_steps = [&](int64_t row_steps, int64_t cols, size_t smem, int nw, int32_t *steps) {
        int64_t st = (row_steps * cols + target - 1) / target;
        st = st < 1 ? 1 : (st > 16 ? 16 : st);
        if (smem > 80 * 1024) {     // one workgroup per CU: the fewest steps that fit one round
            st = 1;
            while (st < 16 && ((row_steps + nw * st - 1) / (nw * st)) * cols > ncu) ++st;
        }
        *steps = int32_t(st);
    };
    {   // K1: T*P pairs x I rows (x 2 projections when split)
        const int rpw = kWave >> p.lpr1_log2;
        const int nz = pl->split ? 2 : 1;
        const int nw = moe_waves_up(pl->wide1);
        plan_steps((gg.OUT + rpw - 1) / rpw, T * P * nz, pl->smem1, nw, &p.steps1);
        if (!pl->split) {
            // the tile's gate and up values meet in LDS after x (8 B per row)
            while (p.steps1 > 1 && pl->smem1 + 16 + 8 * size_t(nw * rpw * p.steps1) > lds_room) --p.steps1;
            pl->smem1 += 16 + 8 * size_t(nw * rpw * p.steps1);
        }
        p.rows_per_wg1 = int32_t(nw * rpw * p.steps1);
        pl->grid1 = dim3(unsigned((gg.OUT + p.rows_per_wg1 - 1) / p.rows_per_wg1), unsigned(T * P),
                         unsigned(nz));
    }
    {   // K2: T tokens x H rows
        const int rpw = kWave >> p.lpr2_log2;
        const int nw = moe_waves_down(pl->wide2);
        plan_steps((gd.OUT + rpw - 1) / rpw, T, pl->smem2, nw, &p.steps2);
        p.rows_per_wg2 = int32_t(nw * rpw * p.steps2);
        pl->grid2 = dim3(unsigned((gd.OUT + p.rows_per_wg2 - 1) / p.rows_per_wg2), unsigned(T), 1);
    }
    // Many pairs: sort once and run each projection as a grouped matrix-core
    // GEMM (weights decoded once per tile of up to 16 pairs of an expert).
    // Batch >= 2 with tables beyond LDS: the sliced-codebook GEMV composition.
    // Otherwise the two fused kernels (partly LDS-staged tables).
    const int64_t N = T * k;
    // grouped: at least one pair per expert on average, or the sparser
    // routings whose d8 tables take the persistent narrow-tile path
    bool grouped = N >= kMoeGroupedMinPairs && (N >= E || seg_tile_rows(m->gate, N, E) < 16) &&
                   seg_ok(m->gate, N) && seg_ok(m->up, N) && seg_ok(m->down, N);
    if (grouped && shared)
        grouped = seg_ok(m->sh_gate, T) && seg_ok(m->sh_up, T) && seg_ok(m->sh_down, T);
    bool big = T >= 2 && big_fits(gg, m->gate) && big_fits(gu, m->up) && big_fits(gd, m->down);
    if (big && shared) {
        Geom a, b, c;
        make_geom(m->sh_gate, &a);
        make_geom(m->sh_up, &b);
        make_geom(m->sh_down, &c);
        big = big_fits(a, m->sh_gate) && big_fits(b, m->sh_up) && big_fits(c, m->sh_down);
    }
    pl->path = grouped ? kMoeGrouped : (big ? kMoeBig : kMoeFused);
    if (pl->path == kMoeFused && (pl->smem1 > 160 * 1024 || pl->smem2 > 160 * 1024))
        return set_error(VQK_ENOTIMPL, "fused layer: LDS need %zu / %zu B exceeds 160 KB",
                         pl->smem1, pl->smem2);
    pl->lay = moe_layout(T, k, P, gg.OUT, gg.IN, pl->path, E, pl->split);
    // One launch: batch 1, gate/up and down workgroups resident together, two
    // per CU (LDS and 128 VGPRs each), tables in LDS (a shared expert's down
    // table beside the routed one), one format, the stamps and words within
    // the header.
    pl->l1 = false;
    pl->smem_l1 = 0;
    pl->l1_nwg = 0;
    if (T == 1 && g_l1_mode.load() == 0 && pl->path == kMoeFused && !pl->split && full1 && full2 &&
        gg.D == gd.D && gg.BITS == gd.BITS && gg.gpb == gd.gpb && l1_instance(gg.D, gg.BITS, gg.gpb) &&
        E <= kL1Slots * kWave && pl->grid1.z == 1 && gg.OUT % 2 == 0 && p.rows_per_wg1 % 2 == 0 &&
        int64_t(P) * gg.OUT / 2 <= kL1MaxWords) {
        const int rpw2 = kWave >> p.lpr2_log2;
        const int64_t rows2 = int64_t(kL1DownWaves) * rpw2;
        const int64_t gx2 = (gd.OUT + rows2 - 1) / rows2;
        const int64_t g1 = int64_t(pl->grid1.x) * pl->grid1.y;
        const int64_t nwg = g1 + gx2 * T;
        const size_t sm = std::max(pl->smem1, (shared ? 2 : 1) * cb2 + xs2);
        if (nwg <= std::min<int64_t>(2 * ncu, kL1MaxWg) && 2 * (sm + sizeof(L1Lds) + 256) <= 160 * 1024) {
            pl->l1 = true;
            pl->smem_l1 = sm;
            pl->l1_nwg = int(nwg);
            p.l1_g1 = int32_t(g1);
            p.l1_gx1 = int32_t(pl->grid1.x);
            p.l1_gx2 = int32_t(gx2);
            p.rows_per_wg2 = int32_t(rows2);
            p.steps2 = 1;
            p.l1_spins = g_l1_spins.load();
        }
    }
    return VQK_OK;
}

int launch_moe_up(const MoeParams &p, int D, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st);
int launch_moe_down(const MoeParams &p, int D, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st);

template <int D, int BITS, int GPB>
static int go_up(const MoeParams &p, dim3 grid, size_t smem, hipStream_t st) {
    return launch_with_lds<k_moe_up<D, BITS, GPB>>(grid, dim3(2 * kThreads), smem, st, p);
}
template <int D, int BITS, int GPB, bool W>
static int go_up_split(const MoeParams &p, dim3 grid, size_t smem, hipStream_t st) {
    return launch_with_lds<k_moe_up_split<D, BITS, GPB, W>>(grid, dim3(moe_waves_up(W) * kWave), smem,
                                                            st, p);
}
// Split gate/up kernel: only the widths whose table exceeds the LDS-resident
// limit (d2 15-16 bits, d4 14-16, d8 13-16).
#define VQK_SPLIT_CASE(D, B, G) \
    if (d == D && bits == B && gpb == G)                                                   \
        return wide ? go_up_split<D, B, G, true>(p, grid, smem, st)                          \
                    : go_up_split<D, B, G, false>(p, grid, smem, st);
static int launch_moe_up_split(const MoeParams &p, int d, int bits, int gpb, bool wide, dim3 grid,
                               size_t smem, hipStream_t st) {
    VQK_SPLIT_CASE(2, 15, 1) VQK_SPLIT_CASE(2, 16, 1)
    VQK_SPLIT_CASE(4, 14, 2) VQK_SPLIT_CASE(4, 15, 2) VQK_SPLIT_CASE(4, 16, 2)
    VQK_SPLIT_CASE(8, 13, 4) VQK_SPLIT_CASE(8, 14, 4) VQK_SPLIT_CASE(8, 15, 4) VQK_SPLIT_CASE(8, 16, 4)
    return set_error(VQK_ENOTIMPL, "fused layer: no split gate/up kernel for d=%d bits=%d", d, bits);
}
template <int D, int BITS, int GPB, bool W = false>
static int go_down(const MoeParams &p, dim3 grid, size_t smem, hipStream_t st) {
    return launch_with_lds<k_moe_down<D, BITS, GPB, W>>(grid, dim3(moe_waves_down(W) * kWave), smem, st, p);
}
// Down kernel with the larger LDS part: the widths whose table is beyond LDS.
#define VQK_DNW_CASE(D, B, G) \
    if (d == D && bits == B && gpb == G) return go_down<D, B, G, true>(p, grid, smem, st);
static int launch_moe_down_wide(const MoeParams &p, int d, int bits, int gpb, dim3 grid, size_t smem,
                                hipStream_t st) {
    VQK_DNW_CASE(2, 15, 1) VQK_DNW_CASE(2, 16, 1)
    VQK_DNW_CASE(4, 14, 2) VQK_DNW_CASE(4, 15, 2) VQK_DNW_CASE(4, 16, 2)
    VQK_DNW_CASE(8, 13, 4) VQK_DNW_CASE(8, 14, 4) VQK_DNW_CASE(8, 15, 4) VQK_DNW_CASE(8, 16, 4)
    return set_error(VQK_ENOTIMPL, "fused layer: no wide down kernel for d=%d bits=%d", d, bits);
}
// Instances: every width for d in {2, 4, 8}, scale groups of 64 weights.
#define VQK_MOE_BITS(X, D, G) \
    X(D, 2, G) X(D, 3, G) X(D, 4, G) X(D, 5, G) X(D, 6, G) X(D, 7, G) X(D, 8, G) X(D, 9, G) \
    X(D, 10, G) X(D, 11, G) X(D, 12, G) X(D, 13, G) X(D, 14, G) X(D, 15, G) X(D, 16, G)
#define VQK_UP_CASE(D, B, G) if (d == D && bits == B && gpb == G) return go_up<D, B, G>(p, grid, smem, st);
#define VQK_DN_CASE(D, B, G) if (d == D && bits == B && gpb == G) return go_down<D, B, G>(p, grid, smem, st);

template <int D, int BITS, int GPB>
static int go_layer1(const MoeParams &p, dim3 grid, size_t smem, hipStream_t st) {
    if (p.shared) return launch_with_lds<k_moe_layer1<D, BITS, GPB, true>>(grid, dim3(2 * kThreads), smem, st, p);
    return launch_with_lds<k_moe_layer1<D, BITS, GPB, false>>(grid, dim3(2 * kThreads), smem, st, p);
}
#define VQK_L1_CASE(D, B, G) if (d == D && bits == B && gpb == G) return go_layer1<D, B, G>(p, grid, smem, st);
static int launch_moe_layer1(const MoeParams &p, int d, int bits, int gpb, dim3 grid, size_t smem,
                             hipStream_t st) {
    VQK_L1_CASE(2, 8, 1) VQK_L1_CASE(2, 9, 1) VQK_L1_CASE(2, 10, 1) VQK_L1_CASE(2, 11, 1) VQK_L1_CASE(2, 12, 1)
    VQK_L1_CASE(4, 8, 2) VQK_L1_CASE(4, 9, 2) VQK_L1_CASE(4, 10, 2) VQK_L1_CASE(4, 11, 2) VQK_L1_CASE(4, 12, 2)
    return set_error(VQK_ENOTIMPL, "fused layer: no one-launch kernel for d=%d bits=%d", d, bits);
}

int launch_moe_up(const MoeParams &p, int d, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st) {
    VQK_MOE_BITS(VQK_UP_CASE, 2, 1)
    VQK_MOE_BITS(VQK_UP_CASE, 4, 2)
    VQK_MOE_BITS(VQK_UP_CASE, 8, 4)
    return set_error(VQK_ENOTIMPL, "fused layer: no kernel for d=%d bits=%d (%d groups/block); "
                     "the fused layer takes scale groups of 64 weights", d, bits, gpb);
}

int launch_moe_down(const MoeParams &p, int d, int bits, int gpb, dim3 grid, size_t smem, hipStream_t st) {
    VQK_MOE_BITS(VQK_DN_CASE, 2, 1)
    VQK_MOE_BITS(VQK_DN_CASE, 4, 2)
    VQK_MOE_BITS(VQK_DN_CASE, 8, 4)
    return set_error(VQK_ENOTIMPL, "fused layer: no kernel for d=%d bits=%d (%d groups/block); "
                     "the fused layer takes scale groups of 64 weights", d, bits, gpb);
}

static void seg_of(const vqk_weights *w, BigSeg *s, const int32_t *eidx, int32_t N, int32_t xkrep,
                   int32_t wg0, int32_t wgpp, int32_t rows) {
    Geom g;
    make_geom(w, &g);
    big_seg_weights(w, g, s);
    s->eidx = eidx;
    s->N = N;
    s->xkrep = xkrep;
    s->wg0 = wg0;
    s->wg_per_pair = wgpp;
    s->rows_per_wg = rows;
}

static int launch_moe_big(const vqk_moe_desc *m, const MoePlan &pl, uint8_t *ws, hipStream_t st) {
    const MoeParams &p = pl.p;
    const int T = p.T, k = p.top_k;
    const bool sh = p.shared != 0;
    float *g = reinterpret_cast<float *>(ws + pl.lay.g), *u = reinterpret_cast<float *>(ws + pl.lay.u);
    float *sgg = reinterpret_cast<float *>(ws + pl.lay.sgg), *sgu = reinterpret_cast<float *>(ws + pl.lay.sgu);
    float *yd = reinterpret_cast<float *>(ws + pl.lay.yd), *ysh = reinterpret_cast<float *>(ws + pl.lay.ysh);
    hipLaunchKernelGGL(k_route_tokens, dim3(unsigned(T)), dim3(kWave), 0, st, p);
    int rc = hip_status(hipGetLastError(), "routing launch");
    if (rc) return rc;
    {   // gate / up, routed and shared: fp32 rows
        BigParams b;
        memset(&b, 0, sizeof b);
        const int rows = big_plan_rows(&b, pl.g1.NB, p.I, int64_t(T) * (sh ? k + 1 : k) * 2 * p.I);
        const int wgpp = (p.I + rows - 1) / rows;
        int wg0 = 0, ns = 0;
        const vqk_weights *mods[4] = {m->gate, m->up, m->sh_gate, m->sh_up};
        float *outs[4] = {g, u, sgg, sgu};
        for (int i = 0; i < (sh ? 4 : 2); ++i) {
            const bool routed = i < 2;
            const int32_t N = routed ? T * k : T;
            BigSeg &s = b.seg[ns++];
            seg_of(mods[i], &s, routed ? p.ids : nullptr, N, routed ? k : 1, wg0, wgpp, rows);
            s.x = p.x;
            s.x_type = p.x_type;
            s.x_stride = p.H;
            s.y = outs[i];
            s.y_type = VQK_F32;
            s.y_stride = p.I;
            wg0 += N * wgpp;
        }
        b.nseg = ns;
        b.IN = p.H;
        b.NB = int32_t(pl.g1.NB);
        if ((rc = launch_gemv_big(b, pl.g1.D, pl.g1.BITS, pl.g1.gpb, dim3(unsigned(big_grid(wg0))), st)))
            return rc;
    }
    {   // down, routed and shared, input silu(g) * u per pair
        BigParams b;
        memset(&b, 0, sizeof b);
        const int rows = big_plan_rows(&b, pl.g2.NB, p.H, int64_t(T) * (sh ? k + 1 : k) * p.H);
        const int wgpp = (p.H + rows - 1) / rows;
        int wg0 = 0, ns = 0;
        for (int i = 0; i < (sh ? 2 : 1); ++i) {
            const bool routed = i == 0;
            const int32_t N = routed ? T * k : T;
            BigSeg &s = b.seg[ns++];
            seg_of(routed ? m->down : m->sh_down, &s, routed ? p.ids : nullptr, N, 1, wg0, wgpp, rows);
            s.xg = routed ? g : sgg;
            s.xu = routed ? u : sgu;
            s.x_stride = p.I;
            s.y = routed ? yd : ysh;
            s.y_type = VQK_F32;
            s.y_stride = p.H;
            wg0 += N * wgpp;
        }
        b.nseg = ns;
        b.IN = p.I;
        b.NB = int32_t(pl.g2.NB);
        if ((rc = launch_gemv_big(b, pl.g2.D, pl.g2.BITS, pl.g2.gpb, dim3(unsigned(big_grid(wg0))), st)))
            return rc;
    }
    hipLaunchKernelGGL(k_moe_combine, dim3(unsigned((p.H + 255) / 256), unsigned(T)), dim3(256), 0, st,
                       p, static_cast<const float *>(yd), static_cast<const float *>(ysh));
    return hip_status(hipGetLastError(), "combine launch");
}

// The batched layer's second stream, one per device (default priority),
// created on first use and kept until the process ends, with the events that
// fork work onto it and join it back: [0] call start, [1] sort done, [2]
// routed up done, [3] shared expert done.
constexpr int kMaxSideDevices = 64;
struct SideStream {
    hipStream_t s = nullptr;
    hipEvent_t e[4] = {};
};
static std::mutex g_side_mu;
static SideStream g_side[kMaxSideDevices];

// The current device's side stream (g_side_mu held), or nullptr when it
// cannot be created or `st` belongs to another device (the layer then runs
// on the caller's stream alone).
static SideStream *side_stream_locked(hipStream_t st) {
    int dev = -1, sdev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxSideDevices ||
        (st && (hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev))) {
        (void)hipGetLastError();
        return nullptr;
    }
    SideStream &ss = g_side[dev];
    if (!ss.s) {
        // never create it while `st` is being captured into a graph: that
        // call runs on the caller's stream alone
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
            (void)hipGetLastError();
            return nullptr;
        }
        SideStream n;
        bool ok = hipStreamCreateWithFlags(&n.s, hipStreamNonBlocking) == hipSuccess;
        for (int i = 0; ok && i < 4; ++i)
            ok = hipEventCreateWithFlags(&n.e[i], hipEventDisableTiming) == hipSuccess;
        if (!ok) {
            (void)hipGetLastError();
            return nullptr;
        }
        ss = n;
    }
    return &ss;
}

// Many pairs: routing (one wave per token), one counting sort of the pairs by
// expert, gate and up as grouped GEMMs into fp32 rows, down as a grouped GEMM
// whose input rows are built as fp16(silu(g) * u) while they are staged, the
// shared expert as the same kernels over the token rows, and the weighted
// combine. The shared expert (independent of the routing) and the routed up
// projection run on the device's second stream beside the routing, the sort
// and the routed gate and down: a persistent launch leaves CUs idle in its
// last, partial round of items, and the other stream's workgroups fill them.
// A mutex holds the whole enqueue sequence, so calls from several host
// threads never interleave their event records; the fork / join pattern is
// also what a graph capture of the call records.
static int launch_moe_grouped(const vqk_moe_desc *m, const MoePlan &pl, uint8_t *ws, hipStream_t st) {
    const MoeParams &p = pl.p;
    const int64_t T = p.T, k = p.top_k, N = T * k;
    float *g = reinterpret_cast<float *>(ws + pl.lay.g), *u = reinterpret_cast<float *>(ws + pl.lay.u);
    float *sgg = reinterpret_cast<float *>(ws + pl.lay.sgg), *sgu = reinterpret_cast<float *>(ws + pl.lay.sgu);
    float *yd = reinterpret_cast<float *>(ws + pl.lay.yd), *ysh = reinterpret_cast<float *>(ws + pl.lay.ysh);
    void *sort = ws + pl.lay.sort;
    std::lock_guard<std::mutex> lk(g_side_mu);
    SideStream *ss = side_stream_locked(st);
    const hipStream_t sb = ss ? ss->s : st;
    int rc = VQK_OK;
    // event i recorded on `from`, waited for by `to` (nothing without a side stream)
    auto link = [&](int i, hipStream_t from, hipStream_t to) {
        if (!ss) return VQK_OK;
        int r = hip_status(hipEventRecord(ss->e[i], from), "hipEventRecord");
        return r ? r : hip_status(hipStreamWaitEvent(to, ss->e[i], 0), "hipStreamWaitEvent");
    };
    // the shared expert is one expert over T rows: its gate / up launches
    // alone would fill few CUs, so they split K (fp32 partials that the down
    // launch adds in a fixed order as it stages its input)
    const int ks = p.shared ? seg_ksplit(m->sh_gate, T) : 1;
    if ((rc = link(0, st, sb))) return rc;
    if (p.shared) {
        SegCall cs{p.x, p.x_type, nullptr, nullptr, 1, sgg, VQK_F32, T, 0, ks};
        if ((rc = seg_run(m->sh_gate, cs, nullptr, sb))) return rc;
        cs.y = sgu;
        if ((rc = seg_run(m->sh_up, cs, nullptr, sb))) return rc;
    }
    hipLaunchKernelGGL(k_route_tokens, dim3(unsigned(T)), dim3(kWave), 0, st, p);
    if ((rc = hip_status(hipGetLastError(), "routing launch"))) return rc;
    // one sort for the three routed projections: its tile rows must suit
    // every kernel run over it (the 16-row kernels take the narrow tiles of
    // either size too)
    const int tok = seg_tile_rows(m->gate, N, p.E);
    if ((rc = seg_sort(reinterpret_cast<const uint32_t *>(p.ids), N, p.E, tok, sort, st))) return rc;
    if ((rc = link(1, st, sb))) return rc;
    SegCall c{p.x, p.x_type, nullptr, nullptr, k, g, VQK_F32, N, tok};
    if ((rc = seg_run(m->gate, c, sort, st))) return rc;
    c.y = u;
    if ((rc = seg_run(m->up, c, sort, sb))) return rc;
    if ((rc = link(2, sb, st))) return rc;
    SegCall d{nullptr, VQK_F32, g, u, 1, yd, VQK_F32, N, tok};
    if ((rc = seg_run(m->down, d, sort, st))) return rc;
    if (p.shared) {
        SegCall ds{nullptr, VQK_F32, sgg, sgu, 1, ysh, VQK_F32, T, 0, 0, ks};
        if ((rc = seg_run(m->sh_down, ds, nullptr, sb))) return rc;
    }
    if ((rc = link(3, sb, st))) return rc;
    hipLaunchKernelGGL(k_moe_combine, dim3(unsigned((p.H + 255) / 256), unsigned(T)), dim3(256), 0, st,
                       p, static_cast<const float *>(yd), static_cast<const float *>(ysh));
    return hip_status(hipGetLastError(), "combine launch");
}

// ------------------------------------------------ no-allocation scratch
// The workspace of vqk_moe_decode_layer_noalloc: a fixed device array, one
// copy per GPU, held until the process ends. Host code never uses the
// array's name as an address (in host code it names a host-side stand-in);
// the device address comes from hipGetSymbolAddress, once per device, with
// that device current.
static __device__ __align__(256) uint8_t scratch[VQK_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxScratchDevices];

// Device address of the current device's scratch array; `stream` (NULL or a
// stream of the current device) is checked against that device.
static int scratch_of_current_device(void *stream, void **out) {
    int dev = -1;
    int rc = hip_status(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxScratchDevices)
        return set_error(VQK_EDEVICE, "device %d outside the scratch table (%d devices)", dev,
                         kMaxScratchDevices);
    if (stream) {
        int sdev = -1;
        if ((rc = hip_status(hipStreamGetDevice(hipStream_t(stream), &sdev), "hipStreamGetDevice")))
            return rc;
        if (sdev != dev)
            return set_error(VQK_EINVAL, "stream belongs to device %d, the current device is %d",
                             sdev, dev);
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if ((rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress")))
            return rc;
        if (!p) return set_error(VQK_EDEVICE, "scratch array has no device address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return VQK_OK;
}

// Zeroes a workspace header (a fill kernel, not a memset: the call may be
// captured into a graph).
__global__ void __launch_bounds__(256) k_zero_header(u32x4 *h, int n) {
    const int i = int(blockIdx.x) * 256 + int(threadIdx.x);
    if (i < n) h[i] = u32x4{0, 0, 0, 0};
}

}  // namespace vqk

using namespace vqk;

extern "C" {

// ---- test hooks: exported, deliberately not in include/vqk.h -------------
// vqk__test_l1_spins: bound of the one-launch layer's waits for calls planned
// after it (n >= 0; returns the previous bound). vqk__test_l1_mode: 0 = one
// launch where it applies (default), 1 = never. vqk__test_moe_path: the path
// a call would take: 0 two fused kernels, 1 sliced-codebook GEMVs, 2 grouped
// GEMMs, 3 one launch.
int vqk__test_l1_spins(int n) { return g_l1_spins.exchange(n < 0 ? kL1Spins : n); }
int vqk__test_l1_mode(int m) { return g_l1_mode.exchange(m); }
int vqk__test_moe_path(const vqk_moe_desc *m, int64_t T, int32_t *path) {
    MoePlan pl;
    const int rc = moe_plan(m, T, &pl);
    if (rc) return rc;
    if (!path) return set_error(VQK_EINVAL, "path is NULL");
    *path = pl.l1 ? 3 : pl.path;
    return VQK_OK;
}

int vqk_moe_layer_status(const void *workspace, void *stream) {
    const void *ws = workspace;
    int rc;
    if (!ws) {
        void *s = nullptr;
        if ((rc = scratch_of_current_device(stream, &s))) return rc;
        ws = s;
    }
    if ((rc = hip_status(hipStreamSynchronize(hipStream_t(stream)), "hipStreamSynchronize"))) return rc;
    uint64_t err = 0;
    if ((rc = hip_status(hipMemcpy(&err, static_cast<const uint8_t *>(ws) + kHdrError, sizeof err,
                                   hipMemcpyDeviceToHost),
                         "reading the layer workspace's error word")))
        return rc;
    if (err)
        return set_error(VQK_EDEVICE,
                         "one-launch MoE layer: %s%s; those calls and every later one-launch call on "
                         "this workspace wrote NaN rows (vqk_moe_layer_reset clears it)",
                         (err & kL1ErrPoll) ? "a down workgroup's wait for the SwiGLU words ran out" : "",
                         (err & kL1ErrStamp) ? ((err & kL1ErrPoll) ? ", and a workgroup never started in time"
                                                                   : "a workgroup never started in time")
                                             : "");
    return VQK_OK;
}

int vqk_moe_layer_reset(void *workspace, void *stream) {
    void *ws = workspace;
    int rc;
    if (!ws && (rc = scratch_of_current_device(stream, &ws))) return rc;
    if (reinterpret_cast<uintptr_t>(ws) & 15)
        return set_error(VQK_EINVAL, "workspace must be 16-byte aligned");
    const int n = int(kHdrBytes / 16);
    hipLaunchKernelGGL(k_zero_header, dim3(unsigned((n + 255) / 256)), dim3(256), 0, hipStream_t(stream),
                       static_cast<u32x4 *>(ws), n);
    return hip_status(hipGetLastError(), "header reset launch");
}

int vqk_moe_decode_layer_workspace(const vqk_moe_desc *m, int64_t T, size_t *bytes) {
    if (!bytes) return set_error(VQK_EINVAL, "bytes is NULL");
    MoePlan pl;
    int rc = moe_plan(m, T, &pl);
    if (rc) return rc;
    *bytes = pl.lay.total;
    return VQK_OK;
}

int vqk_moe_decode_layer(const vqk_moe_desc *m, const void *x, int32_t x_type, int64_t T,
                         const float *logits, void *y, int32_t y_type, int32_t *topk_ids,
                         float *topk_w, void *workspace, size_t ws_bytes, void *stream) {
    MoePlan pl;
    int rc = moe_plan(m, T, &pl);
    if (rc) return rc;
    if (!act_size(x_type) || !out_size(y_type))
        return set_error(VQK_EINVAL, "x/y type must be VQK_F16, VQK_BF16 or VQK_F32");
    if (T == 0) return VQK_OK;              // an empty batch touches no pointer
    if (!x || !y || !logits) return set_error(VQK_EINVAL, "x, logits and y are required");
    if (!workspace || ws_bytes < pl.lay.total)
        return set_error(VQK_ENOSPACE, "workspace %zu B < %zu B", ws_bytes, pl.lay.total);
    MoeParams &p = pl.p;
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    p.ids = reinterpret_cast<int32_t *>(ws + pl.lay.ids);
    p.wts = reinterpret_cast<float *>(ws + pl.lay.wts);
    p.sg = reinterpret_cast<float *>(ws + pl.lay.sg);
    p.h = reinterpret_cast<uint16_t *>(ws + pl.lay.h);
    const bool split = pl.path == kMoeFused && pl.split;
    p.gbuf = split ? reinterpret_cast<float *>(ws + pl.lay.gs) : nullptr;
    p.ubuf = split ? reinterpret_cast<float *>(ws + pl.lay.us) : nullptr;
    p.ids_out = topk_ids;
    p.wts_out = topk_w;
    p.x = x;
    p.x_type = x_type;
    p.logits = logits;
    p.y = y;
    p.y_type = y_type;
    hipStream_t st = hipStream_t(stream);
    if (pl.path == kMoeGrouped) {
        if ((reinterpret_cast<uintptr_t>(x) & 15) != 0)
            return set_error(VQK_EINVAL, "batched layer: x must be 16-byte aligned");
        return launch_moe_grouped(m, pl, ws, st);
    }
    if (pl.path == kMoeBig) return launch_moe_big(m, pl, ws, st);
    if (pl.l1) {
        p.l1_epoch = reinterpret_cast<uint64_t *>(ws + kHdrEpoch);
        p.l1_err = reinterpret_cast<uint64_t *>(ws + kHdrError);
        p.l1_stamp = reinterpret_cast<uint64_t *>(ws + kHdrStamps);
        p.l1_hw = reinterpret_cast<uint64_t *>(ws + kHdrWords);
        return launch_moe_layer1(p, pl.g1.D, pl.g1.BITS, pl.g1.gpb, dim3(unsigned(pl.l1_nwg)), pl.smem_l1, st);
    }
    rc = split ? launch_moe_up_split(p, pl.g1.D, pl.g1.BITS, pl.g1.gpb, pl.wide1, pl.grid1, pl.smem1, st)
               : launch_moe_up(p, pl.g1.D, pl.g1.BITS, pl.g1.gpb, pl.grid1, pl.smem1, st);
    if (rc) return rc;
    if (pl.wide2) return launch_moe_down_wide(p, pl.g2.D, pl.g2.BITS, pl.g2.gpb, pl.grid2, pl.smem2, st);
    return launch_moe_down(p, pl.g2.D, pl.g2.BITS, pl.g2.gpb, pl.grid2, pl.smem2, st);
}

int vqk_moe_decode_layer_noalloc(const vqk_moe_desc *m, const void *x, int32_t x_type, int64_t T,
                                 const float *logits, void *y, int32_t y_type, int32_t *topk_ids,
                                 float *topk_w, void *stream) {
    MoePlan pl;
    int rc = moe_plan(m, T, &pl);
    if (rc) return rc;
    if (pl.lay.total > size_t(VQK_NOALLOC_SCRATCH_BYTES))
        return set_error(VQK_ENOSPACE,
                         "layer call needs %zu B of scratch; the no-allocation entry point has %zu B "
                         "(use vqk_moe_decode_layer with a workspace)",
                         pl.lay.total, size_t(VQK_NOALLOC_SCRATCH_BYTES));
    void *ws = nullptr;
    if ((rc = scratch_of_current_device(stream, &ws))) return rc;
    return vqk_moe_decode_layer(m, x, x_type, T, logits, y, y_type, topk_ids, topk_w, ws,
                                size_t(VQK_NOALLOC_SCRATCH_BYTES), stream);
}

}  // extern "C"
