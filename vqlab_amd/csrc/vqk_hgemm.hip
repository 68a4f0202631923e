// Launchers of the dense prefill GEMM (kernels in vqk_hgemm.h) and the
// conversion of fp32 activations into split bf16 operands.
#include "vqk_hgemm.h"

namespace vqk {

// Tile shapes (measured on MI355X at the dense prefill shapes, M = 2048):
//   0  256 x 256, ping-pong 4 x 2 waves (64 x 128 each), BK 32, 5 stages:
//      the most MFMA work per LDS byte; 5120 -> 17408 is 544 tiles = two
//      rounds of 256 CUs + 32 tiles, whose K is split 8 ways (below)
//   1  256 x 192, ping-pong 4 x 2 waves (64 x 96 each), BK 32, 4 stages
//      5120 -> 17408 whole: 728 tiles = 2.84 rounds, 386 us
//   2  256 x 160, ping-pong 8 x 1 waves (32 x 160 each), BK 64, 3 stages
//      17408 -> 5120: 256 tiles = one round, 325 us
//   3  128 x 128, 4 waves (64 x 64 each), BK 64, 3 stages: small outputs
// The plan takes the shape (and split) whose estimated time -- rounds x tile
// area / relative rate -- is least: a tile count just past a multiple of
// the CU count idles most of the GPU for a whole round (256 x 256 tiles:
// 160 for a 2048 x 5120 output). With R whole rounds and r < C/2 tiles left
// over (C CUs), the r tiles run as r x s K slices (s <= C / r, at most 8, at
// least 4 k steps each) into fp32 partials that k_gemm_reduce adds in a
// fixed order.
struct TileShape { int bm, bn, bk; float rate; bool pp; };
constexpr TileShape kShapes[] = {
    {256, 256, 32, 1.f, true}, {256, 192, 32, 0.8f, true}, {256, 160, 64, 0.87f, true},
    {128, 128, 64, 0.5f, false}};
constexpr float kSplitCost = 1.3f;      // a split slice's time relative to its share of a tile

static int cu_count() {
    int cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;
    return cus;
}

GemmPlan plan_gemm(int64_t M, int64_t Nc, int64_t K, size_t part_room) {
    const int cus = cu_count();
    GemmPlan best{};
    double best_cost = -1.;
    for (int i = 0; i < int(sizeof kShapes / sizeof kShapes[0]); ++i) {
        const TileShape &sh = kShapes[i];
        const int64_t T = ((M + sh.bm - 1) / sh.bm) * ((Nc + sh.bn - 1) / sh.bn);
        const double area = double(sh.bm) * sh.bn / sh.rate;
        GemmPlan pl{i, 0, 0, 0};
        double cost = double((T + cus - 1) / cus) * area;
        const int64_t R = T / cus, r = T % cus, kt = K / sh.bk;
        if (sh.pp && R >= 1 && r > 0 && 2 * r <= cus) {
            int64_t sp = cus / r;
            sp = sp > 8 ? 8 : sp;
            while (sp >= 2 && (kt / sp < 4 || (sp - 1) * ((kt + sp - 1) / sp) >= kt)) --sp;
            const size_t pb = size_t(r) * size_t(sp) * size_t(sh.bm) * size_t(sh.bn) * 4;
            const double c2 = double(R) * area + area / double(sp) * kSplitCost;
            if (sp >= 2 && pb <= part_room && c2 < cost) {
                cost = c2;
                pl.full = int32_t(R * cus);
                pl.splits = int32_t(sp);
                pl.part_bytes = pb;
            }
        }
        if (best_cost < 0. || cost < best_cost) { best = pl; best_cost = cost; }
    }
    return best;
}

template <int OP, int BM, int BN, int WGM, int WGN, int BK, int NST, bool PP>
static int go_gemm(HgemmParams p, hipStream_t st) {
    p.tiles_m = int32_t((p.M + BM - 1) / BM);
    p.tiles_n = int32_t((p.Nc + BN - 1) / BN);
    const int64_t T = int64_t(p.tiles_m) * p.tiles_n;
    const int64_t units = p.splits ? p.full + (T - p.full) * p.splits : T;
    if (units > INT32_MAX) return set_error(VQK_ENOTIMPL, "GEMM grid too large");
    const size_t lds = size_t(NST) * (BM + BN) * BK * 2;
    int rc;
    if constexpr (PP) {
        rc = launch_with_lds<k_pgemm<OP, BM, BN, WGM, WGN, BK, NST>>(dim3(unsigned(units)), dim3(512),
                                                                     lds, st, p);
        if (rc || !p.splits || T == p.full) return rc;
        hipLaunchKernelGGL((k_gemm_reduce<BM, BN, WGM, WGN>), dim3(BM * BN / 1024, unsigned(T - p.full)),
                           dim3(256), 0, st, p);
        return hip_status(hipGetLastError(), "split-K reduce launch");
    } else {
        p.splits = 0;
        return launch_with_lds<k_hgemm<OP, BM, BN, WGM, WGN, BK, NST>>(dim3(unsigned(T)),
                                                                       dim3(64 * WGM * WGN), lds, st, p);
    }
}

template <int OP>
static int gemm_op(const HgemmParams &p, int shape, hipStream_t st) {
    switch (shape) {
        case 0: return go_gemm<OP, 256, 256, 4, 2, 32, 5, true>(p, st);
        case 1: return go_gemm<OP, 256, 192, 4, 2, 32, 4, true>(p, st);
        case 2: return go_gemm<OP, 256, 160, 8, 1, 64, 3, true>(p, st);
        default: return go_gemm<OP, 128, 128, 2, 2, 64, 3, false>(p, st);
    }
}

// y[:, c0 : c0 + Nc] = A . B^T; A [M, K], B [Nc, K] in fp16 (op kOpF16) or
// bf16 (kOpBF16), K % 64 == 0, both 16-byte aligned. `plan` comes from
// plan_gemm(M, Nc, K, room); a split plan needs plan.part_bytes of fp32
// partials at `part` (256-byte aligned).
int launch_hgemm(int op, const GemmPlan &plan, const uint16_t *A, const uint16_t *B, void *y,
                 int32_t y_type, int64_t ldy, int64_t ycol0, int64_t M, int64_t Nc, int64_t K,
                 float *part, hipStream_t st) {
    if (M <= 0 || Nc <= 0) return VQK_OK;
    if (K % 64 || M > INT32_MAX || Nc > INT32_MAX || K > INT32_MAX)
        return set_error(VQK_ENOTIMPL, "GEMM shape M %lld N %lld K %lld", (long long)M, (long long)Nc,
                         (long long)K);
    if (plan.splits && !part) return set_error(VQK_EINVAL, "split GEMM without its partials");
    HgemmParams p;
    p.A = A;
    p.B = B;
    p.y = y;
    p.y_type = y_type;
    p.ldy = ldy;
    p.ycol0 = ycol0;
    p.M = int32_t(M);
    p.Nc = int32_t(Nc);
    p.K = int32_t(K);
    p.full = plan.full;
    p.splits = plan.splits;
    p.part = part;
    return op == kOpBF16 ? gemm_op<kOpBF16>(p, plan.shape, st) : gemm_op<kOpF16>(p, plan.shape, st);
}

// Activation rows for the GEMM, ld >= IN elements per part, zero past IN:
//   split == 0: fp16 / bf16 x copied bit for bit (x misaligned, or IN not a
//               multiple of the GEMM's k step);
//   split == 1: fp32 x as bf16 rows [x_hi | x_hi | x_lo], x_hi = bf16(x),
//               x_lo = bf16(x - x_hi). Against weight rows [W_hi | W_lo | W_hi]
//               (the fp16 weight split the same way, exactly) one bf16 GEMM
//               over 3 * ld sums x_hi W_hi + x_hi W_lo + x_lo W_hi: the fp16
//               weight in full and x to 16 significant bits, every product
//               exact and summed in fp32.
// One thread per 8 output columns of a row; elements are read one by one, so
// x needs no alignment beyond its element size.
__global__ void k_x_stage(const void *x, int32_t x_type, int64_t N, int64_t IN, int64_t ld, int split,
                          uint16_t *out) {
    const int64_t ld8 = ld / 8;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= N * ld8) return;
    const int64_t row = i / ld8, c0 = (i % ld8) * 8;
    uint16_t hi[8], lo[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int64_t c = c0 + u;
        hi[u] = lo[u] = 0;
        if (c >= IN) continue;
        if (!split) {
            hi[u] = static_cast<const uint16_t *>(x)[row * IN + c];
            continue;
        }
        const float v = static_cast<const float *>(x)[row * IN + c];
        hi[u] = f32_to_bf16(v);
        const float h = bf16_to_f32(hi[u]);
        if ((__float_as_uint(h) & 0x7f800000u) != 0x7f800000u) lo[u] = f32_to_bf16(v - h);
    }
    u32x4 H, Lo;
    H.x = hi[0] | (uint32_t(hi[1]) << 16); H.y = hi[2] | (uint32_t(hi[3]) << 16);
    H.z = hi[4] | (uint32_t(hi[5]) << 16); H.w = hi[6] | (uint32_t(hi[7]) << 16);
    Lo.x = lo[0] | (uint32_t(lo[1]) << 16); Lo.y = lo[2] | (uint32_t(lo[3]) << 16);
    Lo.z = lo[4] | (uint32_t(lo[5]) << 16); Lo.w = lo[6] | (uint32_t(lo[7]) << 16);
    u32x4 *dst = reinterpret_cast<u32x4 *>(out + row * (split ? 3 : 1) * ld + c0);
    dst[0] = H;
    if (split) {
        dst[ld8] = H;
        dst[2 * ld8] = Lo;
    }
}

int launch_x_stage(const void *x, int32_t x_type, int64_t N, int64_t IN, int64_t ld, uint16_t *out,
                   hipStream_t st) {
    const int64_t n8 = N * (ld / 8);
    if (n8 == 0) return VQK_OK;
    hipLaunchKernelGGL(k_x_stage, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0, st, x, x_type, N, IN,
                       ld, x_type == VQK_F32 ? 1 : 0, out);
    return hip_status(hipGetLastError(), "x staging launch");
}

}  // namespace vqk
