// Measurement probe and test hooks (not part of include/vqk.h).
// vqk__probe_gather: the random-gather rate an MI355X sustains from an
// L2-resident table -- the access the decode kernels make for codebook
// entries beyond their LDS part. Each lane reads `inflight` random 16-byte
// entries per round, then consumes them. bench.py --workload gather reports
// the rates at several waves per CU.
// vqk__probe_stream: the fastest one-launch streaming read of a buffer --
// 16-byte loads over a grid-stride loop, one word written per workgroup --
// the floor of a decode kernel that must read the same bytes in one launch.
// bench.py --workload stream times it on config 1's weight bytes.
// vqk__test_f32_to_bf16: the library's fp32 -> bf16 conversion (every bf16
// output and weight goes through it), element by element.
#include "vqk_common.h"

namespace vqk {

template <int U>
__global__ void __launch_bounds__(256) k_probe_gather(const u32x4 *table, uint32_t nent, int rounds,
                                                      uint32_t *sink) {
    uint32_t s = (blockIdx.x * 256u + threadIdx.x) * 2654435761u + 12345u;
    uint32_t acc = 0;
    for (int it = 0; it < rounds; ++it) {
        uint32_t idx[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            s = s * 1664525u + 1013904223u;
            idx[u] = (s >> 8) % nent;
        }
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = table[idx[u]];
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].w;
    }
    sink[blockIdx.x * 256u + threadIdx.x] = acc;
}

__global__ void __launch_bounds__(256) k_probe_stream(const u32x4 *p, int64_t n16, uint32_t *sink) {
    __shared__ uint32_t part[4];
    uint32_t acc = 0;
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    for (int o = 32; o >= 1; o >>= 1) acc ^= uint32_t(__shfl_xor(int(acc), o));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

__global__ void __launch_bounds__(256) k_test_f32_to_bf16(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        y[i] = f32_to_bf16(x[i]);
}

}  // namespace vqk

using namespace vqk;

extern "C" {

// workgroups of 256 threads (4 waves): `wgs` of them; sink holds wgs * 256
// uint32; table_bytes a multiple of 16 and >= 16
int vqk__probe_gather(const void *table, uint32_t table_bytes, int wgs, int inflight, int rounds,
                      uint32_t *sink, void *stream) {
    if (!table || !sink || table_bytes < 16 || (table_bytes & 15) || wgs < 1 || rounds < 1)
        return set_error(VQK_EINVAL, "gather probe: bad arguments");
    const uint32_t nent = table_bytes / 16;
    const u32x4 *t = static_cast<const u32x4 *>(table);
    hipStream_t st = hipStream_t(stream);
    const dim3 grid{unsigned(wgs), 1u, 1u}, block{256u, 1u, 1u};
    switch (inflight) {
        case 1: hipLaunchKernelGGL(k_probe_gather<1>, grid, block, 0, st, t, nent, rounds, sink); break;
        case 4: hipLaunchKernelGGL(k_probe_gather<4>, grid, block, 0, st, t, nent, rounds, sink); break;
        case 8: hipLaunchKernelGGL(k_probe_gather<8>, grid, block, 0, st, t, nent, rounds, sink); break;
        default: return set_error(VQK_EINVAL, "gather probe: inflight must be 1, 4 or 8");
    }
    return hip_status(hipGetLastError(), "gather probe launch");
}

// workgroups of 256 threads: `wgs` of them; sink holds wgs uint32; bytes a
// multiple of 16
int vqk__probe_stream(const void *buf, int64_t bytes, int wgs, uint32_t *sink, void *stream) {
    if (!buf || !sink || bytes < 16 || (bytes & 15) || wgs < 1 || wgs > 65535)
        return set_error(VQK_EINVAL, "stream probe: bad arguments");
    hipLaunchKernelGGL(k_probe_stream, dim3(unsigned(wgs)), dim3(256u), 0, hipStream_t(stream),
                       static_cast<const u32x4 *>(buf), bytes / 16, sink);
    return hip_status(hipGetLastError(), "stream probe launch");
}

}  // extern "C"

extern "C" int vqk__test_f32_to_bf16(const float *x, uint16_t *y, int64_t n, void *stream) {
    if (n < 0 || ((!x || !y) && n > 0)) return vqk::set_error(VQK_EINVAL, "bad arguments");
    if (n == 0) return VQK_OK;
    const int64_t blocks = (n + 255) / 256;
    const dim3 grid{unsigned(blocks < 4096 ? blocks : 4096), 1u, 1u}, block{256u, 1u, 1u};
    hipLaunchKernelGGL(vqk::k_test_f32_to_bf16, grid, block, 0, hipStream_t(stream), x, y, n);
    return vqk::hip_status(hipGetLastError(), "bf16 conversion launch");
}
