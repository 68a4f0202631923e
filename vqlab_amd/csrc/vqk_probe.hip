// Measurement probe (test hook, not part of include/vqk.h): the random-gather
// rate an MI355X sustains from an L2-resident table -- the access the decode
// kernels make for codebook entries beyond their LDS part. Each lane reads
// `inflight` random 16-byte entries per round, then consumes them.
// bench.py --workload gather reports the rates at several waves per CU.
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

}  // extern "C"
