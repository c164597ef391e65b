// probe.hip -- a measurement probe, not part of the path: a plain streaming read of a buffer, the
// practical HBM ceiling a single launch of a given size reaches on this part (bench.py --workload
// stream50 reads as many bytes as the config-0 decode weight). Exported for the benchmark only;
// the C ABI header does not declare it.
#include "common.hpp"

namespace splosh {

// Workgroup g reads the contiguous slice [g, g + 1) / grid of the buffer in 16-byte pieces, eight
// loads in flight a thread (non-temporal), and folds them into one word, so the loads cannot be
// dropped; one word a wave is written.
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4 *__restrict__ src, int64_t pieces,
                                                          uint32_t *__restrict__ sink) {
    const int64_t per = (pieces + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per, hi = lo + per < pieces ? lo + per : pieces;
    uint32_t acc = 0;
    int64_t i = lo + threadIdx.x;
    for (; i + 7 * 256 < hi; i += 8 * 256) {
        u32x4 x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = __builtin_nontemporal_load(src + i + j * 256);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
    }
    for (; i < hi; i += 256) {
        const u32x4 a = __builtin_nontemporal_load(src + i);
        acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
    }
    for (int o = 32; o >= 1; o >>= 1) acc ^= __shfl_xor(acc, o, 64);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

}  // namespace splosh

extern "C" int splosh_probe_stream_read(const void *src, int64_t bytes, uint32_t *sink, int grid, hipStream_t stream) {
    if (!src || !sink || bytes < 16 || grid <= 0) return 12;
    hipLaunchKernelGGL(splosh::stream_read_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                       (const splosh::u32x4 *)src, bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 15;
}
