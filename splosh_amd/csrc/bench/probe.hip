// probe.hip -- measurement probes, not part of the path and not in libsplosh_q4.so: built into
// libsplosh_probe.so, which only bench.py loads. They measure the HBM read rate a single launch of
// a given size reaches on this part (bench.py --workload stream50 reads as many bytes as the
// config-0 decode weight), so that the decode kernel can be judged against it.
#include "../common.hpp"

namespace splosh {

// Shape 0, "slices": workgroup g reads the contiguous slice [g, g + 1) / grid of the buffer in
// 16-byte pieces, eight loads in flight a thread (non-temporal), and folds them into one word, so
// the loads cannot be dropped; one word a wave is written.
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

// Shape 1, "persistent": few resident workgroups of 1024 threads (one or two a CU) walk the buffer
// in rounds of 16 KiB a workgroup, the rounds of all workgroups interleaved (round r of workgroup g
// is piece block r * grid + g), with DEPTH loads in flight a thread through buffer loads that
// return zero past the end (so every round is branch-free). One word a wave is written.
template <int DEPTH>
__global__ void __launch_bounds__(1024) persistent_read_kernel(const void *src, uint32_t bytes, uint32_t *sink) {
    const rsrc_t rs = make_rsrc(src, bytes);
    const uint32_t block = 1024u * 16u;  // bytes a workgroup reads a round
    const uint32_t stride = gridDim.x * block;
    uint32_t off = blockIdx.x * block + threadIdx.x * 16u;
    uint32_t acc = 0;
    const uint32_t rounds = (bytes + stride - 1) / stride;
    uint32_t r = 0;
    for (; r + DEPTH <= rounds; r += DEPTH) {
        u32x4 x[DEPTH];
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) x[j] = buffer_load16_cp<2>(rs, off + (uint32_t)j * stride, 0u);
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
        off += DEPTH * stride;
    }
    for (; r < rounds; ++r, off += stride) {
        const u32x4 a = buffer_load16_cp<2>(rs, off, 0u);
        acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
    }
    for (int o = 32; o >= 1; o >>= 1) acc ^= __shfl_xor(acc, o, 64);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 16 + (threadIdx.x >> 6)] = acc;
}

}  // namespace splosh

// shape 0: slices (grid workgroups of 256); shape 1: persistent (grid workgroups of 1024, 8 loads
// in flight a thread); shape 2: persistent with 16 loads in flight. `sink` holds 16 words a
// workgroup.
extern "C" int splosh_probe_stream_read(const void *src, int64_t bytes, uint32_t *sink, int grid, int shape,
                                        hipStream_t stream) {
    if (!src || !sink || bytes < 16 || grid <= 0) return 12;
    if (shape == 0) {
        hipLaunchKernelGGL(splosh::stream_read_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                           (const splosh::u32x4 *)src, bytes / 16, sink);
    } else {
        if (bytes >= ((int64_t)1 << 32)) return 13;
        if (shape == 1)
            hipLaunchKernelGGL(splosh::persistent_read_kernel<8>, dim3((unsigned)grid), dim3(1024), 0, stream, src,
                               (uint32_t)bytes, sink);
        else
            hipLaunchKernelGGL(splosh::persistent_read_kernel<16>, dim3((unsigned)grid), dim3(1024), 0, stream, src,
                               (uint32_t)bytes, sink);
    }
    return hipGetLastError() == hipSuccess ? 0 : 15;
}
