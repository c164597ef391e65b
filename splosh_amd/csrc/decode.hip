// decode.hip -- decode GEMV (one or two activation rows) over tiled q4 weights on every CU.
//
// The decode step reads a 50 MB weight once; the kernel has to spread that read evenly over all
// compute units and keep it in flight while the arithmetic of the groups already loaded runs.
//
// Work split. The output rows form blocks of 32 (one wave's worth: lane l owns row l >> 1 of the
// block and half h = l & 1 of every group), and the (block, group) pairs -- "units" -- are cut into
// gridDim.x equal contiguous ranges, one a workgroup (4 per CU). A range covers parts of two or
// three blocks; within a block segment the four waves take every fourth group. A block that one
// workgroup covers whole is written directly; a block shared by several writes fp32 partials to
// the caller's workspace, and the last of its workgroups to finish (an atomic counter per block,
// reset by that workgroup for the next call) sums them in workgroup order -- deterministic -- and
// applies the epilogue. No second kernel.
//
// Arithmetic. The workgroup first stages the activation rows in LDS in the form the math wants:
// for every code word (8 consecutive k), the four bf16 pairs (x_j, x_{j+4}), j = 0..3, and for
// every half group the sum of its 32 activations. A code word becomes four pairs
// (128 + q_j, 128 + q_{j+4}) with one v_and_or_b32 each, which meet the activation pairs in
// v_dot2_f32_bf16: with P = sum x (128 + q) and S = sum x over a half group,
// acc += s P + (b - 128 s) S (the per-group identity of engine_na.metal:8-20, split over the two
// halves). Eight VALU instructions per eight weights and row, plus two per half group.
//
// Loads in flight. A wave walks its groups in chunks of CH, with the next chunk's codes and
// sidecars loaded before the current chunk is computed.
#include "common.hpp"
#include "launch.hpp"

#include <cstdlib>

namespace splosh {

typedef __bf16 bf16x2_d __attribute__((ext_vector_type(2)));

struct DecodeArgs {
    const uint32_t *packed[2];
    const uint16_t *scales[2];
    const uint16_t *biases[2];
    int64_t n;
    int64_t groups;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
    float *partial;     // [gridDim.x][2][NW][R][32]
    int *counters;      // [n / 32], zero between calls
    int64_t units;      // (n / 32) * groups
    uint32_t code_bytes, sidecar_bytes;
};

#ifndef SPLOSH_DECODE_WGPC
#define SPLOSH_DECODE_WGPC 4
#endif
#ifndef SPLOSH_DECODE_CH
#define SPLOSH_DECODE_CH 4
#endif
constexpr int kDecodeWgPerCu = SPLOSH_DECODE_WGPC;
constexpr int kDecodeFinishMax = 64;  // contributors a block can have (checked on the host)

__device__ __forceinline__ float ddot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_d, a), __builtin_bit_cast(bf16x2_d, b), c, false);
}
__device__ __forceinline__ uint32_t dand_or(uint32_t a, uint32_t mask, uint32_t c) {
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(mask), "v"(c));
    return d;
}
// The value of lane l ^ 1 (DPP quad permutation [1, 0, 3, 2]).
__device__ __forceinline__ uint32_t dswap_pair(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}

// Workgroup i of P covers units [U i / P, U (i + 1) / P).
__device__ __forceinline__ int64_t range_start(int64_t units, int i, int P) { return units * i / P; }

template <int R, int NW, int CH>
__global__ void __launch_bounds__(256)
q4_decode_kernel(DecodeArgs args) {
    extern __shared__ __align__(16) uint32_t lds32[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane & 1, rl = lane >> 1;
    const int G = (int)args.groups;
    const uint32_t G32 = (uint32_t)G;
    const int K = G * kGroup;
    const int words = K / 8;  // code words (and activation pair quads) per row

    // LDS: xp[R][words] (16 bytes each: the four activation pairs of a code word), xs[R][K / 32]
    // (half-group sums), then the reduction area red[4][NW][R][32] and the fix-up flag.
    u32x4 *xp = (u32x4 *)lds32;
    float *xs = (float *)(lds32 + 4 * R * words);
    float *red = xs + R * (K / 32);
    int *flag = (int *)(red + 4 * NW * R * 32);

    const uint32_t kMask = 0x000F000Fu;
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
    rsrc_t q_rsrc[NW];
    const uint16_t *side[NW];  // lane h = 0 fetches the scale, h = 1 the bias; they swap at use
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        q_rsrc[w] = make_rsrc(args.packed[w], args.code_bytes);
        side[w] = h == 0 ? args.scales[w] : args.biases[w];
    }

    const int P = gridDim.x;
    const rsrc_t p_rsrc = make_rsrc(args.partial, (uint32_t)P * 2u * (uint32_t)(NW * R * 32) * 4u);
    const int64_t u_begin = range_start(args.units, blockIdx.x, P), u_stop = range_start(args.units, blockIdx.x + 1, P);
    // Segment state: block blk, groups [ga, gb) of which this wave takes ga + wave + 4 i, i < ng.
    int blk = 0, ga = 0, gb = 0, ng = 0;
    uint32_t rec0 = 0;
    auto begin_segment = [&](int64_t u) {
        blk = (int)(u / G);
        ga = (int)(u % G);
        gb = (int)((int64_t)ga + (u_stop - u) < G ? ga + (u_stop - u) : G);
        ng = (gb - ga - wave + 3) / 4;
        const int64_t rr = (int64_t)blk * 32 + rl;
        const uint32_t row = (uint32_t)(rr < args.n ? rr : args.n - 1);
        rec0 = (row >> 7) * G32 * 128u + (row & 127u);  // record of group 0
    };
    u32x4 cq[2][CH][NW];
    uint32_t cs[2][CH][NW];
    auto load_chunk = [&](int buf, int c0) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            int i = c0 + k;
            i = i < ng ? i : (ng > 0 ? ng - 1 : 0);
            const uint32_t g = (uint32_t)(ga + wave + 4 * i < gb ? ga + wave + 4 * i : gb - 1);
            const uint32_t rec = rec0 + g * 128u;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                cq[buf][k][w] = buffer_load16_cp<2>(q_rsrc[w], rec * 32u + 16u * h, 0);
                cs[buf][k][w] = side[w][rec];
            }
        }
    };

    // The first segment's first loads go out before the activations are staged.
    if (u_begin < u_stop) {
        begin_segment(u_begin);
        load_chunk(0, 0);
    }
    // ---- stage the activations: thread j of the workgroup takes half groups j, j + 256, ... ----
    for (int e = tid; e < R * (K / 32); e += 256) {
        const int m = e / (K / 32), hg = e % (K / 32);
        const int mr = m < args.rows ? m : 0;
        const u32x4 *src = (const u32x4 *)(args.a + (int64_t)mr * args.lda + hg * 32);
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 v = src[k];  // elements 8k .. 8k + 7 of the half group
            u32x4 pq;
            pq.x = perm_bytes(v.z, v.x, 0x05040100u);  // (x0, x4)
            pq.y = perm_bytes(v.z, v.x, 0x07060302u);  // (x1, x5)
            pq.z = perm_bytes(v.w, v.y, 0x05040100u);  // (x2, x6)
            pq.w = perm_bytes(v.w, v.y, 0x07060302u);  // (x3, x7)
            xp[m * words + hg * 4 + k] = pq;
            s0 = ddot2(v.x, 0x3F803F80u, s0);
            s1 = ddot2(v.y, 0x3F803F80u, s1);
            s0 = ddot2(v.z, 0x3F803F80u, s0);
            s1 = ddot2(v.w, 0x3F803F80u, s1);
        }
        xs[m * (K / 32) + hg] = s0 + s1;
    }
    __syncthreads();


    int slot = 0;
    for (int64_t u = u_begin; u < u_stop;) {
        const int64_t u_seg = u;
        const bool whole = ga == 0 && gb == G;
        const int seg_blk = blk;
        slot = u_seg == u_begin ? 0 : 1;  // the first segment of the range uses slot 0
        u += gb - ga;
        float acc[NW][R];
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int m = 0; m < R; ++m) acc[w][m] = 0.0f;
        auto compute_chunk = [&](int buf, int c0) {
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int i = c0 + k;
                const bool live = i < ng;
                const int g = ga + wave + 4 * (live ? i : 0);
                const int hg = 2 * g + h;  // half group of this lane
                u32x4 xv[R][4];
                float sx[R];
#pragma unroll
                for (int m = 0; m < R; ++m) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) xv[m][j] = xp[m * words + hg * 4 + j];
                    sx[m] = xs[m * (K / 32) + hg];
                }
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    float pq[R], pr[R];
#pragma unroll
                    for (int m = 0; m < R; ++m) pq[m] = pr[m] = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t word = cq[buf][k][w][j];
                        const uint32_t b0 = dand_or(word, kMask, magic);
                        const uint32_t b1 = dand_or(word >> 4, kMask, magic);
                        const uint32_t b2 = dand_or(word >> 8, kMask, magic);
                        const uint32_t b3 = dand_or(word >> 12, kMask, magic);
#pragma unroll
                        for (int m = 0; m < R; ++m) {
                            pq[m] = ddot2(b0, xv[m][j][0], pq[m]);
                            pr[m] = ddot2(b1, xv[m][j][1], pr[m]);
                            pq[m] = ddot2(b2, xv[m][j][2], pq[m]);
                            pr[m] = ddot2(b3, xv[m][j][3], pr[m]);
                        }
                    }
                    const uint32_t mine = cs[buf][k][w];
                    const uint32_t other = dswap_pair(mine);
                    const float s = live ? bf16_bits_to_f32(h == 0 ? mine : other) : 0.0f;
                    const float b = bf16_bits_to_f32(h == 0 ? other : mine);
                    const float bp = live ? __builtin_fmaf(-128.0f, s, b) : 0.0f;
#pragma unroll
                    for (int m = 0; m < R; ++m)
                        acc[w][m] = __builtin_fmaf(s, pq[m] + pr[m], __builtin_fmaf(bp, sx[m], acc[w][m]));
                }
            }
        };
        // Chunks of CH groups, the next one's loads issued before the current one's arithmetic.
        for (int c0 = 0; c0 < ng; c0 += 2 * CH) {
            load_chunk(1, c0 + CH);
            compute_chunk(0, c0);
            load_chunk(0, c0 + 2 * CH);
            compute_chunk(1, c0 + CH);
        }

        // The next segment's first loads go out before this one's reduction and fix-up.
        if (u < u_stop) {
            begin_segment(u);
            load_chunk(0, 0);
        }
        const int blk_next = blk;
        blk = seg_blk;

        // ---- reduce: the two half lanes of a row, then the four waves in LDS ----
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int m = 0; m < R; ++m)
                acc[w][m] += __builtin_bit_cast(float, dswap_pair(__builtin_bit_cast(uint32_t, acc[w][m])));
        if (h == 0) {
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int m = 0; m < R; ++m) red[((wave * NW + w) * R + m) * 32 + rl] = acc[w][m];
        }
        __syncthreads();
        constexpr int kOut = NW * R * 32;  // values of a block segment
        float v = 0.0f;
        if (tid < kOut) {
#pragma unroll
            for (int wv = 0; wv < 4; ++wv) v += red[wv * kOut + tid];
        }
        // Value tid = (w R + m) 32 + row of the block.
        auto epilogue = [&](float v0, float v1, int m, int rrow) {
            const int64_t nn = (int64_t)blk * 32 + rrow;
            if (m >= args.rows || nn >= args.n) return;
            float value = v0;
            if constexpr (NW == 2) value = silu(v0) * v1;
            const int64_t index = m * args.ldc + nn;
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) value += ((const float *)args.residual)[index];
                ((float *)args.out)[index] = value;
            } else {
                if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                ((uint16_t *)args.out)[index] = f32_to_bf16(value);
            }
        };
        if (whole) {
            // red is reused: park the sums, then the first R * 32 threads apply the epilogue.
            __syncthreads();
            if (tid < kOut) red[tid] = v;
            __syncthreads();
            if (tid < R * 32) {
                const int m = tid / 32, rrow = tid % 32;
                epilogue(red[m * 32 + rrow], NW == 2 ? red[(R + m) * 32 + rrow] : 0.0f, m, rrow);
            }
        } else {
            // A shared block: this workgroup's partial, then the fix-up by the last contributor.
            // The partials cross XCDs, whose L2 caches are not coherent with each other: they are
            // written and read with device-scope cache policy (sc0 sc1: through to memory), and the
            // counter is a system-scope atomic (also sc0 sc1), so no L2 write-back or invalidation is needed.
            constexpr int kDevice = 1 | 16;  // gfx94x cache policy sc0 | sc1
            const uint32_t pbase = (uint32_t)(((int64_t)blockIdx.x * 2 + slot) * kOut) * 4u;
            if (tid < kOut) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), p_rsrc, pbase + tid * 4u, 0, kDevice);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial has reached memory
            __syncthreads();
            if (tid == 0) {
                // Contributors: the workgroups whose ranges meet [blk G, (blk + 1) G).
                const int64_t lo = (int64_t)blk * G, hi = lo + G;
                const int i_lo = (int)(((lo + 1) * P - 1) / args.units), i_hi = (int)((hi * P - 1) / args.units);
                int count = 0;
                for (int i = i_lo; i <= i_hi; ++i)
                    if (range_start(args.units, i, P) != range_start(args.units, i + 1, P)) ++count;
                const int old = __hip_atomic_fetch_add(args.counters + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                *flag = old == count - 1 ? 1 : 0;
            }
            __syncthreads();
            if (*flag) {
                const int64_t lo = (int64_t)blk * G, hi = lo + G;
                const int i_lo = (int)(((lo + 1) * P - 1) / args.units), i_hi = (int)((hi * P - 1) / args.units);
                float sum = 0.0f;
                if (tid < kOut) {
                    for (int i = i_lo; i <= i_hi; ++i) {
                        const int64_t s = range_start(args.units, i, P);
                        if (s == range_start(args.units, i + 1, P)) continue;
                        const int sl = s < lo ? 1 : 0;
                        const uint32_t off = (uint32_t)(((int64_t)i * 2 + sl) * kOut + tid) * 4u;
                        sum += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(p_rsrc, off, 0, kDevice));
                    }
                }
                __syncthreads();
                if (tid < kOut) red[tid] = sum;
                __syncthreads();
                if (tid < R * 32) {
                    const int m = tid / 32, rrow = tid % 32;
                    epilogue(red[m * 32 + rrow], NW == 2 ? red[(R + m) * 32 + rrow] : 0.0f, m, rrow);
                }
                if (tid == 0) __hip_atomic_store(args.counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
        __syncthreads();  // red is reused by the next segment
        blk = blk_next;
    }
}

// Shapes the kernel takes: tiled weights, 32-row blocks, K staged whole in LDS.
bool decode_fits(int64_t rows, int64_t columns, int64_t inner, int order) {
    if (order != SPLOSH_Q4_TILED128 || rows < 1 || rows > 2 || inner % kGroup != 0 || columns % 128 != 0) return false;
    const int64_t lds = 2 * inner * 2 + 2 * (inner / 32) * 4 + 4 * 2 * 2 * 32 * 4 + 16;
    return lds <= 150 * 1024 && columns * (inner / kGroup) * 32 < ((int64_t)1 << 32) - 256;
}

static int decode_grid() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus * kDecodeWgPerCu;
}

// Workspace: partials [grid][2][2][2][32] floats, then a counter per 32-row block (zero-filled by
// the caller once; every call leaves them zero).
static size_t decode_partial_bytes(int grid) { return (size_t)grid * 2 * 2 * 2 * 32 * sizeof(float); }

size_t decode_workspace_bytes(int64_t columns) {
    return decode_partial_bytes(decode_grid()) + (size_t)(columns / 32) * sizeof(int);
}

bool decode_plan_ok(int64_t columns, int64_t groups, size_t workspace_bytes) {
    const int grid = decode_grid();
    const int64_t units = columns / 32 * groups;
    // Contributors per block: about grid * groups / units + 2.
    return workspace_bytes >= decode_workspace_bytes(columns) && units >= grid &&
           (int64_t)grid * groups / units + 2 <= kDecodeFinishMax;
}

template <int R, int NW>
static hipError_t launch_decode_v(const DecodeArgs &args, int grid, hipStream_t stream) {
    const int K = (int)(args.groups * kGroup);
    const size_t lds = (size_t)R * K * 2 + (size_t)R * (K / 32) * 4 + 4 * NW * R * 32 * 4 + 16;
    auto kernel = q4_decode_kernel<R, NW, SPLOSH_DECODE_CH>;
    static bool once = [&] {
        (void)hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        return true;
    }();
    (void)once;
    hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), lds, stream, args);
    return hipGetLastError();
}

hipError_t launch_q4_decode(const splosh_q4_weight &w, const splosh_q4_weight *up, const uint16_t *a, int64_t lda,
                            void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows, void *workspace,
                            hipStream_t stream) {
    DecodeArgs args;
    args.packed[0] = w.packed;
    args.scales[0] = w.scales;
    args.biases[0] = w.biases;
    args.packed[1] = up ? up->packed : w.packed;
    args.scales[1] = up ? up->scales : w.scales;
    args.biases[1] = up ? up->biases : w.biases;
    args.n = w.rows;
    args.groups = w.inner / kGroup;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = rows;
    args.out_dtype = out_dtype;
    const int grid = decode_grid();
    args.partial = (float *)workspace;
    args.counters = (int *)((char *)workspace + decode_partial_bytes(grid));
    args.units = w.rows / 32 * args.groups;
    args.code_bytes = (uint32_t)(w.rows * args.groups * 32);
    args.sidecar_bytes = (uint32_t)(w.rows * args.groups * 2);
    if (rows == 1)
        return up ? launch_decode_v<1, 2>(args, grid, stream) : launch_decode_v<1, 1>(args, grid, stream);
    return up ? launch_decode_v<2, 2>(args, grid, stream) : launch_decode_v<2, 1>(args, grid, stream);
}

}  // namespace splosh
