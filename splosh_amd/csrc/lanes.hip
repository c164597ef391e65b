// lanes.hip -- decode GEMV (one or two activation rows) over q4 weights, VALU only.
//
// The decode step reads a 50 MB weight once, so the kernel's job is to keep enough of it in
// flight, to read it in whole cache lines, and to spend few VALU instructions per weight.
//
// Mapping. A workgroup owns one 128-row tile of outputs; its waves split the K groups. In a wave,
// lane l works on half h = l & 1 of every group (32 of its 64 k) for the four rows
// r = (l >> 1) + 32 t, t = 0..3. In the 128-row tiled layout (Model/Retile.swift:135-153) a
// group's records of the tile are one contiguous 4 KB slab, and the lanes read it in order (lane l:
// bytes 16 l .. 16 l + 15 of each kilobyte): the four load instructions of a group move the whole
// slab, and no two workgroups share a DRAM page of it.
//
// Arithmetic. A code word becomes four bf16 pairs (128 + q_j, 128 + q_{j+4}) with one
// v_and_or_b32 each (after a shift), and a pair meets the activation pair (x_j, x_{j+4}) in one
// v_dot2_f32_bf16 -- eleven VALU instructions per eight weights and row. Per half group,
// P = sum x (128 + q) and S = sum x, and acc += s P + (b - 128 s) S: the per-group identity of
// engine_na.metal:8-20, split over the two halves (it is linear in P and S). The two lanes of a
// row are summed with one DPP swap at the end, and the waves' partials in LDS.
//
// Activations. A lane loads its half group of activations itself (four 16-byte loads that all
// lanes of the same half share, so they are served from L1/L2), forms the pairs (x_j, x_{j+4})
// with v_perm_b32 and the half-group sum with v_dot2 against ones. Staging them in LDS instead
// costs a barrier that every wave waits at, which was measured slower.
//
// Loads in flight. Waves own GPW <= 8 groups (a compile-time bucket, so the loop is unrolled and
// every register index static) and issue all of their loads at once, right after the activation
// loads: the whole weight is requested within the first microsecond. Groups past the end are
// loaded clamped and weighted zero. (A rolling reload window was measured far slower.)
#include "common.hpp"
#include "launch.hpp"

#include <cstdlib>

namespace splosh {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct LaneArgs {
    const uint32_t *packed[2];
    const uint16_t *scales[2];
    const uint16_t *biases[2];
    int64_t stride_words;
    int64_t n;
    int64_t groups;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
};

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t c) {
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(mask), "v"(c));
    return d;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// The value of lane l ^ 1 (DPP quad permutation [1, 0, 3, 2]).
__device__ __forceinline__ uint32_t swap_pair(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}

// R activation rows, NW weights (2: fused gate+up), GPW groups a wave, PRO activation chunks a
// lane loads at once while staging.
constexpr int kLaneRows = 4;  // rows a lane covers

template <int R, int NW, bool TILED, int GPW, int PRO>
__global__ void __launch_bounds__(1024)
q4_lane_kernel(LaneArgs args, const uint16_t *__restrict__ act) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int sk = blockDim.x / kWave;
    const int h = lane & 1;
    const int64_t G = args.groups;
    const int64_t K = G * kGroup;
    const int64_t g0 = (int64_t)wave * GPW;
    const int64_t g1 = g0 + GPW < G ? g0 + GPW : G;
    const int64_t rbase = (int64_t)blockIdx.x * 32 * kLaneRows;
    // 32-bit offsets from uniform bases keep the address arithmetic off 64-bit VGPR pairs (the
    // host only sends weights of fewer than 2^32 words here).
    uint32_t row[kLaneRows];
#pragma unroll
    for (int t = 0; t < kLaneRows; ++t) {
        const int64_t rr = rbase + 32 * t + (lane >> 1);
        row[t] = (uint32_t)(rr < args.n ? rr : args.n - 1);
    }
    const uint32_t G32 = (uint32_t)G;
    const uint32_t kMask = 0x000F000Fu;
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));

    // 2. Every weight load of the wave.
    u32x4 wbuf[GPW][NW][kLaneRows];
    uint32_t side[GPW][NW][kLaneRows];
    auto load_slot = [&](int slot, int64_t gi) {
        const int64_t g = gi < g1 ? gi : g1 - 1;
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int t = 0; t < kLaneRows; ++t) {
                uint32_t word, sidx;
                const uint32_t g32 = (uint32_t)g;
                if (TILED) {
                    const uint32_t rec = ((row[t] >> 7) * G32 + g32) * 128u + (row[t] & 127u);
                    word = rec * 8u + 4u * h;
                    sidx = rec;
                } else {
                    word = row[t] * (uint32_t)args.stride_words + g32 * 8u + 4u * h;
                    sidx = row[t] * G32 + g32;
                }
                wbuf[slot][w][t] = *(const u32x4 *)(args.packed[w] + word);
                // Lane h = 0 fetches the scale, h = 1 the bias; they swap at use.
                side[slot][w][t] = (h == 0 ? args.scales[w] : args.biases[w])[sidx];
            }
    };
#pragma unroll
    for (int i = 0; i < GPW; ++i) load_slot(i, g0 + i);

    float acc[NW][R][kLaneRows];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int m = 0; m < R; ++m)
#pragma unroll
            for (int t = 0; t < kLaneRows; ++t) acc[w][m][t] = 0.0f;

#pragma unroll
    for (int i = 0; i < GPW; ++i) {
        const int slot = i;
        const int64_t gi = g0 + i;
        const bool live = gi < g1;
        const int64_t g = live ? gi : g1 - 1;
        // The lane's half group of activations, as pairs (x_j, x_{j+4}), and their sum. (The empty
        // asm keeps the compiler from hoisting every group's activation loads to the top, which
        // would spill.)
        asm volatile("" ::: "memory");
        u32x4 xp[R][4];
        float sx[R];
#pragma unroll
        for (int m = 0; m < R; ++m) {
            const u32x4 *src = (const u32x4 *)(act + (uint32_t)((m < args.rows ? m : 0) * args.lda) + (uint32_t)g * kGroup + 32u * h);
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32x4 v = src[k];
                xp[m][k].x = perm_bytes(v.z, v.x, 0x05040100u);
                xp[m][k].y = perm_bytes(v.z, v.x, 0x07060302u);
                xp[m][k].z = perm_bytes(v.w, v.y, 0x05040100u);
                xp[m][k].w = perm_bytes(v.w, v.y, 0x07060302u);
                s0 = dot2(v.x, 0x3F803F80u, s0);
                s1 = dot2(v.y, 0x3F803F80u, s1);
                s0 = dot2(v.z, 0x3F803F80u, s0);
                s1 = dot2(v.w, 0x3F803F80u, s1);
            }
            sx[m] = s0 + s1;
        }
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int t = 0; t < kLaneRows; ++t) {
                float pq[R], pr[R];
#pragma unroll
                for (int m = 0; m < R; ++m) pq[m] = pr[m] = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t word = wbuf[slot][w][t][k];
                    const uint32_t b0 = and_or(word, kMask, magic);
                    const uint32_t b1 = and_or(word >> 4, kMask, magic);
                    const uint32_t b2 = and_or(word >> 8, kMask, magic);
                    const uint32_t b3 = and_or(word >> 12, kMask, magic);
#pragma unroll
                    for (int m = 0; m < R; ++m) {
                        pq[m] = dot2(b0, xp[m][k][0], pq[m]);
                        pr[m] = dot2(b1, xp[m][k][1], pr[m]);
                        pq[m] = dot2(b2, xp[m][k][2], pq[m]);
                        pr[m] = dot2(b3, xp[m][k][3], pr[m]);
                    }
                }
                const uint32_t mine = side[slot][w][t];
                const uint32_t other = swap_pair(mine);
                const float s = live ? bf16_bits_to_f32(h == 0 ? mine : other) : 0.0f;
                const float b = bf16_bits_to_f32(h == 0 ? other : mine);
                const float bp = live ? __builtin_fmaf(-128.0f, s, b) : 0.0f;
#pragma unroll
                for (int m = 0; m < R; ++m)
                    acc[w][m][t] = __builtin_fmaf(s, pq[m] + pr[m], __builtin_fmaf(bp, sx[m], acc[w][m][t]));
            }
    }

    // Sum the two half lanes of each row, then the waves in LDS: red[wave][w][m][128 rows].
    constexpr int kTile = 32 * kLaneRows;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int m = 0; m < R; ++m)
#pragma unroll
            for (int t = 0; t < kLaneRows; ++t)
                acc[w][m][t] += __builtin_bit_cast(float, swap_pair(__builtin_bit_cast(uint32_t, acc[w][m][t])));
    __syncthreads();
    float *red = (float *)lds_raw;
    if (h == 0) {
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int m = 0; m < R; ++m)
#pragma unroll
                for (int t = 0; t < kLaneRows; ++t) red[((wave * NW + w) * R + m) * kTile + 32 * t + (lane >> 1)] = acc[w][m][t];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < R * kTile; e += blockDim.x) {
        const int m = e / kTile, ln = e % kTile;
        const int64_t nn = rbase + ln;
        if (m >= args.rows || nn >= args.n) continue;
        float v[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            float sum = 0.0f;
            for (int s = 0; s < sk; ++s) sum += red[((s * NW + w) * R + m) * kTile + ln];
            v[w] = sum;
        }
        float value = v[0];
        if constexpr (NW == 2) value = silu(v[0]) * v[NW - 1];
        const int64_t index = m * args.ldc + nn;
        if (args.out_dtype == SPLOSH_F32) {
            if (args.residual) value += ((const float *)args.residual)[index];
            ((float *)args.out)[index] = value;
        } else {
            if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
            ((uint16_t *)args.out)[index] = f32_to_bf16(value);
        }
    }
}

// Groups a wave owns: the smallest bucket that lets at most sixteen waves cover K. All of a
// wave's loads are in registers at once (4 rows x 16 bytes x GPW x NW), which bounds GPW.
static const int kLaneGpw[] = {2, 3, 4, 5};

static int lane_bucket(int64_t groups, int nw, int64_t rows) {
    // Register budget of a 1024-thread workgroup: up to five groups for one row and one weight,
    // two otherwise.
    const int cap = nw == 1 && rows == 1 ? 5 : 2;
    for (int b : kLaneGpw)
        if ((groups + b - 1) / b <= 16 && b <= cap) return b;
    return 0;
}

bool lanes_fit(int64_t rows, int64_t columns, int64_t inner, int64_t stride_words, bool mlp) {
    if (rows > 2 || inner % kGroup != 0) return false;
    // 32-bit word offsets.
    const int64_t words = columns * (stride_words > inner / 8 ? stride_words : inner / 8);
    if (words >= ((int64_t)1 << 32) || rows * inner >= ((int64_t)1 << 31)) return false;
    const int64_t groups = inner / kGroup;
    const int gpw = lane_bucket(groups, mlp ? 2 : 1, rows);
    if (gpw == 0) return false;
    return true;
}

StreamPlan plan_lanes(int64_t rows, int64_t columns, int64_t groups, bool mlp) {
    StreamPlan p;
    p.mb = 1;
    p.row_chunks = 1;
    p.rpl = (int)rows;
    p.col_blocks = (int)((columns + 32 * kLaneRows - 1) / (32 * kLaneRows));
    p.j = lane_bucket(groups, mlp ? 2 : 1, rows);
    p.sk = (int)((groups + p.j - 1) / p.j);
    return p;
}

template <int R, int NW, int GPW>
static hipError_t launch_lane_v(const StreamPlan &p, bool tiled, const LaneArgs &args, hipStream_t stream) {
    dim3 grid((unsigned)p.col_blocks);
    dim3 block((unsigned)(p.sk * kWave));
    const size_t lds = (size_t)p.sk * NW * R * 32 * kLaneRows * 4;
    if (tiled)
        hipLaunchKernelGGL((q4_lane_kernel<R, NW, true, GPW, 8>), grid, block, lds, stream, args, args.a);
    else
        hipLaunchKernelGGL((q4_lane_kernel<R, NW, false, GPW, 8>), grid, block, lds, stream, args, args.a);
    return hipGetLastError();
}

template <int R, int NW>
static hipError_t launch_lane_rn(const StreamPlan &p, bool tiled, const LaneArgs &args, hipStream_t stream) {
    switch (p.j) {
        case 2: return launch_lane_v<R, NW, 2>(p, tiled, args, stream);
        case 3: if constexpr (NW == 1 && R == 1) return launch_lane_v<R, NW, 3>(p, tiled, args, stream); break;
        case 4: if constexpr (NW == 1 && R == 1) return launch_lane_v<R, NW, 4>(p, tiled, args, stream); break;
        case 5: if constexpr (NW == 1 && R == 1) return launch_lane_v<R, NW, 5>(p, tiled, args, stream); break;
        default: break;
    }
    return hipErrorInvalidValue;
}

hipError_t launch_q4_lanes(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                           const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                           int64_t rows, hipStream_t stream) {
    LaneArgs args;
    args.packed[0] = w.packed;
    args.scales[0] = w.scales;
    args.biases[0] = w.biases;
    args.packed[1] = up ? up->packed : w.packed;
    args.scales[1] = up ? up->scales : w.scales;
    args.biases[1] = up ? up->biases : w.biases;
    args.stride_words = w.row_stride_words;
    args.n = w.rows;
    args.groups = w.inner / kGroup;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = rows;
    args.out_dtype = out_dtype;
    const bool tiled = w.order == SPLOSH_Q4_TILED128;
    if (rows == 1)
        return up ? launch_lane_rn<1, 2>(plan, tiled, args, stream) : launch_lane_rn<1, 1>(plan, tiled, args, stream);
    return up ? launch_lane_rn<2, 2>(plan, tiled, args, stream) : launch_lane_rn<2, 1>(plan, tiled, args, stream);
}

}  // namespace splosh
