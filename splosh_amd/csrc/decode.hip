// decode.hip -- decode GEMV (one to four activation rows) over tiled q4 weights on every CU.
//
// The decode step reads a 50 MB weight once. The kernel spreads that read over many small
// workgroups, keeps it in flight while the arithmetic of the groups already loaded runs, and needs
// no reduction across workgroups.
//
// Mapping. A workgroup owns a block of B output rows (B = 8, 16 or 32, inside one 128-row tile) over
// the whole of K: N / B workgroups, several a CU, so the read is spread evenly. In the tiled layout
// (Model/Retile.swift:135-153) the block's records of one group are B * 32 contiguous bytes. Lane l
// of a wave takes half h = l & 1 of row (l >> 1) % B of the group (l >> 1) / B of a step of
// 64 / (2 B) groups, so one 16-byte load a lane reads the step's records in order. The four waves
// take every fourth step.
//
// Activations. The workgroup first stages the activation rows in LDS in the form the arithmetic
// wants: for every 8 consecutive k the four bf16 pairs (x_j, x_{j+4}), and for every half group the
// sum of its 32 activations. Their loads go out before the weight loads (loads complete in order,
// so staging waits for nothing else).
//
// Arithmetic. A code word becomes four bf16 pairs (128 + q_j, 128 + q_{j+4}) with one v_and_or_b32
// each (after a shift), which meet the activation pairs in v_dot2_f32_bf16: with P = sum x (128 + q)
// and S = sum x over the lane's half group, acc += s P + (b - 128 s) S (the per-group identity of
// engine_na.metal:8-20, split over the two halves). Eleven VALU instructions per eight weights and
// row.
//
// Loads in flight. Each wave keeps D steps in flight in a register ring; the loads of a step are
// issued D steps before its arithmetic. Groups past K read an out-of-range buffer offset, which
// returns zero (scale and bias zero: no contribution) without touching memory.
//
// Reduction. The two half lanes of a row meet in a DPP swap, then the waves (and the groups of a
// step) in LDS, and the workgroup writes its B rows (silu(g) * u for the fused gate+up).
//
// Balance. A CU that holds one block more than the others sets the time of the call (at
// K=5120: 512 blocks 10.3 us, 516 blocks 11.6). With a workspace the last round of blocks is
// split over K (plan_balance / balance_block / balance_merge in common.hpp), one slice a CU.
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
    int groups;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int rows;
    int out_dtype;
    uint32_t code_bytes, sidecar_bytes;
    // Balance split (slices > 1): blocks [0, nwhole) whole, blocks nwhole + [0, tail) in `slices`
    // slices of K each; partials [tail][slices][NW][rows][B] fp32 after the counters.
    int nwhole, tail, slices;
    float *partial;
    int *counters;
    uint32_t partial_bytes;
};



// Steps in flight a wave: 3 for one weight when each CU holds a few blocks (a long, latency-bound
// loop: K5120 -> N17408 11.0 -> 10.5 us, K17408 -> N5120 16.7 -> 15.3), else 2 (the fused gate+up
// 18.2 -> 19.6 us and the lm_head, 30 blocks a CU, 101.6 -> 102.5 us at 3; 4 is slower everywhere).
constexpr int kDecodeDepth = 2, kDecodeDeepDepth = 3;
constexpr int kDecodeDeepBlocksPerCu = 4;  // the most blocks a CU for the deeper ring
constexpr int kDecodeWg = 256;   // threads a workgroup
constexpr int kDecodeWaves = kDecodeWg / 64;

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

template <int R, int NW, int B, int D>
__global__ void __launch_bounds__(kDecodeWg)
q4_decode_kernel(DecodeArgs args) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int GPS = 64 / (2 * B);  // groups a step
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane & 1, row = (lane >> 1) % B, gsub = (lane >> 1) / B;
    const int G = args.groups;
    const int K = G * kGroup;
    // This workgroup's block and its groups [ga, gb): all of K, or slice sl of tail block tb.
    int blk, ga, gb, tb, sl;
    balance_block(blockIdx.x, gridDim.x, args.nwhole, args.tail, args.slices, G, blk, ga, gb, tb, sl);
    const int GS = gb - ga;  // groups of this workgroup
    const int steps = (GS + GPS - 1) / GPS;

    // LDS: xp[R][K / 8] (16 bytes: the four activation pairs of a code word), xs[R][K / 32]
    // (half-group sums), red[waves][GPS][NW][R][B] (the partial sums).
    u32x4 *xp = (u32x4 *)lds;
    float *xs = (float *)(xp + R * (K / 8));
    float *red = xs + R * (K / 32);

    // 1. This thread's first activation slices (a half group: 32 values, four 16-byte loads). Item
    // e is half group 2 ga + e mod 2 GS of row e / 2 GS, staged at index m (K / 32) + hg.
    const int items = R * 2 * GS;
    auto item_row = [&](int e) { return e / (2 * GS); };
    auto item_hg = [&](int e) { return 2 * ga + e % (2 * GS); };
    constexpr int kStage = 2;
    u32x4 xin[kStage][4];
#pragma unroll
    for (int t = 0; t < kStage; ++t) {
        const int e = threadIdx.x + t * kDecodeWg;
        const int m = e < items ? item_row(e) : 0, hg = e < items ? item_hg(e) : 2 * ga;
        const u32x4 *src = (const u32x4 *)(args.a + (int64_t)(m < args.rows ? m : 0) * args.lda + hg * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) xin[t][j] = src[j];
    }
    auto stage = [&](int e, const u32x4 (&v)[4]) {  // e: the staging index m (K / 32) + hg
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u32x4 pq;
            pq.x = perm_bytes(v[j].z, v[j].x, 0x05040100u);  // (x0, x4)
            pq.y = perm_bytes(v[j].z, v[j].x, 0x07060302u);  // (x1, x5)
            pq.z = perm_bytes(v[j].w, v[j].y, 0x05040100u);  // (x2, x6)
            pq.w = perm_bytes(v[j].w, v[j].y, 0x07060302u);  // (x3, x7)
            xp[e * 4 + j] = pq;
            s0 = ddot2(v[j].x, 0x3F803F80u, s0);
            s1 = ddot2(v[j].y, 0x3F803F80u, s1);
            s0 = ddot2(v[j].z, 0x3F803F80u, s0);
            s1 = ddot2(v[j].w, 0x3F803F80u, s1);
        }
        xs[e] = s0 + s1;
    };

    // 2. The first D steps' weight loads.
    rsrc_t q_rsrc[NW], s_rsrc[NW], b_rsrc[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        q_rsrc[w] = make_rsrc(args.packed[w], args.code_bytes);
        s_rsrc[w] = make_rsrc(args.scales[w], args.sidecar_bytes);
        b_rsrc[w] = make_rsrc(args.biases[w], args.sidecar_bytes);
    }
    const int64_t r0 = (int64_t)blk * B;
    const uint32_t tile_base = (uint32_t)(r0 >> 7) * (uint32_t)G * 128u + (uint32_t)(r0 & 127) + (uint32_t)row;
    u32x4 cq[D][NW];
    uint32_t cs[D][NW], cb[D][NW];
    auto issue = [&](int slot, int t) {
        // Step t of this wave: groups ga + (wave + 4 t) GPS + gsub.
        const int g = ga + (wave + kDecodeWaves * t) * GPS + gsub;
        const bool live = g < gb;
        const uint32_t rec = tile_base + (uint32_t)(live ? g : 0) * 128u;
        // Out of range: zero, no memory traffic. (Every load is unconditional: a load under a branch
        // makes the compiler's wait counts conservative, which stalls the ring.)
        const uint32_t off = live ? rec * 32u + 16u * h : 0xFFFFFFF0u;
        const uint32_t soff = live ? rec * 2u : 0xFFFFFFF0u;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            cq[slot][w] = buffer_load16_cp<2>(q_rsrc[w], off, 0);
            cs[slot][w] = buffer_load_u16(s_rsrc[w], soff, 0);
            cb[slot][w] = buffer_load_u16(b_rsrc[w], soff, 0);
        }
    };
    // Every wave runs the same number of steps (those past K load zeros and add nothing), so the
    // loop body is straight-line code and the compiler's wait counts keep D steps in flight.
    const int my_steps = (steps + kDecodeWaves - 1) / kDecodeWaves;
#pragma unroll
    for (int k = 0; k < D; ++k) {
        issue(k, k);
        __builtin_amdgcn_sched_barrier(0);  // the same load order as the loop's refills
    }

    // 3. Stage the activations (the rest of them, for long K, after the weight loads went out).
#pragma unroll
    for (int t = 0; t < kStage; ++t) {
        const int e = threadIdx.x + t * kDecodeWg;
        if (e < items) stage(item_row(e) * (K / 32) + item_hg(e), xin[t]);
    }
    for (int e = threadIdx.x + kStage * kDecodeWg; e < items; e += kDecodeWg) {
        const int m = item_row(e), hg = item_hg(e);
        const u32x4 *src = (const u32x4 *)(args.a + (int64_t)(m < args.rows ? m : 0) * args.lda + hg * 32);
        u32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[j];
        stage(m * (K / 32) + hg, v);
    }
    lds_barrier();  // LDS only: the weight loads stay in flight

    const uint32_t kMask = 0x000F000Fu;
    uint32_t magic;  // the bf16 exponent of 128 in both halves
    asm("v_mov_b32 %0, 0x43004300" : "=v"(magic));

    float acc[NW][R];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int m = 0; m < R; ++m) acc[w][m] = 0.0f;

    for (int t0 = 0; t0 < my_steps; t0 += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const int t = t0 + k;
            {
                const int g = ga + (wave + kDecodeWaves * t) * GPS + gsub;
                const int hg = 2 * (g < gb ? g : gb - 1) + h;  // the lane's half group
                u32x4 xq[R][4];
                float sx[R];
#pragma unroll
                for (int m = 0; m < R; ++m) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) xq[m][j] = xp[(m * (K / 32) + hg) * 4 + j];
                    sx[m] = xs[m * (K / 32) + hg];
                }
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    float pq[R], pr[R];
#pragma unroll
                    for (int m = 0; m < R; ++m) pq[m] = pr[m] = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t word = cq[k][w][j];
                        const uint32_t b0 = dand_or(word, kMask, magic);
                        const uint32_t b1 = dand_or(word >> 4, kMask, magic);
                        const uint32_t b2 = dand_or(word >> 8, kMask, magic);
                        const uint32_t b3 = dand_or(word >> 12, kMask, magic);
#pragma unroll
                        for (int m = 0; m < R; ++m) {
                            pq[m] = ddot2(b0, xq[m][j].x, pq[m]);
                            pr[m] = ddot2(b1, xq[m][j].y, pr[m]);
                            pq[m] = ddot2(b2, xq[m][j].z, pq[m]);
                            pr[m] = ddot2(b3, xq[m][j].w, pr[m]);
                        }
                    }
                    const float s = bf16_bits_to_f32(cs[k][w]);
                    const float bp = __builtin_fmaf(-128.0f, s, bf16_bits_to_f32(cb[k][w]));
#pragma unroll
                    for (int m = 0; m < R; ++m)
                        acc[w][m] = __builtin_fmaf(s, pq[m] + pr[m], __builtin_fmaf(bp, sx[m], acc[w][m]));
                }
            }
            issue(k, t + D);
            // Keep the refill here, in the prologue's order: left to itself the scheduler sinks all of
            // them to the end of the unrolled body (and the merged wait counts at the loop head turn
            // conservative), which drains the ring every D steps.
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // 4. Sum the half lanes, then the waves and the groups of a step in LDS; write the B rows.
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int m = 0; m < R; ++m)
            acc[w][m] += __builtin_bit_cast(float, dswap_pair(__builtin_bit_cast(uint32_t, acc[w][m])));
    if (h == 0) {
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int m = 0; m < R; ++m) red[(((wave * GPS + gsub) * NW + w) * R + m) * B + row] = acc[w][m];
    }
    __syncthreads();
    const int tid = threadIdx.x;
    constexpr int RB = R * B;
    const int m = tid / B, rr = tid % B;
    const int64_t nn = r0 + rr;
    float v[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        float sum = 0.0f;
        if (tid < RB) {
#pragma unroll
            for (int p = 0; p < kDecodeWaves * GPS; ++p) sum += red[((p * NW + w) * R + m) * B + rr];
        }
        v[w] = sum;
    }
    auto write_rows = [&] {
        if (tid < RB && m < args.rows && nn < args.n) {
            float value = v[0];
            if constexpr (NW == 2) value = silu(v[0]) * v[1];
            const int64_t index = m * args.ldc + nn;
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) value += ((const float *)args.residual)[index];
                ((float *)args.out)[index] = value;
            } else {
                if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                ((uint16_t *)args.out)[index] = f32_to_bf16(value);
            }
        }
    };
    if (tb >= 0 && !balance_merge<NW>(v, tid, RB, tb, sl, args.slices, args.partial, args.partial_bytes, args.counters))
        return;  // a slice whose block another slice finishes
    write_rows();
}

static int decode_cus() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus;
}

// Row block: 32 rows when that gives at least two workgroups a CU; else 8 for long K (at least 128
// groups), where 16-row blocks would leave a CU one or two workgroups for a long loop (K17408 ->
// N5120: 640 blocks of 8 rows with the balance split 13.3 us, 320 of 16 rows 15.4 us); else 16
// (K5120 -> N5120: 6.5 us at 16 rows, 7.1 at 8).
static int decode_block(int64_t columns, int64_t groups) {
    const int64_t cus = decode_cus();
    if (columns / 32 >= 2 * cus) return 32;
    return groups >= 128 && columns / 16 < 2 * cus ? 8 : 16;
}

static size_t decode_lds(int64_t rows, int64_t inner, int nw, int block) {
    return (size_t)rows * inner * 2 + (size_t)rows * (inner / 32) * 4 +
           (size_t)kDecodeWaves * (64 / (2 * block)) * nw * rows * block * 4;
}

// Activation rows the kernel stages for `rows` rows: 1, 2, or 4 for three or four (a fourth row slot
// reads row 0 again and is not written). Four rows of K5120 -> N17408 (gate+up): 25.6 us against
// 30.0 on the M <= 64 MFMA kernel.
static int decode_rows(int64_t rows) { return rows <= 2 ? (int)rows : 4; }

// LDS a workgroup may take: two workgroups a CU still fit (two rows of K17408: 73 KB).
constexpr size_t kDecodeMaxLds = 80 * 1024;

// Shapes the kernel takes: tiled weights, 32-bit offsets, staged activations within kDecodeMaxLds.
bool decode_fits(int64_t rows, int64_t columns, int64_t inner, int order) {
    if (order != SPLOSH_Q4_TILED128 || rows < 1 || rows > 4 || inner % kGroup != 0 || columns % 128 != 0) return false;
    return decode_lds(decode_rows(rows), inner, 2, 16) <= kDecodeMaxLds &&
           columns * (inner / kGroup) * 32 < ((int64_t)1 << 32) - 4096;
}

static BalanceSplit plan_decode_split(int64_t columns, int groups) {
    return plan_balance(columns / decode_block(columns, groups), decode_cus(), groups);
}

size_t decode_workspace_bytes(int64_t rows, int64_t columns, int64_t inner, int nw) {
    if (rows < 1 || rows > 4 || inner % kGroup != 0 || columns % 128 != 0) return 0;
    const BalanceSplit p = plan_decode_split(columns, (int)(inner / kGroup));
    if (p.slices < 2) return 0;
    return kBalanceCounterBytes +
           (size_t)p.tail * p.slices * nw * decode_rows(rows) * decode_block(columns, inner / kGroup) * sizeof(float);
}

// Raises a kernel's dynamic LDS limit to kDecodeMaxLds once (the default is 64 KB).
template <int R, int NW, int B, int D>
static void decode_lds_attribute() {
    static const bool done = [] {
        (void)hipFuncSetAttribute((const void *)q4_decode_kernel<R, NW, B, D>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)kDecodeMaxLds);
        return true;
    }();
    (void)done;
}

template <int R, int NW, int B>
static hipError_t launch_decode_v(const DecodeArgs &args, hipStream_t stream) {
    const size_t lds = decode_lds(R, (int64_t)args.groups * kGroup, NW, B);
    if (lds > 64 * 1024) {
        decode_lds_attribute<R, NW, B, kDecodeDepth>();
        decode_lds_attribute<R, NW, B, kDecodeDeepDepth>();
    }
    const unsigned grid = args.slices > 1 ? (unsigned)(args.nwhole + args.tail * args.slices) : (unsigned)(args.n / B);
    if (NW == 1 && args.n / B <= (int64_t)kDecodeDeepBlocksPerCu * decode_cus())
        hipLaunchKernelGGL((q4_decode_kernel<R, NW, B, kDecodeDeepDepth>), dim3(grid), dim3(kDecodeWg), lds, stream,
                           args);
    else
        hipLaunchKernelGGL((q4_decode_kernel<R, NW, B, kDecodeDepth>), dim3(grid), dim3(kDecodeWg), lds, stream, args);
    return hipGetLastError();
}

template <int R, int NW>
static hipError_t launch_decode_rn(const DecodeArgs &args, hipStream_t stream) {
    switch (decode_block(args.n, args.groups)) {
        case 32: return launch_decode_v<R, NW, 32>(args, stream);
        case 16: return launch_decode_v<R, NW, 16>(args, stream);
        default: return launch_decode_v<R, NW, 8>(args, stream);
    }
}

hipError_t launch_q4_decode(const splosh_q4_weight &w, const splosh_q4_weight *up, const uint16_t *a, int64_t lda,
                            void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                            void *workspace, size_t workspace_bytes, hipStream_t stream) {
    DecodeArgs args = {};
    args.packed[0] = w.packed;
    args.scales[0] = w.scales;
    args.biases[0] = w.biases;
    args.packed[1] = up ? up->packed : w.packed;
    args.scales[1] = up ? up->scales : w.scales;
    args.biases[1] = up ? up->biases : w.biases;
    args.n = w.rows;
    args.groups = (int)(w.inner / kGroup);
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = (int)rows;
    args.out_dtype = out_dtype;
    args.code_bytes = (uint32_t)(w.rows * args.groups * 32);
    args.sidecar_bytes = (uint32_t)(w.rows * args.groups * 2);
    // The balance split when the workspace holds its partials (else every block whole).
    const int nw = up ? 2 : 1;
    const BalanceSplit split = plan_decode_split(w.rows, args.groups);
    const size_t need = decode_workspace_bytes(rows, w.rows, w.inner, nw);
    if (need > 0 && workspace && workspace_bytes >= need) {
        args.nwhole = split.nwhole;
        args.tail = split.tail;
        args.slices = split.slices;
        args.counters = (int *)workspace;
        args.partial = (float *)((char *)workspace + kBalanceCounterBytes);
        args.partial_bytes = (uint32_t)(need - kBalanceCounterBytes);
    } else {
        args.slices = 1;
    }
    if (rows > 2) return up ? launch_decode_rn<4, 2>(args, stream) : launch_decode_rn<4, 1>(args, stream);
    if (rows == 1)
        return up ? launch_decode_rn<1, 2>(args, stream) : launch_decode_rn<1, 1>(args, stream);
    return up ? launch_decode_rn<2, 2>(args, stream) : launch_decode_rn<2, 1>(args, stream);
}

}  // namespace splosh
