// q5k_decode.hip -- decode GEMV (one activation row) over GGUF Q5_K (and Q4_K) planes on every CU.
//
// The same structure as the q4 decode kernel (decode.hip): a workgroup owns a block of B output
// rows over the whole of K, stages the activation row in LDS once, and streams the block's records
// through a short register ring of straight-line loads; no reduction across workgroups.
//
// Mapping. Lane l takes row l % B of the block and one 32-element group, (l / B) of the step's
// 64 / B groups; the four waves take every fourth step. Per group a lane reads its 16-byte plane0
// record (low nibbles in chunk order), its 4-byte plane1 record (fifth bits) and the 16-byte meta
// record of the group's block (fp16 d, dmin, packed 6-bit scales and minimums;
// Model/GgufPlanes.swift:8-20).
//
// Arithmetic. In chunk order (gguf_formats.h:17-21) pair p of plane0 word c, (w >> 4p) & 0x000F000F,
// holds two consecutive elements e0, e0 + 1 (e0 = 16 (p >> 1) + 4 c + 2 (p & 1)) in its 16-bit
// halves, so the activations need no permutation: the pair meets the bf16 pair (x_e0, x_e0+1) as
// staged. Their fifth bits are plane1 bits 8 c + 2 p and 8 c + 2 p + 1: a 256-entry LDS table,
// indexed by plane1 byte c, holds for each of the word's four pairs those two bits at bits 4 and 20
// over the bf16 exponent of 128, so one v_and_or_b32 of the shifted word into table word p gives
// the bf16 pair (128 + code_e0, 128 + code_e0+1), code = nibble + 16 bit (one 16-byte LDS read a
// word instead of three VALU a pair). With P = sum x (128 + code)
// and S = sum x over the group, sum x w = ds P - (128 ds + dm) S for w = code ds - dm, ds = d sc,
// dm = dmin mn (GgufQuant.swift:191-212).
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

typedef __bf16 bf16x2_q __attribute__((ext_vector_type(2)));

struct Q5DecodeArgs {
    const uint8_t *plane0, *plane1, *meta;
    int64_t n;
    int groups;  // 32-element groups a row
    const uint16_t *a;
    void *out;
    const void *residual;
    int out_dtype;
    uint32_t p0_bytes, p1_bytes, meta_bytes;
    int hs, vph;  // value-head order of the activations (head_group); hs < 0: none
    // Balance split of the last round of blocks (slices > 1; common.hpp): partials
    // [tail][slices][B] fp32 after the counters.
    int nwhole, tail, slices;
    float *partial;
    int *counters;
    uint32_t partial_bytes;
};

constexpr int kQ5DecodeDepth = 2;  // steps in flight a wave
constexpr int kQ5DecodeWg = 256;
constexpr int kQ5DecodeWaves = kQ5DecodeWg / 64;
static_assert(kQ5DecodeWg == 256, "one thread builds each of the 256 fifth-bit table entries");

__device__ __forceinline__ float qdot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_q, a), __builtin_bit_cast(bf16x2_q, b), c, false);
}
__device__ __forceinline__ uint32_t qand_or(uint32_t a, uint32_t mask, uint32_t c) {
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(mask), "v"(c));
    return d;
}

// FIFTH = false: Q4_K (no plane1; the codes are the nibbles).
template <int B, int D, bool FIFTH>
__global__ void __launch_bounds__(kQ5DecodeWg)
q5k_decode_kernel(Q5DecodeArgs args) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int GPS = 64 / B;  // groups a step
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row = lane % B, gsub = lane / B;
    const int G = args.groups;
    const int K = G * 32;
    const uint32_t blocks = (uint32_t)G / 8u;
    // This workgroup's block and its groups [ga, gb): all of K, or slice sl of tail block tb.
    int blk, ga, gb, tb, sl;
    balance_block(blockIdx.x, gridDim.x, args.nwhole, args.tail, args.slices, G, blk, ga, gb, tb, sl);
    const int GS = gb - ga;
    const int steps = (GS + GPS - 1) / GPS;

    // LDS: fifth[256] (the fifth-bit table), xa[K / 8] (16 bytes: 8 activations as staged), xs[G]
    // (group sums), red[waves][GPS][B].
    u32x4 *fifth = (u32x4 *)lds;
    u32x4 *xa = fifth + 256;
    float *xs = (float *)(xa + K / 8);
    float *red = xs + G;

    // 1. This thread's first activation groups (32 values, four 16-byte loads each): groups
    // ga + e of this workgroup's range.
    constexpr int kStage = 2;
    u32x4 xin[kStage][4];
#pragma unroll
    for (int t = 0; t < kStage; ++t) {
        const int e = threadIdx.x + t * kQ5DecodeWg;
        const u32x4 *src = (const u32x4 *)(args.a + head_group(ga + (e < GS ? e : 0), args.hs, args.vph) * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) xin[t][j] = src[j];
    }
    auto stage = [&](int e, const u32x4 (&v)[4]) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xa[e * 4 + j] = v[j];
            s0 = qdot2(v[j].x, 0x3F803F80u, s0);
            s1 = qdot2(v[j].y, 0x3F803F80u, s1);
            s0 = qdot2(v[j].z, 0x3F803F80u, s0);
            s1 = qdot2(v[j].w, 0x3F803F80u, s1);
        }
        xs[e] = s0 + s1;
    };

    // 2. The first D steps' loads. Every load is unconditional (groups past K read an out-of-range
    // offset: zeros, no memory traffic), so the compiler's wait counts keep the ring in flight.
    const rsrc_t p0_rsrc = make_rsrc(args.plane0, args.p0_bytes);
    const rsrc_t p1_rsrc = make_rsrc(FIFTH ? args.plane1 : args.plane0, FIFTH ? args.p1_bytes : 0u);
    const rsrc_t m_rsrc = make_rsrc(args.meta, args.meta_bytes);
    const int64_t r0 = (int64_t)blk * B;
    const uint32_t rr = (uint32_t)(r0 & 127) + (uint32_t)row;
    const uint32_t tile = (uint32_t)(r0 >> 7);
    u32x4 c0[D], cm[D];
    uint32_t c1[D] = {};
    auto issue = [&](int slot, int t) {
        const int g = ga + (wave + kQ5DecodeWaves * t) * GPS + gsub;
        const bool live = g < gb;
        const uint32_t gg = live ? (uint32_t)g : 0u;
        const uint32_t rec = (tile * (uint32_t)G + gg) * 128u + rr;
        const uint32_t mrec = (tile * blocks + gg / 8u) * 128u + rr;
        c0[slot] = buffer_load16_cp<2>(p0_rsrc, live ? rec * 16u : 0xFFFFFFF0u, 0);
        if constexpr (FIFTH) c1[slot] = buffer_load_u32(p1_rsrc, live ? rec * 4u : 0xFFFFFFF0u, 0);
        cm[slot] = buffer_load16(m_rsrc, live ? mrec * 16u : 0xFFFFFFF0u, 0);
    };
    const int my_steps = (steps + kQ5DecodeWaves - 1) / kQ5DecodeWaves;
#pragma unroll
    for (int k = 0; k < D; ++k) {
        issue(k, k);
        __builtin_amdgcn_sched_barrier(0);  // the same load order as the loop's refills
    }

    // 3. The fifth-bit table (entry x, word p: bits 2p and 2p + 1 of x at bits 4 and 20, over
    // 0x43004300), and the activations (the rest, for long K, after the weight loads went out).
    if constexpr (FIFTH) {
        const uint32_t x = threadIdx.x;  // kQ5DecodeWg == 256 entries
        u32x4 e;
#pragma unroll
        for (int p = 0; p < 4; ++p) e[p] = 0x43004300u | (((x >> (2 * p)) & 1u) << 4) | (((x >> (2 * p + 1)) & 1u) << 20);
        fifth[x] = e;
    }
#pragma unroll
    for (int t = 0; t < kStage; ++t)
        if (threadIdx.x + t * kQ5DecodeWg < GS) stage(ga + threadIdx.x + t * kQ5DecodeWg, xin[t]);
    for (int e = threadIdx.x + kStage * kQ5DecodeWg; e < GS; e += kQ5DecodeWg) {
        const u32x4 *src = (const u32x4 *)(args.a + head_group(ga + e, args.hs, args.vph) * 32);
        u32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[j];
        stage(ga + e, v);
    }
    lds_barrier();  // LDS only: the weight loads stay in flight

    const uint32_t kMask = 0x000F000Fu;
    uint32_t magic;  // the bf16 exponent of 128 in both halves
    asm("v_mov_b32 %0, 0x43004300" : "=v"(magic));

    float acc = 0.0f;
    for (int t0 = 0; t0 < my_steps; t0 += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const int t = t0 + k;
            const int g0 = ga + (wave + kQ5DecodeWaves * t) * GPS + gsub;
            const int g = g0 < gb ? g0 : gb - 1;  // past the range: zero scales, no contribution
            u32x4 xq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) xq[j] = xa[g * 4 + j];
            const float sx = xs[g];
            // Scale and minimum of group j = g % 8 (GgufQuant.swift:196-203): packed byte k is meta
            // byte 4 + k; both forms are computed and one is selected (no divergent branch).
            const u32x4 m = cm[k];
            const uint32_t j = (uint32_t)g & 7u, sh = 8u * (j & 3u);
            const uint32_t sc_lo = __builtin_amdgcn_ubfe(m[1], sh, 6), mn_lo = __builtin_amdgcn_ubfe(m[2], sh, 6);
            const uint32_t sc_hi = __builtin_amdgcn_ubfe(m[3], sh, 4) | (__builtin_amdgcn_ubfe(m[1], sh + 6, 2) << 4);
            const uint32_t mn_hi = __builtin_amdgcn_ubfe(m[3], sh + 4, 4) | (__builtin_amdgcn_ubfe(m[2], sh + 6, 2) << 4);
            const bool upper = j >= 4u;
            const float d = half_bits_to_f32(m[0]), dmin = half_bits_to_f32(m[0] >> 16);
            const float ds = d * (float)(upper ? sc_hi : sc_lo);
            const float dm = dmin * (float)(upper ? mn_hi : mn_lo);
            float pa = 0.0f, pb = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t w = c0[k][c];
                u32x4 hi = {};  // the pairs' fifth bits over the exponent of 128
                if constexpr (FIFTH) hi = fifth[__builtin_amdgcn_ubfe(c1[k], 8 * c, 8)];
                // The word's four pairs first, then their dot products (a pair consumed by the very
                // next instruction costs a wait state).
                uint32_t pair[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) pair[p] = qand_or(p ? w >> (4 * p) : w, kMask, FIFTH ? hi[p] : magic);
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint32_t xw = xq[(p >> 1) * 2 + (c >> 1)][(c & 1) * 2 + (p & 1)];  // x u32 8(p>>1) + 2c + (p&1)
                    if (p & 1) pb = qdot2(pair[p], xw, pb);
                    else pa = qdot2(pair[p], xw, pa);
                }
            }
            const float live = g0 < gb ? 1.0f : 0.0f;
            acc = __builtin_fmaf(ds * live, pa + pb, __builtin_fmaf(-__builtin_fmaf(128.0f, ds, dm) * live, sx, acc));
            issue(k, t + D);
            // Keep the refill here, in the prologue's order (else the scheduler sinks the refills
            // to the end of the unrolled body and the ring drains every D steps).
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // 4. The groups of a step and the waves meet in LDS; the workgroup writes its B rows.
    red[(wave * GPS + gsub) * B + row] = acc;
    __syncthreads();
    const int tid = threadIdx.x;
    float v[1] = {0.0f};
    if (tid < B) {
#pragma unroll
        for (int p = 0; p < kQ5DecodeWaves * GPS; ++p) v[0] += red[p * B + tid];
    }
    if (tb >= 0 && !balance_merge<1>(v, tid, B, tb, sl, args.slices, args.partial, args.partial_bytes, args.counters))
        return;  // a slice whose block another slice finishes
    if (tid < B) {
        const int64_t nn = r0 + tid;
        float value = v[0];
        if (nn < args.n) {
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) value += ((const float *)args.residual)[nn];
                ((float *)args.out)[nn] = value;
            } else {
                if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[nn]);
                ((uint16_t *)args.out)[nn] = f32_to_bf16(value);
            }
        }
    }
}

static size_t q5k_decode_lds(int64_t inner, int block) {
    return (size_t)256 * 16 + (size_t)inner * 2 + (size_t)(inner / 32) * 4 +
           (size_t)kQ5DecodeWaves * (64 / block) * block * 4;
}

bool q5k_decode_fits(int64_t rows, int64_t columns, int64_t inner) {
    return rows == 1 && columns % 128 == 0 && inner % 256 == 0 && q5k_decode_lds(inner, 8) <= 64 * 1024 &&
           columns * (inner / 32) * 16 < ((int64_t)1 << 32) - 4096;
}

static int q5k_decode_cus() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus;
}

// Row block: the largest of 32, 16 and 8 that gives at least two workgroups a CU.
static int q5k_decode_block(int64_t columns) {
    const int64_t cus = q5k_decode_cus();
    return columns / 32 >= 2 * cus ? 32 : columns / 16 >= 2 * cus ? 16 : 8;
}

size_t q5k_decode_workspace_bytes(int64_t rows, int64_t columns, int64_t inner) {
    if (rows != 1 || columns % 128 != 0 || inner % 256 != 0) return 0;
    const int block = q5k_decode_block(columns);
    const BalanceSplit p = plan_balance(columns / block, q5k_decode_cus(), (int)(inner / 32));
    return p.slices < 2 ? 0 : kBalanceCounterBytes + (size_t)p.tail * p.slices * block * sizeof(float);
}

template <int B, bool FIFTH>
static hipError_t launch_q5k_decode_b(const Q5DecodeArgs &args, hipStream_t stream) {
    const unsigned grid = args.slices > 1 ? (unsigned)(args.nwhole + args.tail * args.slices) : (unsigned)(args.n / B);
    hipLaunchKernelGGL((q5k_decode_kernel<B, kQ5DecodeDepth, FIFTH>), dim3(grid), dim3(kQ5DecodeWg),
                       q5k_decode_lds((int64_t)args.groups * 32, B), stream, args);
    return hipGetLastError();
}

hipError_t launch_q5k_decode(const splosh_q5k_weight &w, const uint16_t *a, void *out, int out_dtype,
                             const void *residual, void *workspace, size_t workspace_bytes, hipStream_t stream, int hs,
                             int vph) {
    Q5DecodeArgs args = {};
    args.hs = hs;
    args.vph = vph;
    args.plane0 = w.plane0;
    args.plane1 = w.plane1;
    args.meta = w.meta;
    args.n = w.rows;
    args.groups = (int)(w.inner / 32);
    args.a = a;
    args.out = out;
    args.residual = residual;
    args.out_dtype = out_dtype;
    args.p0_bytes = (uint32_t)(w.rows * args.groups * 16);
    args.p1_bytes = w.plane1 ? (uint32_t)(w.rows * args.groups * 4) : 0u;
    args.meta_bytes = (uint32_t)(w.rows * (args.groups / 8) * 16);
    const int block = q5k_decode_block(w.rows);
    // The balance split when the workspace holds its partials (else every block whole).
    const size_t need = q5k_decode_workspace_bytes(1, w.rows, w.inner);
    args.slices = 1;
    if (need > 0 && workspace && workspace_bytes >= need) {
        const BalanceSplit p = plan_balance(w.rows / block, q5k_decode_cus(), args.groups);
        args.nwhole = p.nwhole;
        args.tail = p.tail;
        args.slices = p.slices;
        args.counters = (int *)workspace;
        args.partial = (float *)((char *)workspace + kBalanceCounterBytes);
        args.partial_bytes = (uint32_t)(need - kBalanceCounterBytes);
    }
    const bool fifth = w.plane1 != nullptr;  // null: Q4_K
    if (block == 32)
        return fifth ? launch_q5k_decode_b<32, true>(args, stream) : launch_q5k_decode_b<32, false>(args, stream);
    if (block == 16)
        return fifth ? launch_q5k_decode_b<16, true>(args, stream) : launch_q5k_decode_b<16, false>(args, stream);
    return fifth ? launch_q5k_decode_b<8, true>(args, stream) : launch_q5k_decode_b<8, false>(args, stream);
}

}  // namespace splosh
