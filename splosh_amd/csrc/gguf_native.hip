// gguf_native.hip -- GGUF Q8_0, Q6_K, Q3_K, IQ4_NL, IQ4_XS and IQ3_S weights read in their
// native blocks.
//
// The reference decodes these formats with GgufTensorType.decode (GgufQuant.swift:136-275) and
// multiplies them on its staged GGUF path (engine_gguf.metal, one decoder a format). Here a weight
// stays in the blocks the GGUF file holds ([rows][inner / block elements] blocks, row after row):
//
//  * gguf_dequant_kernel: one thread a 32-element group, the reference decoder's fp32 operations
//    in its order (bit-exact).
//  * gguf_pairs_kernel: out[m][n] = sum_k a[m][k] w[n][k] for a few rows of activations. A wave
//    owns two weight rows; its lanes take the rows' 32-element groups in turn, 64 a round. Each
//    format forms exact bf16 weight pairs without fp32 arithmetic (group_pairs) and sums with
//    v_dot2. The activations come from LDS, staged once per workgroup (a round at a time from two
//    rows, the whole row for Q8_0 at one), or, for the other formats at one row, from memory. Up
//    to MR activation rows (4, or 8 above four rows) a pass; the partial sums meet in a shuffle
//    tree; further rows take further passes over the weight (grid.y).
//  * gguf_gemv_kernel: Q8_0 at one row when the row does not fit the LDS (K > 32768): a wave
//    owns one weight row, decodes each group into registers exactly as the dequant kernel does
//    and accumulates it in fp32.
//
// Blocks are 2-byte aligned at best (Q8_0: 34 bytes, Q6_K: 210): a run of bytes is read as the
// dword-aligned window that covers it, in 16-byte loads, and shifted into place per lane.
#include "common.hpp"
#include "gguf_decode.hpp"
#include "launch.hpp"

namespace splosh {

struct GgufNativeArgs {
    const uint8_t *w;
    uint32_t w_bytes, row_bytes;
    int64_t rows, inner;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t m;
    int out_dtype;
    float *dense;
    int hs, vph;  // value-head order of the activations (head_group); hs < 0: none
    int rows32;   // the weight in the ROWS32 order (gguf_row)
};

template <int TYPE>
__global__ void __launch_bounds__(256) gguf_dequant_kernel(GgufNativeArgs args) {
    const int64_t groups = args.inner / 32;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= args.rows * groups) return;
    const int64_t n = t / groups;
    const int g = (int)(t % groups);
    const rsrc_t r = make_rsrc(args.w, args.w_bytes);
    float v[32];
    decode_group<TYPE>(r, gguf_row<TYPE>((uint32_t)n, args.row_bytes, args.rows32), g, v);
    f32x4 *dst = (f32x4 *)(args.dense + n * args.inner + (int64_t)g * 32);
#pragma unroll
    for (int q = 0; q < 8; ++q) dst[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
}

// sp_gguf_embed (engine_gguf.metal:302-318) on native blocks: one thread a group of 32 of one
// token's row; an id past the table gives zeros. `dense` receives fp32 (bit-exact) or, with
// out_dtype bf16, bf16 (RNE); args.m is the token count and args.ldc the output row stride.
template <int TYPE>
__global__ void __launch_bounds__(256) gguf_embed_kernel(GgufNativeArgs args, const uint32_t *__restrict__ tokens) {
    const int64_t groups = args.inner / 32;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= args.m * groups) return;
    const int64_t i = t / groups;
    const int g = (int)(t % groups);
    const int64_t row = tokens[i];
    float v[32];
    if (row >= args.rows) {
#pragma unroll
        for (int e = 0; e < 32; ++e) v[e] = 0.0f;
    } else {
        const rsrc_t r = make_rsrc(args.w, args.w_bytes);
        decode_group<TYPE>(r, gguf_row<TYPE>((uint32_t)row, args.row_bytes, args.rows32), g, v);
    }
    if (args.out_dtype == SPLOSH_F32) {
        float *dst = (float *)args.out + i * args.ldc + (int64_t)g * 32;
#pragma unroll
        for (int e = 0; e < 32; ++e) dst[e] = v[e];
    } else {
        uint16_t *dst = (uint16_t *)args.out + i * args.ldc + (int64_t)g * 32;
#pragma unroll
        for (int e = 0; e < 32; ++e) dst[e] = f32_to_bf16(v[e]);
    }
}

typedef __bf16 bf16x2_g __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float gdot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_g, a), __builtin_bit_cast(bf16x2_g, b), c, false);
}

// One group of a weight row as 16 bf16 pairs for v_dot2, with the scales of its two 16-element
// sub-blocks (equal where the format has one scale a group). Pair d holds elements 2 d and 2 d + 1,
// except for IQ4 (elements 4 q + e and 16 + 4 q + e at pair 4 q + e; the activations are paired
// the same way). No fp32 arithmetic touches a weight:
//  * Q6_K, Q3_K (GgufQuant.swift:218-230, 238-256): the raw codes. The bf16 0x4300 | c is exactly
//    128 + c for a code c < 128, so for a sub-block with scale ds and offset o (32, 4),
//    sum x w = ds (sum x (128 + c) - (128 + o) sum x), ds as the reference forms it;
//  * IQ3_S (:283-300): the codebook magnitudes (odd, 1..15) from an LDS table of bf16 pairs, the
//    sign bits moved to bits 15 and 31 of each pair by one multiply and two byte permutes;
//  * IQ4_NL, IQ4_XS (:179-185, 261-275): a code byte's two table values (integers below 128 in
//    magnitude) as one bf16 pair from an LDS table.
// Exact weights and fp32 sums: about three VALU an element where decoding to fp32 and multiplying
// there took six.
struct GroupPairs {
    uint32_t p[16];
    float ds0, ds1;
};

__device__ __forceinline__ void code_pairs(const uint32_t (&codes)[8], GroupPairs &gp) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        gp.p[2 * q] = __builtin_amdgcn_perm(0x43434343u, codes[q], 0x04010400u);
        gp.p[2 * q + 1] = __builtin_amdgcn_perm(0x43434343u, codes[q], 0x04030402u);
    }
}

template <int TYPE>
__device__ __forceinline__ GroupPairs group_pairs(rsrc_t r, GgufRow row, int g, const uint32_t *lut) {
    GroupPairs gp;
    if constexpr (TYPE == 8) {
        const GgufRaw<8> w = gguf_fetch<8>(r, row, g);
        uint32_t h[8];
        align_span(w.codes, h);
        gp.ds0 = gp.ds1 = half_bits_to_f32(w.d);
#pragma unroll
        for (int d = 0; d < 16; ++d)
            gp.p[d] = f32x2_to_bf16x2((float)(int8_t)byte_of(h, 2 * d), (float)(int8_t)byte_of(h, 2 * d + 1));
    } else if constexpr (TYPE == 14) {
        const GgufRaw<14> w = gguf_fetch<14>(r, row, g);
        const int quarter = w.j & 3;
        const float d = half_bits_to_f32(w.d);
        gp.ds0 = d * (float)(int8_t)(w.sc & 0xFF);
        gp.ds1 = d * (float)(int8_t)(w.sc >> 8);
        uint32_t ql[8], qh[8], codes[8];
        align_span(w.ql, ql);
        align_span(w.qh, qh);
        const int lsh = 4 * (quarter >> 1), hsh = 2 * quarter;
#pragma unroll
        for (int q = 0; q < 8; ++q) codes[q] = ((ql[q] >> lsh) & 0x0F0F0F0Fu) | (((qh[q] >> hsh) & 0x03030303u) << 4);
        code_pairs(codes, gp);
    } else if constexpr (TYPE == 11) {
        const GgufRaw<11> w = gguf_fetch<11>(r, row, g);
        const int j = w.j, shift = 2 * (j & 3), word = j >> 1;
        const float d = half_bits_to_f32(w.d);
        const uint32_t lows = w.lows >> (4 * (word >> 1)), highs = w.highs >> (2 * word);
        gp.ds0 = d * ((float)((lows & 0xF) | ((highs & 3) << 4)) - 32.0f);
        gp.ds1 = d * ((float)(((lows >> 8) & 0xF) | (((highs >> 8) & 3) << 4)) - 32.0f);
        uint32_t hm[8], qs[8], codes[8];
        align_span(w.hm, hm);
        align_span(w.qs, qs);
#pragma unroll
        for (int q = 0; q < 8; ++q) codes[q] = ((qs[q] >> shift) & 0x03030303u) | (((hm[q] >> j) & 0x01010101u) << 2);
        code_pairs(codes, gp);
    } else if constexpr (TYPE == 21) {
        const GgufRaw<21> w = gguf_fetch<21>(r, row, g);
        const int j = w.j;
        const float d = half_bits_to_f32(w.d);
        const uint32_t scale = (w.scale >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
        gp.ds0 = gp.ds1 = d * (1.0f + 2.0f * (float)scale);
        const uint32_t ninth = (w.ninth >> (8 * (j & 1))) & 0xFF;
        uint32_t cb[2], sg[1];
        align_span(w.cb, cb);
        align_span(w.sg, sg);
        const uint2 *tab = (const uint2 *)lut;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t code = ((cb[k >> 2] >> (8 * (k & 3))) & 0xFF) | (((ninth >> k) & 1) << 8);
            const uint2 m = tab[code];
            // Sign bit t of elements 4 k + t to bit 7 of byte t, then to bits 15 and 31 of the pairs.
            const uint32_t spread = ((((sg[0] >> (4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u) << 7;
            gp.p[2 * k] = m.x ^ __builtin_amdgcn_perm(0u, spread, 0x010C000Cu);
            gp.p[2 * k + 1] = m.y ^ __builtin_amdgcn_perm(0u, spread, 0x030C020Cu);
        }
    } else {
        uint32_t h[4];
        if constexpr (TYPE == 20) {
            const GgufRaw<20> w = gguf_fetch<20>(r, row, g);
            align_span(w.codes, h);
            gp.ds0 = gp.ds1 = half_bits_to_f32(w.d);
        } else {
            const GgufRaw<23> w = gguf_fetch<23>(r, row, g);
            const int j = w.j;
            const uint32_t low = (w.lowb >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
            const uint32_t scale = low | (((w.high >> (2 * j)) & 3) << 4);
            h[0] = w.q[0], h[1] = w.q[1], h[2] = w.q[2], h[3] = w.q[3];
            gp.ds0 = gp.ds1 = half_bits_to_f32(w.d) * ((float)scale - 32.0f);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) gp.p[4 * q + e] = lut[(h[q] >> (8 * e)) & 0xFFu];
    }
    return gp;
}

// The formats above: R weight rows a wave (a workgroup's four waves take 4 R consecutive rows), so
// each activation row is loaded, paired and summed once for R weight rows; its lanes take the
// rows' 32-element groups in turn, 64 groups a round.
// SA = 1 (from two activation rows): a round's activations are staged in LDS once for the
// workgroup's four waves instead of each wave reading them through the texture path (at K17408 ->
// N5120 and four rows: Q8_0 47.7 -> 35.3 us, Q6_K 50.3 -> 38.2, IQ4_NL 41.3 -> 33.1; at one row
// the barrier a round cost more than it saved, 0.3 - 3 us). SA = 2 (Q8_0 at one row): the whole
// activation row staged once. SA = 0: each lane reads its group's activations from memory.
template <int TYPE, int MR, int R, int SA>
__global__ void __launch_bounds__(256) gguf_pairs_kernel(GgufNativeArgs args) {
    constexpr bool kIq4 = TYPE == 20 || TYPE == 23;
    constexpr float kBias = TYPE == 14 ? 160.0f : TYPE == 11 ? 132.0f : 0.0f;
    // Lookup tables in LDS, built before any wave leaves: IQ3_S's codebook as bf16 magnitude
    // pairs (512 x 8 bytes), the IQ4 values of both nibbles of a byte as a bf16 pair (256 x 4).
    __shared__ __align__(8) uint32_t lut[TYPE == 21 ? 1024 : kIq4 ? 256 : 1];
    if constexpr (kIq4) {
        const uint32_t kv[4] = {kIq4Tab0, kIq4Tab1, kIq4Tab2, kIq4Tab3};
        auto bf = [&](uint32_t i) {
            return __builtin_bit_cast(uint32_t, (float)(int8_t)((kv[i >> 2] >> (8 * (i & 3))) & 0xFFu)) >> 16;
        };
        for (int c = threadIdx.x; c < 256; c += blockDim.x) lut[c] = bf(c & 15) | (bf(c >> 4) << 16);
        __syncthreads();
    }
    if constexpr (TYPE == 21) {
        for (int c = threadIdx.x; c < 512; c += blockDim.x) {
            const uint32_t packed = kIq3sPacked[c];
            uint32_t h[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                h[t] = __builtin_bit_cast(uint32_t, (float)(2u * ((packed >> (3 * t)) & 7u) + 1u)) >> 16;
            lut[2 * c] = h[0] | (h[1] << 16);
            lut[2 * c + 1] = h[2] | (h[3] << 16);
        }
        __syncthreads();
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n0 = ((int64_t)xcd_block(blockIdx.x, gridDim.x) * 4 + wave) * R;
    // A wave past the last weight row leaves, or with SA stages its share of the activations and
    // meets the barriers.
    const bool live = n0 < args.rows;
    if (SA == 0 && !live) return;
    const int64_t m0 = (int64_t)blockIdx.y * MR;
    const int mr = (int)(args.m - m0 < MR ? args.m - m0 : MR);  // activation rows of this pass
    const int groups = (int)(args.inner / 32);
    const rsrc_t rs = make_rsrc(args.w, args.w_bytes);
    GgufRow row[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
        row[r] = gguf_row<TYPE>((uint32_t)(n0 + r < args.rows ? n0 + r : args.rows - 1), args.row_bytes, args.rows32);
    float acc[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < MR; ++i) acc[r][i] = 0.0f;
    // SA: round c's activations, 64 groups of each row (4 KB a row) in buffer c % 2. Wave w loads
    // groups 16 w .. 16 w + 15 of every row, one 16-byte LDS-DMA a lane (lane l: piece l % 4 of
    // the 16 w + l / 4th group, as head_group orders them). Piece p of slot j sits at
    // 4 j + (p ^ (j / 4 % 4)), so that the lanes' 16-byte reads of their own slot, 64 bytes apart,
    // spread over all banks.
    __shared__ __align__(16) u32x4 act_lds[SA == 1 ? 2 : 1][SA == 1 ? MR : 1][SA == 1 ? 256 : 1];
    // SA == 2: every activation row whole, in the same swizzled form (group j of row i at
    // 4 (i groups + j)), staged once before the first round: one barrier for the call.
    extern __shared__ __align__(16) u32x4 act_all[];
    const int aslot = 16 * wave + (lane >> 2);
    const uint32_t apiece = (uint32_t)((lane & 3) ^ ((aslot >> 2) & 3));
    const rsrc_t ars =
        make_rsrc(args.a + m0 * args.lda, SA != 0 ? (uint32_t)(((int64_t)(mr - 1) * args.lda + args.inner) * 2) : 0u);
    auto stage_act = [&](int c) {
        const int g = c * 64 + aslot < groups ? c * 64 + aslot : groups - 1;
        const uint32_t off = (uint32_t)(head_group(g, args.hs, args.vph) * 32 + 8 * apiece) * 2u;
#pragma unroll
        for (int i = 0; i < MR; ++i)
            if (i < mr) buffer_load_lds16(ars, &act_lds[c & 1][i][64 * wave], off + (uint32_t)(i * args.lda * 2));
    };
    const int rounds = (groups + 63) / 64;
    if constexpr (SA == 1) stage_act(0);
    if constexpr (SA == 2) {
        const int total = mr * groups * 4;  // 16-byte pieces; the buffer is rounded up to 256 of them
        for (int base = 64 * wave; base < total; base += 256) {
            const int l = base + lane < total ? base + lane : total - 1;
            const int i = l / (groups * 4), j = (l >> 2) - i * groups;
            const uint32_t p = (uint32_t)((l & 3) ^ ((j >> 2) & 3));
            const uint32_t off = (uint32_t)((int64_t)i * args.lda + head_group(j, args.hs, args.vph) * 32 + 8 * p) * 2u;
            buffer_load_lds16(ars, &act_all[base], off);
        }
        wait_vmcnt<0>();
        __syncthreads();
        if (!live) return;
    }
    for (int c = 0; c < rounds; ++c) {
        if constexpr (SA == 1) {
            // This wave's loads of round c have landed; past the barrier every wave's have, and
            // every wave is done with round c - 1, whose buffer round c + 1 then takes.
            wait_vmcnt<0>();
            __syncthreads();
            if (c + 1 < rounds) stage_act(c + 1);
            asm volatile("" ::: "memory");
        }
        const int g = c * 64 + lane;
        if (!live || g >= groups) continue;
        GroupPairs gp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) gp[r] = group_pairs<TYPE>(rs, row[r], g, lut);
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            if (i >= mr) break;
            uint32_t x[16];
            if constexpr (SA != 0) {
                const u32x4 *ap = SA == 1 ? &act_lds[c & 1][i][4 * lane] : &act_all[4 * (i * groups + g)];
                const int sw = (lane >> 2) & 3;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4 v = ap[q ^ sw];
                    x[4 * q] = v[0], x[4 * q + 1] = v[1], x[4 * q + 2] = v[2], x[4 * q + 3] = v[3];
                }
            } else {
                const u32x4 *ap =
                    (const u32x4 *)(args.a + (m0 + i) * args.lda + (int64_t)head_group(g, args.hs, args.vph) * 32);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4 v = ap[q];
                    x[4 * q] = v[0], x[4 * q + 1] = v[1], x[4 * q + 2] = v[2], x[4 * q + 3] = v[3];
                }
            }
            if constexpr (kIq4) {
                // Elements 4 q + e and 16 + 4 q + e: the low (e even) or high halves of dwords
                // 2 q + e / 2 and 8 + 2 q + e / 2.
                uint32_t y[16];
#pragma unroll
                for (int d = 0; d < 16; ++d) {
                    const int dw = 2 * (d >> 2) + ((d & 3) >> 1);
                    y[d] = __builtin_amdgcn_perm(x[8 + dw], x[dw], (d & 1) ? 0x07060302u : 0x05040100u);
                }
#pragma unroll
                for (int d = 0; d < 16; ++d) x[d] = y[d];
            }
            float t0 = 0.0f, t1 = 0.0f;
            if constexpr (kBias != 0.0f) {
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    t0 = gdot2(x[d], 0x3F803F80u, t0);
                    t1 = gdot2(x[8 + d], 0x3F803F80u, t1);
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    s0 = gdot2(x[d], gp[r].p[d], s0);
                    s1 = gdot2(x[8 + d], gp[r].p[8 + d], s1);
                }
                if constexpr (kBias != 0.0f) {
                    s0 = __builtin_fmaf(-kBias, t0, s0);
                    s1 = __builtin_fmaf(-kBias, t1, s1);
                }
                acc[r][i] = __builtin_fmaf(gp[r].ds0, s0, acc[r][i]);
                acc[r][i] = __builtin_fmaf(gp[r].ds1, s1, acc[r][i]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < MR; ++i) {
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) acc[r][i] += __shfl_xor(acc[r][i], o, 64);
        }
    if (!live || lane != 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (n0 + r >= args.rows) break;
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            if (m0 + i >= args.m) break;
            const int64_t index = (m0 + i) * args.ldc + n0 + r;
            float value = acc[r][i];
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) value += ((const float *)args.residual)[index];
                ((float *)args.out)[index] = value;
            } else {
                if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                ((uint16_t *)args.out)[index] = f32_to_bf16(value);
            }
        }
    }
}

// Q8_0: the group decoded to fp32 in the reference's order, dotted in fp32.
template <int TYPE, int MR>
__global__ void __launch_bounds__(256) gguf_gemv_kernel(GgufNativeArgs args) {
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)xcd_block(blockIdx.x, gridDim.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (n >= args.rows) return;
    const int64_t m0 = (int64_t)blockIdx.y * MR;
    const int groups = (int)(args.inner / 32);
    const rsrc_t r = make_rsrc(args.w, args.w_bytes);
    const GgufRow row = gguf_row<TYPE>((uint32_t)n, args.row_bytes, args.rows32);
    float acc[MR];
#pragma unroll
    for (int i = 0; i < MR; ++i) acc[i] = 0.0f;
    // Two groups an iteration (the second 64 groups on), both decoded before either is used so
    // that their loads are in flight together; the groups left over one at a time.
    auto accumulate = [&](int g, const float (&v)[32]) {
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            if (m0 + i >= args.m) break;
            const u32x4 *ap =
                (const u32x4 *)(args.a + (m0 + i) * args.lda + (int64_t)head_group(g, args.hs, args.vph) * 32);
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4 x = ap[q];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s = __builtin_fmaf(bf16_bits_to_f32(x[e] & 0xffffu), v[8 * q + 2 * e], s);
                    s = __builtin_fmaf(bf16_bits_to_f32(x[e] >> 16), v[8 * q + 2 * e + 1], s);
                }
            }
            acc[i] += s;
        }
    };
    int g = lane;
    // Measured: pairs pay off for Q8_0 (27.8 -> 24.7 us at K17408 -> N5120), not for the formats
    // whose decode holds more registers.
    constexpr bool kPairs = TYPE == 8;
    for (; kPairs && g + 64 < groups; g += 128) {
        float v0[32], v1[32];
        decode_group<TYPE>(r, row, g, v0);
        decode_group<TYPE>(r, row, g + 64, v1);
        accumulate(g, v0);
        accumulate(g + 64, v1);
    }
    for (; g < groups; g += 64) {
        {
            float v[32];
            decode_group<TYPE>(r, row, g, v);
            accumulate(g, v);
        }
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) acc[i] += __shfl_xor(acc[i], o, 64);
    }
    if (lane != 0) return;
#pragma unroll
    for (int i = 0; i < MR; ++i) {
        if (m0 + i >= args.m) break;
        const int64_t index = (m0 + i) * args.ldc + n;
        float value = acc[i];
        if (args.out_dtype == SPLOSH_F32) {
            if (args.residual) value += ((const float *)args.residual)[index];
            ((float *)args.out)[index] = value;
        } else {
            if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
            ((uint16_t *)args.out)[index] = f32_to_bf16(value);
        }
    }
}

int gguf_native_block(int type, int *elems, int *bytes) {
    switch (type & 0xFF) {
        case 8: *elems = 32; *bytes = 34; return 1;
        case 20: *elems = 32; *bytes = 18; return 1;
        case 14: *elems = 256; *bytes = 210; return 1;
        case 23: *elems = 256; *bytes = 136; return 1;
        case 11: *elems = 256; *bytes = 110; return 1;
        case 21: *elems = 256; *bytes = 110; return 1;
        default: return 0;
    }
}

// Fills the weight fields; returns the type id without its layout flag.
static int fill_args(GgufNativeArgs &args, int type, const uint8_t *w, int64_t rows, int64_t inner) {
    args.rows32 = gguf_layout(type);
    int elems = 0, bytes = 0;
    gguf_native_block(type, &elems, &bytes);
    args.w = w;
    args.rows = rows;
    args.inner = inner;
    args.row_bytes = (uint32_t)(inner / elems * bytes);
    const int64_t stored = args.rows32 ? (rows + 31) / 32 * 32 : rows;
    args.w_bytes = (uint32_t)(stored * (int64_t)args.row_bytes);
    return type;
}

// One thread a 2-byte word of the ROWS32 weight: its unit (row n, unit u) and the word's place in
// it, copied from the native order (zero for the padding rows). Every block is an even number of
// bytes, so words never straddle a unit.
__global__ void __launch_bounds__(256) gguf_rows32_kernel(const uint16_t *__restrict__ native, int64_t rows,
                                                          int64_t units, int unit_words, uint16_t *__restrict__ out,
                                                          int64_t total) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;
    const int64_t slot = t / unit_words, wd = t - slot * unit_words;  // slot: unit position in ROWS32
    const int64_t grp = slot / (units * 32), rem = slot - grp * units * 32;
    const int64_t u = rem / 32, n = grp * 32 + rem % 32;
    out[t] = n < rows ? native[(n * units + u) * unit_words + wd] : (uint16_t)0;
}

hipError_t launch_gguf_repack_rows32(int type, const uint8_t *native, int64_t rows, int64_t inner, uint8_t *out,
                                     hipStream_t stream) {
    type &= 0xFF;
    int elems = 0, bytes = 0;
    gguf_native_block(type, &elems, &bytes);
    const int unit_words = 256 / elems * bytes / 2;
    const int64_t units = inner / 256, total = (rows + 31) / 32 * 32 * units * unit_words;
    hipLaunchKernelGGL(gguf_rows32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       (const uint16_t *)native, rows, units, unit_words, (uint16_t *)out, total);
    return hipGetLastError();
}

hipError_t launch_gguf_dequant(int type, const uint8_t *w, int64_t rows, int64_t inner, float *dense,
                               hipStream_t stream) {
    GgufNativeArgs args = {};
    type = fill_args(args, type, w, rows, inner);
    args.dense = dense;
    const int64_t threads = rows * (inner / 32);
    const dim3 grid((unsigned)((threads + 255) / 256));
    switch (type) {
        case 8: hipLaunchKernelGGL(gguf_dequant_kernel<8>, grid, dim3(256), 0, stream, args); break;
        case 20: hipLaunchKernelGGL(gguf_dequant_kernel<20>, grid, dim3(256), 0, stream, args); break;
        case 14: hipLaunchKernelGGL(gguf_dequant_kernel<14>, grid, dim3(256), 0, stream, args); break;
        case 11: hipLaunchKernelGGL(gguf_dequant_kernel<11>, grid, dim3(256), 0, stream, args); break;
        case 21: hipLaunchKernelGGL(gguf_dequant_kernel<21>, grid, dim3(256), 0, stream, args); break;
        default: hipLaunchKernelGGL(gguf_dequant_kernel<23>, grid, dim3(256), 0, stream, args); break;
    }
    return hipGetLastError();
}

hipError_t launch_gguf_embed(int type, const uint8_t *w, int64_t rows, int64_t inner, const uint32_t *tokens,
                             int64_t count, void *out, int64_t ldo, int out_dtype, hipStream_t stream) {
    GgufNativeArgs args = {};
    type = fill_args(args, type, w, rows, inner);
    args.m = count;
    args.out = out;
    args.ldc = ldo;
    args.out_dtype = out_dtype;
    const dim3 grid((unsigned)((count * (inner / 32) + 255) / 256));
    switch (type) {
        case 8: hipLaunchKernelGGL(gguf_embed_kernel<8>, grid, dim3(256), 0, stream, args, tokens); break;
        case 20: hipLaunchKernelGGL(gguf_embed_kernel<20>, grid, dim3(256), 0, stream, args, tokens); break;
        case 14: hipLaunchKernelGGL(gguf_embed_kernel<14>, grid, dim3(256), 0, stream, args, tokens); break;
        case 11: hipLaunchKernelGGL(gguf_embed_kernel<11>, grid, dim3(256), 0, stream, args, tokens); break;
        case 21: hipLaunchKernelGGL(gguf_embed_kernel<21>, grid, dim3(256), 0, stream, args, tokens); break;
        default: hipLaunchKernelGGL(gguf_embed_kernel<23>, grid, dim3(256), 0, stream, args, tokens); break;
    }
    return hipGetLastError();
}

#ifndef GGUF_PAIRS_R
#define GGUF_PAIRS_R 2
#endif
constexpr int kPairsRows = GGUF_PAIRS_R;  // weight rows a wave of gguf_pairs_kernel

template <int MR, int SA>
static void launch_pairs(int type, const GgufNativeArgs &args, dim3 grid, size_t lds, hipStream_t stream) {
    constexpr int R = kPairsRows;
    switch (type) {
        case 8: hipLaunchKernelGGL((gguf_pairs_kernel<8, MR, R, SA>), grid, dim3(256), lds, stream, args); break;
        case 20: hipLaunchKernelGGL((gguf_pairs_kernel<20, MR, R, SA>), grid, dim3(256), lds, stream, args); break;
        case 14: hipLaunchKernelGGL((gguf_pairs_kernel<14, MR, R, SA>), grid, dim3(256), lds, stream, args); break;
        case 11: hipLaunchKernelGGL((gguf_pairs_kernel<11, MR, R, SA>), grid, dim3(256), lds, stream, args); break;
        case 21: hipLaunchKernelGGL((gguf_pairs_kernel<21, MR, R, SA>), grid, dim3(256), lds, stream, args); break;
        default: hipLaunchKernelGGL((gguf_pairs_kernel<23, MR, R, SA>), grid, dim3(256), lds, stream, args); break;
    }
}

template <int MR>
static void launch_gemv_mr(int type, const GgufNativeArgs &args, hipStream_t stream) {
    constexpr int R = kPairsRows;
    const dim3 grid((unsigned)((args.rows + 4 * R - 1) / (4 * R)), (unsigned)((args.m + MR - 1) / MR));
    if constexpr (MR == 4) {
        if (args.m == 1) {
            // One activation row. Q8_0 stages the whole row in LDS (up to 64 KB: K <= 32768) and
            // takes the pairs form: 26.3 -> 22.9 us at K17408 -> N5120, 30.3 -> 24.9 at K5120 ->
            // N17408, against its fp32 decode reading the activations from memory (which still
            // serves longer rows). For the other formats the whole-row staging measured slower
            // (IQ4_XS 17.3 -> 20.3 us, Q3_K 21.7 -> 23.5), and they read the activations directly.
            const size_t whole = (size_t)((args.inner / 32 * 4 + 255) / 256 * 256) * 16;
            if (type == 8 && whole <= 65536)
                hipLaunchKernelGGL((gguf_pairs_kernel<8, MR, R, 2>), grid, dim3(256), whole, stream, args);
            else if (type == 8)
                hipLaunchKernelGGL((gguf_gemv_kernel<8, MR>), dim3((unsigned)((args.rows + 3) / 4), grid.y),
                                   dim3(256), 0, stream, args);
            else
                launch_pairs<MR, 0>(type, args, grid, 0, stream);
            return;
        }
    }
    launch_pairs<MR, 1>(type, args, grid, 0, stream);
}

// One 16-byte piece (8 activations) a thread: piece p of row m comes from group head_group(p / 4).
__global__ void __launch_bounds__(256) head_gather_kernel(const uint16_t *__restrict__ a, int64_t lda, int64_t m,
                                                          int64_t inner, int hs, int vph, uint16_t *__restrict__ dst) {
    const int64_t pieces = inner / 8;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= m * pieces) return;
    const int64_t row = t / pieces, p = t - row * pieces;
    const int g = (int)(p >> 2);
    const int64_t src = row * lda + (int64_t)head_group(g, hs, vph) * 32 + (p & 3) * 8;
    *(u32x4 *)(dst + row * inner + p * 8) = *(const u32x4 *)(a + src);
}

hipError_t launch_head_gather(const uint16_t *a, int64_t lda, int64_t m, int64_t inner, int hs, int vph,
                              uint16_t *dst, hipStream_t stream) {
    const int64_t total = m * (inner / 8);
    hipLaunchKernelGGL(head_gather_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, a, lda, m,
                       inner, hs, vph, dst);
    return hipGetLastError();
}

// Activation rows a pass over the weight: four up to four rows, eight above (one pass up to
// eight rows instead of two).
hipError_t launch_gguf_gemv(int type, const uint8_t *w, int64_t rows, int64_t inner, const uint16_t *a, int64_t lda,
                            void *out, int64_t ldc, int out_dtype, const void *residual, int64_t m,
                            hipStream_t stream, int hs, int vph) {
    GgufNativeArgs args = {};
    type = fill_args(args, type, w, rows, inner);
    args.hs = hs;
    args.vph = vph;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.out_dtype = out_dtype;
    args.residual = residual;
    args.m = m;
    if (m > 4)
        launch_gemv_mr<8>(type, args, stream);
    else
        launch_gemv_mr<4>(type, args, stream);
    return hipGetLastError();
}

}  // namespace splosh
