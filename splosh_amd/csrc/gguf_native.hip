// gguf_native.hip -- GGUF Q8_0, Q6_K, Q3_K, IQ4_NL, IQ4_XS and IQ3_S weights read in their
// native blocks.
//
// The reference decodes these formats with GgufTensorType.decode (GgufQuant.swift:136-275) and
// multiplies them on its staged GGUF path (engine_gguf.metal, one decoder a format). Here a weight
// stays in the blocks the GGUF file holds ([rows][inner / block elements] blocks, row after row):
//
//  * gguf_dequant_kernel: one thread a 32-element group, the reference decoder's fp32 operations
//    in its order (bit-exact).
//  * gguf_gemv_kernel: out[m][n] = sum_k a[m][k] w[n][k] for a few rows of activations. A wave
//    owns one weight row; its lanes take the row's 32-element groups in turn, decode each into
//    registers exactly as the dequant kernel does and accumulate it against up to MR activation
//    rows (fp32); Q6_K and Q3_K instead multiply their raw codes as bf16 and apply the scales
//    per sub-block (raw_code_dot), IQ3_S its signed codebook magnitudes (iq3s_dot), IQ4_NL and
//    IQ4_XS their table values (iq4_dot), all as bf16 pairs into v_dot2. The wave's partial sums meet in a shuffle tree. Rows beyond
//    MR (4, or 8 above four rows) take further passes over the weight (grid.y).
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
    decode_group<TYPE>(r, (uint32_t)(n * args.row_bytes), g, v);
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
        decode_group<TYPE>(r, (uint32_t)(row * args.row_bytes), g, v);
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

// A K-quant group on its raw codes (Q6_K, GgufQuant.swift:218-230; Q3_K, :238-256): the bf16
// 0x4300 | c is exactly 128 + c for a code c < 128, so with x the activations of one 16-element
// sub-block, sum x w = ds (sum x (128 + c) - (128 + o) sum x) for w = ds (c - o), ds as the
// reference forms it (o = 32 for Q6_K, 4 for Q3_K). Both sums are v_dot2 on bf16 pairs (exact
// products, fp32 sums): about three VALU an element in place of six for decoding to fp32 and
// multiplying there. `codes[q]` holds the codes of elements 4 q .. 4 q + 3, a byte each.
template <int MR>
__device__ __forceinline__ void raw_code_dot(const uint32_t (&codes)[8], float ds0, float ds1, float bias,
                                             const GgufNativeArgs &args, int64_t m0, int g, float (&acc)[MR]) {
    uint32_t p[16];  // bf16 pairs (128 + c) of elements 2 i, 2 i + 1
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        p[2 * q] = __builtin_amdgcn_perm(0x43434343u, codes[q], 0x04010400u);
        p[2 * q + 1] = __builtin_amdgcn_perm(0x43434343u, codes[q], 0x04030402u);
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
        if (m0 + i >= args.m) break;
        const u32x4 *ap = (const u32x4 *)(args.a + (m0 + i) * args.lda + (int64_t)g * 32);
        float s[2] = {0.0f, 0.0f}, t[2] = {0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 x = ap[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s[q >> 1] = gdot2(x[e], p[4 * q + e], s[q >> 1]);
                t[q >> 1] = gdot2(x[e], 0x3F803F80u, t[q >> 1]);
            }
        }
        acc[i] = __builtin_fmaf(ds0, __builtin_fmaf(-bias, t[0], s[0]), acc[i]);
        acc[i] = __builtin_fmaf(ds1, __builtin_fmaf(-bias, t[1], s[1]), acc[i]);
    }
}

template <int MR>
__device__ __forceinline__ void q6k_dot(const GgufRaw<14> &w, const GgufNativeArgs &args, int64_t m0, int g,
                                        float (&acc)[MR]) {
    const int quarter = w.j & 3;
    const float d = half_bits_to_f32(w.d);
    const float ds0 = d * (float)(int8_t)(w.sc & 0xFF), ds1 = d * (float)(int8_t)(w.sc >> 8);
    uint32_t ql[8], qh[8], codes[8];
    align_span(w.ql, ql);
    align_span(w.qh, qh);
    const int lsh = 4 * (quarter >> 1), hsh = 2 * quarter;
#pragma unroll
    for (int q = 0; q < 8; ++q) codes[q] = ((ql[q] >> lsh) & 0x0F0F0F0Fu) | (((qh[q] >> hsh) & 0x03030303u) << 4);
    raw_code_dot<MR>(codes, ds0, ds1, 160.0f, args, m0, g, acc);
}

template <int MR>
__device__ __forceinline__ void q3k_dot(const GgufRaw<11> &w, const GgufNativeArgs &args, int64_t m0, int g,
                                        float (&acc)[MR]) {
    const int j = w.j, shift = 2 * (j & 3), word = j >> 1;
    const float d = half_bits_to_f32(w.d);
    const uint32_t lows = w.lows >> (4 * (word >> 1)), highs = w.highs >> (2 * word);
    const float s0 = (float)((lows & 0xF) | ((highs & 3) << 4)) - 32.0f;
    const float s1 = (float)(((lows >> 8) & 0xF) | (((highs >> 8) & 3) << 4)) - 32.0f;
    uint32_t hm[8], qs[8], codes[8];
    align_span(w.hm, hm);
    align_span(w.qs, qs);
#pragma unroll
    for (int q = 0; q < 8; ++q) codes[q] = ((qs[q] >> shift) & 0x03030303u) | (((hm[q] >> j) & 0x01010101u) << 2);
    raw_code_dot<MR>(codes, d * s0, d * s1, 132.0f, args, m0, g, acc);
}

// IQ3_S group g (GgufQuant.swift:283-300) on bf16 weights formed without fp32 arithmetic: `tab`
// holds each codebook entry's four magnitudes (odd, 1..15: exact in bf16) as two bf16 pairs, the
// sign bits are spread to bits 15 and 31 of each pair by one multiply and two byte permutes, and
// the group's d (1 + 2 scale) multiplies the v_dot2 sum once.
template <int MR>
__device__ __forceinline__ void iq3s_dot(const GgufRaw<21> &w, const uint2 *tab, const GgufNativeArgs &args,
                                         int64_t m0, int g, float (&acc)[MR]) {
    const int j = w.j;
    const float d = half_bits_to_f32(w.d);
    const uint32_t scale = (w.scale >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
    const float weight = d * (1.0f + 2.0f * (float)scale);
    const uint32_t ninth = (w.ninth >> (8 * (j & 1))) & 0xFF;
    uint32_t cb[2], sg[1], p[16];
    align_span(w.cb, cb);
    align_span(w.sg, sg);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t code = ((cb[k >> 2] >> (8 * (k & 3))) & 0xFF) | (((ninth >> k) & 1) << 8);
        const uint2 m = tab[code];
        // Sign bit t of elements 4 k + t to bit 7 of byte t, then to bits 15 and 31 of the pairs.
        const uint32_t spread = ((((sg[0] >> (4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u) << 7;
        p[2 * k] = m.x ^ __builtin_amdgcn_perm(0u, spread, 0x010C000Cu);
        p[2 * k + 1] = m.y ^ __builtin_amdgcn_perm(0u, spread, 0x030C020Cu);
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
        if (m0 + i >= args.m) break;
        const u32x4 *ap = (const u32x4 *)(args.a + (m0 + i) * args.lda + (int64_t)g * 32);
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 x = ap[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) s = gdot2(x[e], p[4 * q + e], s);
        }
        acc[i] = __builtin_fmaf(weight, s, acc[i]);
    }
}

// IQ4_NL / IQ4_XS group (GgufQuant.swift:179-185, 261-275): `tab[b]` holds the table values of
// both nibbles of a code byte b as a bf16 pair (the values are integers below 128 in magnitude:
// exact), for elements 4 q + e (low nibble) and 16 + 4 q + e (high nibble) of byte e of word q;
// one byte permute pairs the activations the same way, and the group's scale multiplies the
// v_dot2 sum once.
template <int MR>
__device__ __forceinline__ void iq4_dot(const uint32_t (&h)[4], float scale, const uint32_t *tab,
                                        const GgufNativeArgs &args, int64_t m0, int g, float (&acc)[MR]) {
    uint32_t w[16];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * q + e] = tab[(h[q] >> (8 * e)) & 0xFFu];
#pragma unroll
    for (int i = 0; i < MR; ++i) {
        if (m0 + i >= args.m) break;
        const u32x4 *ap = (const u32x4 *)(args.a + (m0 + i) * args.lda + (int64_t)g * 32);
        uint32_t x[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = ap[q];
            x[4 * q] = v[0], x[4 * q + 1] = v[1], x[4 * q + 2] = v[2], x[4 * q + 3] = v[3];
        }
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // Elements 4 q + e and 16 + 4 q + e: the low (e even) or high halves of activation
                // dwords 2 q + e / 2 and 8 + 2 q + e / 2.
                const int dw = 2 * q + (e >> 1);
                const uint32_t pair =
                    __builtin_amdgcn_perm(x[8 + dw], x[dw], (e & 1) ? 0x07060302u : 0x05040100u);
                s = gdot2(pair, w[4 * q + e], s);
            }
        acc[i] = __builtin_fmaf(scale, s, acc[i]);
    }
}

template <int TYPE, int MR>
__global__ void __launch_bounds__(256) gguf_gemv_kernel(GgufNativeArgs args) {
    // Lookup tables in LDS, built before any wave leaves: IQ3_S's codebook as bf16 magnitude
    // pairs (512 x 8 bytes), the IQ4 values of both nibbles of a byte as a bf16 pair (256 x 4).
    constexpr bool kIq4 = TYPE == 20 || TYPE == 23;
    __shared__ __align__(8) uint32_t lut[TYPE == 21 ? 1024 : kIq4 ? 256 : 1];
    uint2 *iq3s_tab = (uint2 *)lut;
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
            iq3s_tab[c] = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
        __syncthreads();
    }
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)xcd_block(blockIdx.x, gridDim.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (n >= args.rows) return;
    const int64_t m0 = (int64_t)blockIdx.y * MR;
    const int groups = (int)(args.inner / 32);
    const rsrc_t r = make_rsrc(args.w, args.w_bytes);
    const uint32_t row = (uint32_t)(n * args.row_bytes);
    float acc[MR];
#pragma unroll
    for (int i = 0; i < MR; ++i) acc[i] = 0.0f;
    // Two groups an iteration (the second 64 groups on), both decoded before either is used so
    // that their loads are in flight together; the groups left over one at a time.
    auto accumulate = [&](int g, const float (&v)[32]) {
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            if (m0 + i >= args.m) break;
            const u32x4 *ap = (const u32x4 *)(args.a + (m0 + i) * args.lda + (int64_t)g * 32);
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
        if constexpr (TYPE == 14) {
            q6k_dot<MR>(gguf_fetch<14>(r, row, g), args, m0, g, acc);
        } else if constexpr (TYPE == 11) {
            q3k_dot<MR>(gguf_fetch<11>(r, row, g), args, m0, g, acc);
        } else if constexpr (TYPE == 21) {
            iq3s_dot<MR>(gguf_fetch<21>(r, row, g), iq3s_tab, args, m0, g, acc);
        } else if constexpr (TYPE == 20) {
            const GgufRaw<20> w = gguf_fetch<20>(r, row, g);
            uint32_t h[4];
            align_span(w.codes, h);
            iq4_dot<MR>(h, half_bits_to_f32(w.d), lut, args, m0, g, acc);
        } else if constexpr (TYPE == 23) {
            const GgufRaw<23> w = gguf_fetch<23>(r, row, g);
            const int j = w.j;
            const uint32_t low = (w.lowb >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
            const uint32_t scale = low | (((w.high >> (2 * j)) & 3) << 4);
            const uint32_t h[4] = {w.q[0], w.q[1], w.q[2], w.q[3]};
            iq4_dot<MR>(h, half_bits_to_f32(w.d) * ((float)scale - 32.0f), lut, args, m0, g, acc);
        } else {
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
    switch (type) {
        case 8: *elems = 32; *bytes = 34; return 1;
        case 20: *elems = 32; *bytes = 18; return 1;
        case 14: *elems = 256; *bytes = 210; return 1;
        case 23: *elems = 256; *bytes = 136; return 1;
        case 11: *elems = 256; *bytes = 110; return 1;
        case 21: *elems = 256; *bytes = 110; return 1;
        default: return 0;
    }
}

static void fill_args(GgufNativeArgs &args, int type, const uint8_t *w, int64_t rows, int64_t inner) {
    int elems = 0, bytes = 0;
    gguf_native_block(type, &elems, &bytes);
    args.w = w;
    args.rows = rows;
    args.inner = inner;
    args.row_bytes = (uint32_t)(inner / elems * bytes);
    args.w_bytes = (uint32_t)(rows * (int64_t)args.row_bytes);
}

hipError_t launch_gguf_dequant(int type, const uint8_t *w, int64_t rows, int64_t inner, float *dense,
                               hipStream_t stream) {
    GgufNativeArgs args = {};
    fill_args(args, type, w, rows, inner);
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
    fill_args(args, type, w, rows, inner);
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

template <int MR>
static void launch_gemv_mr(int type, const GgufNativeArgs &args, hipStream_t stream) {
    const dim3 grid((unsigned)((args.rows + 3) / 4), (unsigned)((args.m + MR - 1) / MR));
    switch (type) {
        case 8: hipLaunchKernelGGL((gguf_gemv_kernel<8, MR>), grid, dim3(256), 0, stream, args); break;
        case 20: hipLaunchKernelGGL((gguf_gemv_kernel<20, MR>), grid, dim3(256), 0, stream, args); break;
        case 14: hipLaunchKernelGGL((gguf_gemv_kernel<14, MR>), grid, dim3(256), 0, stream, args); break;
        case 11: hipLaunchKernelGGL((gguf_gemv_kernel<11, MR>), grid, dim3(256), 0, stream, args); break;
        case 21: hipLaunchKernelGGL((gguf_gemv_kernel<21, MR>), grid, dim3(256), 0, stream, args); break;
        default: hipLaunchKernelGGL((gguf_gemv_kernel<23, MR>), grid, dim3(256), 0, stream, args); break;
    }
}

// Activation rows a pass over the weight: four up to four rows, eight above (one pass up to
// eight rows instead of two).
hipError_t launch_gguf_gemv(int type, const uint8_t *w, int64_t rows, int64_t inner, const uint16_t *a, int64_t lda,
                            void *out, int64_t ldc, int out_dtype, const void *residual, int64_t m,
                            hipStream_t stream) {
    GgufNativeArgs args = {};
    fill_args(args, type, w, rows, inner);
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
