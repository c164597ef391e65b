// gguf_native.hip -- GGUF Q8_0, Q6_K, IQ4_NL and IQ4_XS weights read in their native blocks.
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
//    rows (fp32). The wave's partial sums meet in a shuffle tree. Rows beyond MR take further
//    passes over the weight (grid.y).
//
// Blocks are 2-byte aligned at best (Q8_0: 34 bytes, Q6_K: 210): a run of bytes is read as the
// dword-aligned window that covers it, in 16-byte loads, and shifted into place per lane.
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

// IQ4_NL / IQ4_XS code values (llama.cpp's kvalues_iq4nl, the format's table: -127, -104, -83,
// -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113) as int8 bytes, four to a dword.
constexpr uint32_t kIq4Tab0 = 0xBFAD9881u, kIq4Tab1 = 0xF6EADDCFu, kIq4Tab2 = 0x26190D01u, kIq4Tab3 = 0x71594535u;

// Table values (int8) of the four 4-bit codes in the bytes of `idx`: entries 0..7 and 8..15 by two
// byte permutes, then per byte the half that bit 3 of the code picks.
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t idx) {
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = perm_bytes(kIq4Tab1, kIq4Tab0, sel), hi = perm_bytes(kIq4Tab3, kIq4Tab2, sel);
    const uint32_t mask = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (hi & mask) | (lo & ~mask);
}

template <int TYPE>
struct GgufGeom;
template <> struct GgufGeom<8> { static constexpr int kElems = 32, kBytes = 34; };    // Q8_0
template <> struct GgufGeom<20> { static constexpr int kElems = 32, kBytes = 18; };   // IQ4_NL
template <> struct GgufGeom<14> { static constexpr int kElems = 256, kBytes = 210; }; // Q6_K
template <> struct GgufGeom<23> { static constexpr int kElems = 256, kBytes = 136; }; // IQ4_XS

__device__ __forceinline__ uint32_t ld16(rsrc_t r, uint32_t off) { return buffer_load_u16(r, off, 0); }

// W dwords of bytes starting at a 2-aligned `off` (all 4 W of them inside the weight): the dword-aligned window that covers them (W + 1
// dwords, the first in 16-byte pieces; buffer loads need only dword alignment) shifted into place
// by the lane's 0- or 2-byte misalignment (v_alignbyte_b32). Every byte read lies in the weight.
template <int W>
__device__ __forceinline__ void load_span(rsrc_t r, uint32_t off, uint32_t (&out)[W]) {
    const uint32_t a0 = off & ~3u, sh = off & 3u;
    uint32_t win[W + 1];
#pragma unroll
    for (int q = 0; q < (W + 1) / 4; ++q) {
        const u32x4 x = buffer_load16(r, a0 + 16u * q, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) win[4 * q + e] = x[e];
    }
#pragma unroll
    for (int e = (W + 1) / 4 * 4; e < W; ++e) win[e] = buffer_load_u32(r, a0 + 4u * e, 0);
    // Only the low half of the last window dword is ever used (when off is 2 mod 4), and its high
    // half may lie past the weight, where a dword load would read zero for the whole dword.
    win[W] = buffer_load_u16(r, a0 + 4u * W, 0);
#pragma unroll
    for (int i = 0; i < W; ++i) out[i] = __builtin_amdgcn_alignbyte(win[i + 1], win[i], sh);
}
template <int W>
__device__ __forceinline__ uint32_t byte_of(const uint32_t (&w)[W], int e) { return (w[e >> 2] >> (8 * (e & 3))) & 0xFF; }

// Group g of a row whose blocks start at byte `row` (GgufQuant.swift decode, fp32 op order).
template <int TYPE>
__device__ __forceinline__ void decode_group(rsrc_t r, uint32_t row, int g, float (&v)[32]) {
    if constexpr (TYPE == 8) {  // Q8_0 (GgufQuant.swift:172-175)
        const uint32_t b = row + (uint32_t)g * 34u;
        const float d = half_bits_to_f32(ld16(r, b));
        uint32_t h[8];   // the 32 codes
        load_span<8>(r, b + 2, h);
#pragma unroll
        for (int e = 0; e < 32; ++e) v[e] = d * (float)(int8_t)byte_of(h, e);
    } else if constexpr (TYPE == 20) {  // IQ4_NL (:179-185)
        const uint32_t b = row + (uint32_t)g * 18u;
        const float d = half_bits_to_f32(ld16(r, b));
        uint32_t h[4];   // 16 bytes of two codes
        load_span<4>(r, b + 2, h);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t lo = iq4_lookup4(h[q] & 0x0F0F0F0Fu), hi = iq4_lookup4((h[q] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[4 * q + e] = d * (float)(int8_t)((lo >> (8 * e)) & 0xFF);
                v[16 + 4 * q + e] = d * (float)(int8_t)((hi >> (8 * e)) & 0xFF);
            }
        }
    } else if constexpr (TYPE == 14) {  // Q6_K (:218-230): ql[128], qh[64], scales[16], d
        const int j = g & 7, half = j >> 2, quarter = j & 3;
        const uint32_t b = row + (uint32_t)(g >> 3) * 210u;
        const float d = half_bits_to_f32(ld16(r, b + 208));
        const uint32_t sc = ld16(r, b + 192 + 2 * j);
        const float ds0 = d * (float)(int8_t)(sc & 0xFF), ds1 = d * (float)(int8_t)(sc >> 8);
        uint32_t ql[8], qh[8];
        load_span<8>(r, b + 64 * half + 32 * (quarter & 1), ql);
        load_span<8>(r, b + 128 + 32 * half, qh);
        const int lsh = 4 * (quarter >> 1), hsh = 2 * quarter;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const uint32_t low = (byte_of(ql, e) >> lsh) & 15, high = (byte_of(qh, e) >> hsh) & 3;
            const float code = (float)(low | (high << 4)) - 32.0f;
            v[e] = (e < 16 ? ds0 : ds1) * code;
        }
    } else {  // IQ4_XS (:261-275): d, scales_h, scales_l[4], qs[128]
        const int j = g & 7;
        const uint32_t b = row + (uint32_t)(g >> 3) * 136u;
        const float d = half_bits_to_f32(ld16(r, b));
        const uint32_t high = ld16(r, b + 2);
        const uint32_t lowb = ld16(r, b + 4 + 2 * (j >> 2));   // bytes 4 + 2 (j / 4) .. + 1
        const uint32_t low = (lowb >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
        const uint32_t scale = low | (((high >> (2 * j)) & 3) << 4);
        const float scaled = d * ((float)scale - 32.0f);
        const u32x4 q = buffer_load16(r, b + 8 + 16 * j, 0);   // blocks of 136 bytes: 8-aligned runs
        const uint32_t qs[4] = {q[0], q[1], q[2], q[3]};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = iq4_lookup4(qs[k] & 0x0F0F0F0Fu), hi = iq4_lookup4((qs[k] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[4 * k + e] = scaled * (float)(int8_t)((lo >> (8 * e)) & 0xFF);
                v[16 + 4 * k + e] = scaled * (float)(int8_t)((hi >> (8 * e)) & 0xFF);
            }
        }
    }
}

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

template <int TYPE, int MR>
__global__ void __launch_bounds__(256) gguf_gemv_kernel(GgufNativeArgs args) {
    const int lane = threadIdx.x & 63;
    const int64_t n = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
        float v[32];
        decode_group<TYPE>(r, row, g, v);
        accumulate(g, v);
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
        default: hipLaunchKernelGGL(gguf_dequant_kernel<23>, grid, dim3(256), 0, stream, args); break;
    }
    return hipGetLastError();
}

constexpr int kGgufMR = 4;

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
    const dim3 grid((unsigned)((rows + 3) / 4), (unsigned)((m + kGgufMR - 1) / kGgufMR));
    switch (type) {
        case 8: hipLaunchKernelGGL((gguf_gemv_kernel<8, kGgufMR>), grid, dim3(256), 0, stream, args); break;
        case 20: hipLaunchKernelGGL((gguf_gemv_kernel<20, kGgufMR>), grid, dim3(256), 0, stream, args); break;
        case 14: hipLaunchKernelGGL((gguf_gemv_kernel<14, kGgufMR>), grid, dim3(256), 0, stream, args); break;
        default: hipLaunchKernelGGL((gguf_gemv_kernel<23, kGgufMR>), grid, dim3(256), 0, stream, args); break;
    }
    return hipGetLastError();
}

}  // namespace splosh
