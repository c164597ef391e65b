// q5k.hip -- GGUF Q5_K on the device: the plane repack/unpack, the bit-exact fp32 decoder and the
// weight-streaming GEMM.
//
// Q5_K (Model/GgufQuant.swift:191-212): a 256-element block of 176 bytes holds fp16 d and dmin,
// twelve bytes of eight 6-bit scales and minimums, 32 bytes of fifth bits and 128 bytes of low
// nibbles; w = code * (d * sc_j) - dmin * mn_j for element e of group j, code = nibble + 16 * bit.
// The kernels read the GgufPlanes form (Model/GgufPlanes.swift:8-20): per (row, 32-group) a
// 16-byte plane0 record of nibbles in chunk order and a 4-byte plane1 record of fifth bits, and per
// (row, block) the block's first 16 bytes as meta, all tiled by 128 rows. Q4_K (decodeQ45K with
// fifthBit false, GgufQuant.swift:44,151,191-212: 144-byte blocks without the fifth bits;
// GgufPlanes.swift:64: no plane1) runs through the same kernels with a null plane1.
//
// Chunk order (gguf_formats.h:17-21): word c of a plane0 record holds elements 4c..4c+3 and
// 16+4c..16+4c+3; pair p of the word (bits 4p and 16 + 4p) is elements e0, e0 + 1 with
// e0 = 16 (p >> 1) + 4c + 2 (p & 1), slot 8c + 2p (+1). So (w >> 4p) & 0x000F000F is already a
// pair of consecutive elements in two 16-bit lanes: the MFMA operand needs no permutation.
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

constexpr int kQ5BlockBytes = 176;
constexpr int kQ4KBlockBytes = 144;  // Q4_K: the same block without the 32 bytes of fifth bits

// GgufPlanes.slot (Model/GgufPlanes.swift:93-95).
__device__ __forceinline__ int gguf_slot(int e) { return 8 * ((e >> 2) & 3) + 4 * (e >> 4) + (e & 3); }

__device__ __forceinline__ int64_t plane_record(int64_t row, int64_t block, int64_t blocks) {
    return ((row >> 7) * blocks + block) * kTileRows + (row & (kTileRows - 1));
}

// The 6-bit scale and minimum of group j from the twelve packed bytes (GgufQuant.swift:196-203).
__device__ __forceinline__ void q5k_scale_min(const uint8_t *packed, int j, uint32_t *sc, uint32_t *mn) {
    if (j < 4) {
        *sc = packed[j] & 63u;
        *mn = packed[j + 4] & 63u;
    } else {
        *sc = (packed[j + 4] & 0xfu) | ((uint32_t)(packed[j - 4] >> 6) << 4);
        *mn = (uint32_t)(packed[j + 4] >> 4) | ((uint32_t)(packed[j] >> 6) << 4);
    }
}

// ---- repack / unpack: a workgroup per (32 rows, native block) ------------------------------------
//
// The 32 rows' blocks are copied between memory and LDS with consecutive lanes on consecutive dwords
// of a block; thread (j, row) = (tid / 32, tid % 32) then builds (or takes apart) the plane record
// of group j, so that a wave's plane stores (or loads) are runs of 32 consecutive 16-byte records.
constexpr int kRepackRows = 32;

__global__ void __launch_bounds__(256)
q5k_repack_kernel(const uint8_t *__restrict__ native, int64_t rows, int64_t inner, uint8_t *__restrict__ p0,
                  uint8_t *__restrict__ p1, uint8_t *__restrict__ meta, int fifth) {
    __shared__ uint32_t blk[kRepackRows * kQ5BlockBytes / 4];
    const int64_t blocks = inner / 256, groups = inner / 32;
    const int64_t r0 = (int64_t)blockIdx.x * kRepackRows, block = blockIdx.y;
    const int bytes = fifth ? kQ5BlockBytes : kQ4KBlockBytes, qs = fifth ? 48 : 16, words = bytes / 4;
    const int tid = threadIdx.x;
    for (int d = tid; d < kRepackRows * words; d += 256) {
        const int64_t row = r0 + d / words;
        if (row < rows) blk[d] = *(const uint32_t *)(native + (row * blocks + block) * bytes + 4 * (d % words));
    }
    __syncthreads();
    const int j = tid / kRepackRows, lr = tid % kRepackRows;
    const int64_t row = r0 + lr;
    if (row >= rows) return;
    const uint8_t *b = (const uint8_t *)blk + lr * bytes;
    uint32_t w[4] = {0u, 0u, 0u, 0u}, bits = 0u;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const int slot = gguf_slot(e), i = slot & 7;
        const uint32_t low = (b[qs + 32 * (j / 2) + e] >> (4 * (j % 2))) & 15u;
        w[slot >> 3] |= low << ((i & 1) * 16 + 4 * (i >> 1));
        if (fifth) bits |= ((b[16 + e] >> j) & 1u) << slot;
    }
    const int64_t rec = plane_record(row, block * 8 + j, groups);
    *(u32x4 *)(p0 + rec * 16) = u32x4{w[0], w[1], w[2], w[3]};
    if (fifth) *(uint32_t *)(p1 + rec * 4) = bits;
    if (j == 0) {
        const uint32_t *m = blk + lr * words;
        *(u32x4 *)(meta + plane_record(row, block, blocks) * 16) = u32x4{m[0], m[1], m[2], m[3]};
    }
}

__global__ void __launch_bounds__(256)
q5k_unpack_kernel(const uint8_t *__restrict__ p0, const uint8_t *__restrict__ p1, const uint8_t *__restrict__ meta,
                  int64_t rows, int64_t inner, uint8_t *__restrict__ native, int fifth) {
    // The 5-bit codes of the 32 rows' blocks ([row][element 0..255]), then the block bytes.
    __shared__ uint8_t codes[kRepackRows * 256];
    __shared__ u32x4 metas[kRepackRows];
    const int64_t blocks = inner / 256, groups = inner / 32;
    const int64_t r0 = (int64_t)blockIdx.x * kRepackRows, block = blockIdx.y;
    const int bytes = fifth ? kQ5BlockBytes : kQ4KBlockBytes, qs = fifth ? 48 : 16, words = bytes / 4;
    const int tid = threadIdx.x;
    {
        const int j = tid / kRepackRows, lr = tid % kRepackRows;
        const int64_t row = r0 + lr;
        if (row < rows) {
            const int64_t rec = plane_record(row, block * 8 + j, groups);
            const u32x4 w = *(const u32x4 *)(p0 + rec * 16);
            const uint32_t bits = fifth ? *(const uint32_t *)(p1 + rec * 4) : 0u;
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const int slot = gguf_slot(e), i = slot & 7;
                const uint32_t low = (w[slot >> 3] >> ((i & 1) * 16 + 4 * (i >> 1))) & 15u;
                codes[lr * 256 + 32 * j + e] = (uint8_t)(low | (((bits >> slot) & 1u) << 4));
            }
            if (j == 0) metas[lr] = *(const u32x4 *)(meta + plane_record(row, block, blocks) * 16);
        }
    }
    __syncthreads();
    for (int d = tid; d < kRepackRows * words; d += 256) {
        const int lr = d / words, o = 4 * (d % words);
        const int64_t row = r0 + lr;
        if (row >= rows) continue;
        const uint8_t *c = codes + lr * 256;
        uint32_t v = 0u;
        for (int k = 0; k < 4; ++k) {
            const int at = o + k;
            uint32_t byte;
            if (at < 16) {
                byte = (metas[lr][at >> 2] >> (8 * (at & 3))) & 0xFFu;
            } else if (at < qs) {  // fifth bits: bit j of byte 16 + e is element e of group j
                const int e = at - 16;
                byte = 0u;
                for (int j = 0; j < 8; ++j) byte |= (uint32_t)(c[32 * j + e] >> 4) << j;
            } else {  // low nibble: group 2 q, high nibble: group 2 q + 1
                const int q = (at - qs) / 32, e = (at - qs) % 32;
                byte = (c[64 * q + e] & 15u) | ((uint32_t)(c[64 * q + 32 + e] & 15u) << 4);
            }
            v |= byte << (8 * k);
        }
        *(uint32_t *)(native + (row * blocks + block) * bytes + o) = v;
    }
}

hipError_t launch_q5k_repack(const uint8_t *native, int64_t rows, int64_t inner, uint8_t *p0, uint8_t *p1,
                             uint8_t *meta, bool inverse, hipStream_t stream, bool fifth) {
    const dim3 grid((unsigned)((rows + kRepackRows - 1) / kRepackRows), (unsigned)(inner / 256));
    if (inverse)
        hipLaunchKernelGGL(q5k_unpack_kernel, grid, dim3(256), 0, stream, p0, p1, meta, rows, inner,
                           const_cast<uint8_t *>(native), fifth ? 1 : 0);
    else
        hipLaunchKernelGGL(q5k_repack_kernel, grid, dim3(256), 0, stream, native, rows, inner, p0, p1, meta,
                           fifth ? 1 : 0);
    return hipGetLastError();
}

// ---- bit-exact decode: one thread per (row, 32-group) -------------------------------------------

// w = code * (d * sc) - dmin * mn. d * sc and dmin * mn are exact in fp32 (11-bit times 6-bit
// integers) and so is code * (d * sc) (<= 22 bits), so the subtraction is the one rounding and an
// FMA gives the same bits as the reference's separate multiply and subtract.
__device__ __forceinline__ void q5k_group_coefficients(const uint8_t *m, int j, float *scaled, float *offset) {
    const float d = half_bits_to_f32((uint32_t)m[0] | ((uint32_t)m[1] << 8));
    const float dmin = half_bits_to_f32((uint32_t)m[2] | ((uint32_t)m[3] << 8));
    uint32_t sc, mn;
    q5k_scale_min(m + 4, j, &sc, &mn);
    *scaled = d * (float)sc;
    *offset = dmin * (float)mn;
}

__global__ void __launch_bounds__(256)
q5k_dequant_kernel(splosh_q5k_weight w, float *__restrict__ out) {
    const int64_t groups = w.inner / 32, blocks = w.inner / 256;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= w.rows * groups) return;
    const int64_t row = idx / groups, g = idx % groups;
    const int64_t rec = plane_record(row, g, groups);
    const u32x4 words = *(const u32x4 *)(w.plane0 + rec * 16);
    const uint32_t bits = w.plane1 ? *(const uint32_t *)(w.plane1 + rec * 4) : 0u;  // null: Q4_K
    uint8_t m[16];
    const int64_t mrec = plane_record(row, g / 8, blocks);
    for (int i = 0; i < 16; ++i) m[i] = w.meta[mrec * 16 + i];
    float scaled, offset;
    q5k_group_coefficients(m, (int)(g % 8), &scaled, &offset);
    float *dst = out + row * w.inner + g * 32;
    for (int e = 0; e < 32; ++e) {
        const int slot = gguf_slot(e);
        const int i = slot & 7;
        const uint32_t code = ((words[slot >> 3] >> ((i & 1) * 16 + 4 * (i >> 1))) & 15u) | (((bits >> slot) & 1u) << 4);
        const float p = (float)code * scaled;
        dst[e] = p - offset;
    }
}

// sp_gguf_embed (engine_gguf.metal:302-318) on Q5_K / Q4_K planes: out[i] = decode(row tokens[i]),
// one thread a group of 32 of one token; fp32 (bit-identical to the decoder) or bf16 (RNE). An id
// past the table gives zeros.
__global__ void __launch_bounds__(256)
q5k_embed_kernel(splosh_q5k_weight w, const uint32_t *__restrict__ tokens, int64_t count, void *__restrict__ out,
                 int64_t ldo, int out_dtype) {
    const int64_t groups = w.inner / 32, blocks = w.inner / 256;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= count * groups) return;
    const int64_t i = idx / groups, g = idx % groups;
    const int64_t row = tokens[i];
    float v[32];
    if (row >= w.rows) {
        for (int e = 0; e < 32; ++e) v[e] = 0.0f;
    } else {
        const int64_t rec = plane_record(row, g, groups);
        const u32x4 words = *(const u32x4 *)(w.plane0 + rec * 16);
        const uint32_t bits = w.plane1 ? *(const uint32_t *)(w.plane1 + rec * 4) : 0u;  // null: Q4_K
        uint8_t m[16];
        const int64_t mrec = plane_record(row, g / 8, blocks);
        for (int k = 0; k < 16; ++k) m[k] = w.meta[mrec * 16 + k];
        float scaled, offset;
        q5k_group_coefficients(m, (int)(g % 8), &scaled, &offset);
        for (int e = 0; e < 32; ++e) {
            const int slot = gguf_slot(e);
            const int k = slot & 7;
            const uint32_t code = ((words[slot >> 3] >> ((k & 1) * 16 + 4 * (k >> 1))) & 15u) | (((bits >> slot) & 1u) << 4);
            const float p = (float)code * scaled;
            v[e] = p - offset;
        }
    }
    if (out_dtype == SPLOSH_F32) {
        float *dst = (float *)out + i * ldo + g * 32;
        for (int e = 0; e < 32; ++e) dst[e] = v[e];
    } else {
        uint16_t *dst = (uint16_t *)out + i * ldo + g * 32;
        for (int e = 0; e < 32; ++e) dst[e] = f32_to_bf16(v[e]);
    }
}

hipError_t launch_q5k_embed(const splosh_q5k_weight &w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                            int out_dtype, hipStream_t stream) {
    const int64_t total = count * (w.inner / 32);
    hipLaunchKernelGGL(q5k_embed_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, w, tokens, count,
                       out, ldo, out_dtype);
    return hipGetLastError();
}

hipError_t launch_q5k_dequant(const splosh_q5k_weight &w, float *out, hipStream_t stream) {
    const int64_t total = w.rows * (w.inner / 32);
    hipLaunchKernelGGL(q5k_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, w, out);
    return hipGetLastError();
}

// ---- scalar GEMM (odd shapes) -------------------------------------------------------------------

__global__ void __launch_bounds__(256)
q5k_gemm_scalar_kernel(splosh_q5k_weight w, const uint16_t *__restrict__ a, int64_t lda, void *out, int64_t ldc,
                       int out_dtype, const void *residual, int64_t rows) {
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t mrow = blockIdx.y;
    if (n >= w.rows || mrow >= rows) return;
    const int64_t groups = w.inner / 32, blocks = w.inner / 256;
    const uint16_t *ar = a + mrow * lda;
    float sum = 0.0f;
    for (int64_t g = 0; g < groups; ++g) {
        const int64_t rec = plane_record(n, g, groups);
        const u32x4 words = *(const u32x4 *)(w.plane0 + rec * 16);
        const uint32_t bits = w.plane1 ? *(const uint32_t *)(w.plane1 + rec * 4) : 0u;  // null: Q4_K
        uint8_t m[16];
        const int64_t mrec = plane_record(n, g / 8, blocks);
        for (int i = 0; i < 16; ++i) m[i] = w.meta[mrec * 16 + i];
        float scaled, offset;
        q5k_group_coefficients(m, (int)(g % 8), &scaled, &offset);
        for (int e = 0; e < 32; ++e) {
            const int slot = gguf_slot(e);
            const int i = slot & 7;
            const uint32_t code = ((words[slot >> 3] >> ((i & 1) * 16 + 4 * (i >> 1))) & 15u) | (((bits >> slot) & 1u) << 4);
            const float weight = (float)code * scaled - offset;
            sum += bf16_bits_to_f32(ar[g * 32 + e]) * weight;
        }
    }
    const int64_t index = mrow * ldc + n;
    if (out_dtype == SPLOSH_F32) {
        if (residual) sum += ((const float *)residual)[index];
        ((float *)out)[index] = sum;
    } else {
        if (residual) sum += bf16_bits_to_f32(((const uint16_t *)residual)[index]);
        ((uint16_t *)out)[index] = f32_to_bf16(sum);
    }
}

hipError_t launch_q5k_gemm_scalar(const splosh_q5k_weight &w, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                                  int out_dtype, const void *residual, int64_t rows, hipStream_t stream) {
    dim3 grid((unsigned)((w.rows + 255) / 256), (unsigned)rows);
    hipLaunchKernelGGL(q5k_gemm_scalar_kernel, grid, dim3(256), 0, stream, w, a, lda, out, ldc, out_dtype, residual, rows);
    return hipGetLastError();
}

// ---- weight-streaming GEMM ---------------------------------------------------------------------
//
// Same scheme as the q4 streaming kernel (stream.hip): codes become bf16 128 + code, one
// v_mfma_f32_16x16x32_bf16 per 32-group and 16x16 block gives P = 128 S + sum(a code), a second
// against ones gives S = sum(a), and acc += s P - (128 s + mn) S with s = d sc, mn = dmin min.
// The fifth bit goes to bit 4 of each 16-bit lane: a 2-bit field t of plane1 times 0x00080010,
// masked with 0x00100010, puts bit 0 of t at bit 4 and bit 1 at bit 20.

struct Q5StreamArgs {
    splosh_q5k_weight w;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
};

__device__ __forceinline__ bf16x8 q5k_codes_operand(uint32_t w, uint32_t hc) {
    u32x4 d;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t t = __builtin_amdgcn_ubfe(hc, 2 * p, 2);
        const uint32_t high = ((t * 0x00080010u) & 0x00100010u) | 0x43004300u;
        d[p] = ((w >> (4 * p)) & 0x000F000Fu) | high;
    }
    return as_bf16x8(d);
}

template <int MB, int J, int RPL>
__global__ void __launch_bounds__(512)
q5k_stream_kernel(Q5StreamArgs args) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sk = blockDim.x / kWave;
    const int r = lane & 15, c = lane >> 4;
    const int64_t n_total = args.w.rows;
    const int64_t n0 = (int64_t)blockIdx.x * 16 * J;
    const int64_t m0 = (int64_t)blockIdx.y * 16 * MB;
    const int64_t groups = args.w.inner / 32, blocks = args.w.inner / 256;
    const int64_t b0 = blocks * wave / sk, b1 = blocks * (wave + 1) / sk;

    int64_t col[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t n = n0 + 16 * j + r;
        col[j] = n < n_total ? n : n_total - 1;
    }
    const uint16_t *arow[MB];
    bool mvalid[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int64_t m = m0 + 16 * mb + r;
        mvalid[mb] = m < args.rows;
        arow[mb] = args.a + (mvalid[mb] ? m : 0) * args.lda + 4 * c;
    }
    float acc[J][MB][RPL];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < RPL; ++i) acc[j][mb][i] = 0.0f;

    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

    struct Stage {
        u32x4 meta[J];
        uint32_t w[8][J];
        uint32_t h[8][J];
    };
    auto load_block = [&](Stage &st, int64_t blk) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            st.meta[j] = *(const u32x4 *)(args.w.meta + plane_record(col[j], blk, blocks) * 16);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int64_t rec = plane_record(col[j], blk * 8 + jj, groups);
                st.w[jj][j] = *(const uint32_t *)(args.w.plane0 + rec * 16 + 4 * c);
                st.h[jj][j] = args.w.plane1 ? *(const uint32_t *)(args.w.plane1 + rec * 4) : 0u;  // null: Q4_K
            }
        }
    };
    auto use_block = [&](const Stage &st, int64_t blk) {
        float d[J], dmin[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            d[j] = half_bits_to_f32(st.meta[j].x);
            dmin[j] = half_bits_to_f32(st.meta[j].x >> 16);
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int64_t g = blk * 8 + jj;
            bf16x8 av[MB];
            f32x4 sx[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                u32x2 lo = {0u, 0u}, hi = {0u, 0u};
                if (mvalid[mb]) {
                    lo = *(const u32x2 *)(arow[mb] + g * 32);
                    hi = *(const u32x2 *)(arow[mb] + g * 32 + 16);
                }
                av[mb] = __builtin_bit_cast(bf16x8, u32x4{lo.x, lo.y, hi.x, hi.y});
                sx[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mb], ones, zero, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < J; ++j) {
                // 6-bit scale and minimum of group jj from meta bytes 4..15 (GgufQuant.swift:196-203).
                const uint32_t p03 = st.meta[j].y, p47 = st.meta[j].z, p811 = st.meta[j].w;
                uint32_t sc, mn;
                if (jj < 4) {
                    sc = (p03 >> (8 * jj)) & 63u;
                    mn = (p47 >> (8 * jj)) & 63u;
                } else {
                    const int t = jj - 4;
                    sc = ((p811 >> (8 * t)) & 0xfu) | (((p03 >> (8 * t + 6)) & 3u) << 4);
                    mn = ((p811 >> (8 * t + 4)) & 0xfu) | (((p47 >> (8 * t + 6)) & 3u) << 4);
                }
                const float s = d[j] * (float)sc;
                const float off = __builtin_fmaf(128.0f, s, dmin[j] * (float)mn);
                const bf16x8 bq = q5k_codes_operand(st.w[jj][j], st.h[jj][j] >> (8 * c));
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mb], bq, zero, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < RPL; ++i)
                        acc[j][mb][i] = __builtin_fmaf(s, p[i], __builtin_fmaf(-off, sx[mb][i], acc[j][mb][i]));
                }
            }
        }
    };

    Stage st0, st1;
    if (b0 < b1) load_block(st0, b0);
    for (int64_t blk = b0; blk < b1; blk += 2) {
        if (blk + 1 < b1) load_block(st1, blk + 1);
        use_block(st0, blk);
        if (blk + 1 >= b1) break;
        if (blk + 2 < b1) load_block(st0, blk + 2);
        use_block(st1, blk + 1);
    }

    constexpr int kPerWave = J * MB * RPL * kWave;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < RPL; ++i) red[wave * kPerWave + ((j * MB + mb) * RPL + i) * kWave + lane] = acc[j][mb][i];
    __syncthreads();
    for (int e = threadIdx.x; e < kPerWave; e += blockDim.x) {
        float v = 0.0f;
        for (int s = 0; s < sk; ++s) v += red[s * kPerWave + e];
        const int ln = e % kWave;
        const int i = (e / kWave) % RPL;
        const int mb = (e / (kWave * RPL)) % MB;
        const int j = e / (kWave * RPL * MB);
        const int64_t m = m0 + 16 * mb + 4 * (ln >> 4) + i;
        const int64_t n = n0 + 16 * j + (ln & 15);
        if (m < args.rows && n < n_total) {
            const int64_t index = m * args.ldc + n;
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) v += ((const float *)args.residual)[index];
                ((float *)args.out)[index] = v;
            } else {
                if (args.residual) v += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                ((uint16_t *)args.out)[index] = f32_to_bf16(v);
            }
        }
    }
}

template <int MB, int J, int RPL>
static hipError_t launch_q5k_variant(const StreamPlan &plan, const Q5StreamArgs &args, hipStream_t stream) {
    dim3 grid((unsigned)plan.col_blocks, (unsigned)plan.row_chunks);
    dim3 block((unsigned)(plan.sk * kWave));
    const size_t lds = (size_t)plan.sk * J * MB * RPL * kWave * sizeof(float);
    hipLaunchKernelGGL((q5k_stream_kernel<MB, J, RPL>), grid, block, lds, stream, args);
    return hipGetLastError();
}

hipError_t launch_q5k_stream(const StreamPlan &p, const splosh_q5k_weight &w, const uint16_t *a, int64_t lda,
                             void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                             hipStream_t stream) {
    Q5StreamArgs args{w, a, lda, out, ldc, residual, rows, out_dtype};
#define SPLOSH_Q5_CASE(MB_, J_, RPL_) \
    if (p.mb == MB_ && p.j == J_ && p.rpl == RPL_) return launch_q5k_variant<MB_, J_, RPL_>(p, args, stream);
    SPLOSH_Q5_CASE(1, 2, 1) SPLOSH_Q5_CASE(1, 1, 1)
    SPLOSH_Q5_CASE(1, 2, 2) SPLOSH_Q5_CASE(1, 1, 2)
    SPLOSH_Q5_CASE(1, 2, 4) SPLOSH_Q5_CASE(1, 1, 4)
    SPLOSH_Q5_CASE(2, 2, 4) SPLOSH_Q5_CASE(2, 1, 4)
    SPLOSH_Q5_CASE(4, 2, 4) SPLOSH_Q5_CASE(4, 1, 4)
#undef SPLOSH_Q5_CASE
    return hipErrorInvalidValue;
}

}  // namespace splosh
