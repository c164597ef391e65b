/*
 * splosh_oracle.c -- CPU restatement of the reference's quantized-matmul algorithms.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never shipped or measured as the
 * product. Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg only.
 * Built with -O2 -ffp-contract=off so that every product and sum is a separately rounded fp32
 * operation, as in the Swift reference (which does not contract a*b+c).
 *
 * Each function restates the reference file:line named beside it (ajaxharg/Splosh tree).
 */
#include "splosh_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- scalar conversions ------------------------------------------------------------------ */

static inline float bits_to_f32(uint32_t bits) {
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint32_t f32_to_bits(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    return bits;
}

/* Q4BufferLayout.bf16 (Q4BufferLayout.swift:123-125). */
float or_bf16_to_f32(uint16_t bits) { return bits_to_f32((uint32_t)bits << 16); }

/* Q4BufferLayout.bf16Bits (Q4BufferLayout.swift:127-129): (bits + 0x8000) >> 16. */
uint16_t or_f32_to_bf16_halfup(float value) {
    return (uint16_t)((f32_to_bits(value) + 0x8000u) >> 16);
}

/* IEEE round-to-nearest-even to bf16; NaN stays a quiet NaN. */
uint16_t or_f32_to_bf16_rne(float value) {
    uint32_t bits = f32_to_bits(value);
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu) != 0)
        return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}

void or_f32_to_bf16_rne_n(const float *src, uint16_t *dst, int64_t count) {
    for (int64_t i = 0; i < count; ++i) dst[i] = or_f32_to_bf16_rne(src[i]);
}

/* IEEE binary16 -> binary32, exact (the widening `Float(Float16(bitPattern:))` performs,
 * GgufQuant.swift:300-305 `half(at:)`). */
static float half_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t mantissa = h & 0x3ffu;
    if (exponent == 0x1fu) return bits_to_f32(sign | 0x7f800000u | (mantissa << 13));
    if (exponent == 0) {
        if (mantissa == 0) return bits_to_f32(sign);
        /* subnormal: mantissa * 2^-24, exact in fp32 */
        float v = (float)mantissa * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_to_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* ---- MLX affine q4 ------------------------------------------------------------------------ */

/* DequantOracle.dequantize (DequantOracle.swift:11-25) over the padded row-major buffer that
 * Q4BufferLayout addresses (wordIndex :82-90, nibbleShift :94-98, sidecarIndex :100-104). */
void or_q4_dequant_rowmajor(const uint32_t *words, int64_t stride_words, const uint16_t *scales,
                            const uint16_t *biases, int64_t N, int64_t K, float *out) {
    const int64_t groups = (K + 63) / 64;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            const uint32_t word = words[n * stride_words + k / 8];
            const float q = (float)((word >> (4 * (k % 8))) & 0xfu);
            const int64_t g = n * groups + k / 64;
            const float s = or_bf16_to_f32(scales[g]);
            const float b = or_bf16_to_f32(biases[g]);
            const float sq = s * q;
            out[n * K + k] = sq + b;
        }
    }
}

/* The tiled record of (row n, group g): ((n / 128) * groups + g) * 128 + n % 128, as
 * Converter.tile places it (Retile.swift:142-147). */
static inline int64_t tiled_record(int64_t n, int64_t g, int64_t groups) {
    return ((n / 128) * groups + g) * 128 + (n % 128);
}

void or_q4_dequant_tiled(const uint32_t *words, const uint16_t *scales, const uint16_t *biases,
                         int64_t N, int64_t K, float *out) {
    const int64_t groups = K / 64;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t r = tiled_record(n, g, groups);
            const float s = or_bf16_to_f32(scales[r]);
            const float b = or_bf16_to_f32(biases[r]);
            for (int64_t j = 0; j < 64; ++j) {
                const uint32_t word = words[r * 8 + j / 8];
                const float q = (float)((word >> (4 * (j % 8))) & 0xfu);
                const float sq = s * q;
                out[n * K + g * 64 + j] = sq + b;
            }
        }
    }
}

/* Converter.tile (Retile.swift:135-153). */
void or_tile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes) {
    const uint8_t *s = (const uint8_t *)src;
    uint8_t *d = (uint8_t *)dst;
    for (int64_t tile = 0; tile < rows / 128; ++tile)
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t base = (tile * groups + g) * 128;
            for (int64_t n = 0; n < 128; ++n)
                memcpy(d + (base + n) * element_bytes,
                       s + ((tile * 128 + n) * groups + g) * element_bytes, (size_t)element_bytes);
        }
}

void or_untile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes) {
    const uint8_t *s = (const uint8_t *)src;
    uint8_t *d = (uint8_t *)dst;
    for (int64_t tile = 0; tile < rows / 128; ++tile)
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t base = (tile * groups + g) * 128;
            for (int64_t n = 0; n < 128; ++n)
                memcpy(d + ((tile * 128 + n) * groups + g) * element_bytes,
                       s + (base + n) * element_bytes, (size_t)element_bytes);
        }
}

/* ---- GEMM --------------------------------------------------------------------------------- */

/* GemmOracleTests.swift:139-148: sum += bf16(a) * dequant in fp32, k sequential. */
void or_gemm_a_bf16_w_f32(const uint16_t *a, int64_t lda, const float *w, int64_t M, int64_t N,
                          int64_t K, float *out) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float sum = 0.0f;
            const float *wr = w + n * K;
            const uint16_t *ar = a + m * lda;
            for (int64_t k = 0; k < K; ++k) {
                const float p = or_bf16_to_f32(ar[k]) * wr[k];
                sum += p;
            }
            out[m * N + n] = sum;
        }
}

/* GemmOracle.bf16 (GemmOracle.swift:6-29). */
void or_gemm_bf16(const uint16_t *a, const uint16_t *b, int64_t M, int64_t N, int64_t K, float *out) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float sum = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float p = or_bf16_to_f32(a[m * K + k]) * or_bf16_to_f32(b[k * N + n]);
                sum += p;
            }
            out[m * N + n] = sum;
        }
}

/* Dequantize one row (DequantOracle.swift:16-23 for a single row). */
static void q4_row(const uint32_t *words, int64_t stride_words, const uint16_t *scales,
                   const uint16_t *biases, int64_t n, int64_t K, float *row) {
    const int64_t groups = (K + 63) / 64;
    for (int64_t k = 0; k < K; ++k) {
        const uint32_t word = words[n * stride_words + k / 8];
        const float q = (float)((word >> (4 * (k % 8))) & 0xfu);
        const float s = or_bf16_to_f32(scales[n * groups + k / 64]);
        const float b = or_bf16_to_f32(biases[n * groups + k / 64]);
        const float sq = s * q;
        row[k] = sq + b;
    }
}

void or_q4_gemm_rowmajor(const uint16_t *a, int64_t lda, const uint32_t *words, int64_t stride_words,
                         const uint16_t *scales, const uint16_t *biases, int64_t M, int64_t N, int64_t K,
                         int64_t n0, int64_t n1, float *out, int threads) {
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
    {
        float *w = (float *)malloc((size_t)K * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t n = n0; n < n1; ++n) {
            q4_row(words, stride_words, scales, biases, n, K, w);
            for (int64_t m = 0; m < M; ++m) {
                float sum = 0.0f;
                const uint16_t *ar = a + m * lda;
                for (int64_t k = 0; k < K; ++k) {
                    const float p = or_bf16_to_f32(ar[k]) * w[k];
                    sum += p;
                }
                out[m * N + n] = sum;
            }
        }
        free(w);
    }
    (void)threads;
}

/* engine.metal:24 sp_silu, applied as in sp_mlp_in_* (engine.metal:2050). */
void or_silu_mul(const float *gate, const float *up, int64_t count, float *out) {
    for (int64_t i = 0; i < count; ++i) {
        const float g = gate[i];
        const float e = expf(-g);
        const float d = 1.0f + e;
        const float s = g / d;
        out[i] = s * up[i];
    }
}

/* ---- operand producers ------------------------------------------------------------------------ */

static float or_silu(float x) {
    const float e = expf(-x);
    const float d = 1.0f + e;
    return x / d;
}

/* Sums of 64 rounded values in column order. */
static float or_sum64(const uint16_t *bits) {
    float s = 0.0f;
    for (int i = 0; i < 64; ++i) s += or_bf16_to_f32(bits[i]);
    return s;
}

void or_prepare_operand(const float *in, int64_t rows, int64_t inner, uint16_t *out, float *sums) {
    const int64_t groups = inner / 64;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < inner; ++k) out[r * inner + k] = or_f32_to_bf16_rne(in[r * inner + k]);
        for (int64_t g = 0; g < groups; ++g) sums[r * groups + g] = or_sum64(out + r * inner + g * 64);
    }
}

void or_silu_mul_operand(const float *gate, const float *up, const float *row_inv, int64_t rows, int64_t dim,
                         uint16_t *out, float *sums) {
    const int64_t groups = dim / 64;
    for (int64_t r = 0; r < rows; ++r) {
        const float s = row_inv ? row_inv[r] : 1.0f;
        for (int64_t k = 0; k < dim; ++k) {
            const float g = gate[r * dim + k] * s, u = up[r * dim + k] * s;
            const float v = or_silu(g) * u;
            out[r * dim + k] = or_f32_to_bf16_rne(v);
        }
        for (int64_t g = 0; g < groups; ++g) sums[r * groups + g] = or_sum64(out + r * dim + g * 64);
    }
}

void or_emit_operand(const float *hidden, const uint16_t *norm_weight, int64_t rows, int64_t dim, uint16_t *values,
                     float *sums, float *squares) {
    const int64_t groups = dim / 64;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < dim; ++k) {
            const float h = hidden[r * dim + k];
            const float v = h * or_bf16_to_f32(norm_weight[k]);
            values[r * dim + k] = or_f32_to_bf16_rne(v);
        }
        for (int64_t g = 0; g < groups; ++g) {
            sums[r * groups + g] = or_sum64(values + r * dim + g * 64);
            float q = 0.0f;
            for (int i = 0; i < 64; ++i) {
                const float h = hidden[r * dim + g * 64 + i];
                const float hh = h * h;
                q += hh;
            }
            squares[r * groups + g] = q;
        }
    }
}

void or_row_inv(const float *squares, int64_t rows, int64_t groups, int64_t dim, float eps, float *inv) {
    for (int64_t r = 0; r < rows; ++r) {
        float total = 0.0f;
        for (int64_t g = 0; g < groups; ++g) total += squares[r * groups + g];
        const float mean = total / (float)dim;
        inv[r] = 1.0f / sqrtf(mean + eps);
    }
}

/* ---- GGUF Q4_K / Q5_K --------------------------------------------------------------------- */

/* The 6-bit scale and minimum of group j (GgufQuant.swift:196-203). */
static void q45k_scale_min(const uint8_t *b, int j, uint8_t *scale, uint8_t *minimum) {
    const uint8_t *packed = b + 4;
    if (j < 4) {
        *scale = packed[j] & 63;
        *minimum = packed[j + 4] & 63;
    } else {
        *scale = (uint8_t)((packed[j + 4] & 0xf) | ((packed[j - 4] >> 6) << 4));
        *minimum = (uint8_t)((packed[j + 4] >> 4) | ((packed[j] >> 6) << 4));
    }
}

/* GgufTensorType.decodeQ45K (GgufQuant.swift:191-212). */
void or_q45k_decode(const uint8_t *blocks, int64_t nblocks, int fifth_bit, float *out) {
    const int64_t size = fifth_bit ? 176 : 144;
    const int codes = fifth_bit ? 48 : 16;
    for (int64_t i = 0; i < nblocks; ++i) {
        const uint8_t *b = blocks + i * size;
        float *values = out + i * 256;
        const float d = half_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        const float dmin = half_to_f32((uint16_t)(b[2] | (b[3] << 8)));
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, mn;
            q45k_scale_min(b, j, &sc, &mn);
            const float scaled = d * (float)sc;
            const float offset = dmin * (float)mn;
            for (int e = 0; e < 32; ++e) {
                const uint8_t byte = b[codes + 32 * (j / 2) + e];
                float code = (float)(j % 2 == 0 ? (byte & 15) : (byte >> 4));
                if (fifth_bit) code += 16.0f * (float)((b[16 + e] >> j) & 1);
                const float p = code * scaled;
                values[32 * j + e] = p - offset;
            }
        }
    }
}

/* The sixteen IQ4_NL / IQ4_XS code values, llama.cpp's kvalues_iq4nl (the format's table, as the
 * reference keeps it at GgufQuant.swift:56). */
static const int8_t kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* The IQ3_S codebook (the format's table: llama.cpp's iq3s_grid, which the reference keeps as
 * GgufTensorType.iq3sGrid, GgufQuant.swift:60). An entry is four magnitudes, each an odd number
 * 1..15; here entry i is stored as twelve bits, magnitude t = 2 ((code >> 3t) & 7) + 1. The
 * tests compare the expansion with the 512 entries read from the reference's file. */
static const uint16_t kIq3sPacked[512] = {
    0x000, 0x001, 0x002, 0x005, 0x007, 0x008, 0x009, 0x00a, 0x00c, 0x00e, 0x010, 0x011, 0x015, 0x01b, 0x020, 0x022,
    0x025, 0x027, 0x029, 0x02b, 0x030, 0x032, 0x039, 0x03c, 0x03f, 0x040, 0x041, 0x042, 0x044, 0x048, 0x049, 0x04d,
    0x050, 0x053, 0x057, 0x059, 0x05d, 0x064, 0x071, 0x075, 0x07a, 0x080, 0x081, 0x085, 0x087, 0x088, 0x08b, 0x08e,
    0x091, 0x095, 0x098, 0x09c, 0x0a2, 0x0a5, 0x0a7, 0x0a9, 0x0ab, 0x0b8, 0x0bb, 0x0c3, 0x0c9, 0x0cd, 0x0d0, 0x0d2,
    0x0d9, 0x0db, 0x0de, 0x0e4, 0x0e8, 0x0ea, 0x0f7, 0x0f9, 0x0fd, 0x100, 0x10b, 0x10f, 0x111, 0x114, 0x11a, 0x120,
    0x123, 0x129, 0x138, 0x142, 0x144, 0x150, 0x152, 0x156, 0x15b, 0x161, 0x165, 0x167, 0x176, 0x17b, 0x186, 0x189,
    0x18b, 0x199, 0x1aa, 0x1b9, 0x1c0, 0x1c2, 0x1c4, 0x1d0, 0x1d2, 0x1d6, 0x1db, 0x1e8, 0x1ec, 0x200, 0x201, 0x202,
    0x204, 0x208, 0x209, 0x20b, 0x20d, 0x20f, 0x210, 0x212, 0x219, 0x21c, 0x21e, 0x22c, 0x22e, 0x231, 0x23a, 0x240,
    0x241, 0x243, 0x246, 0x248, 0x24c, 0x251, 0x258, 0x25b, 0x261, 0x268, 0x26a, 0x278, 0x27e, 0x280, 0x28a, 0x28d,
    0x28f, 0x290, 0x294, 0x29a, 0x2a0, 0x2a3, 0x2ad, 0x2b0, 0x2ba, 0x2c1, 0x2c4, 0x2c7, 0x2c8, 0x2cb, 0x2d1, 0x2d7,
    0x2d8, 0x2dc, 0x2e1, 0x2f2, 0x2f8, 0x303, 0x305, 0x30a, 0x30c, 0x319, 0x31b, 0x322, 0x326, 0x328, 0x32c, 0x341,
    0x348, 0x34b, 0x351, 0x358, 0x35a, 0x369, 0x390, 0x394, 0x397, 0x3a4, 0x3a6, 0x3c1, 0x3c3, 0x3c8, 0x3ca, 0x3d1,
    0x3dd, 0x3e1, 0x3f2, 0x3f8, 0x400, 0x401, 0x403, 0x405, 0x407, 0x408, 0x40a, 0x40c, 0x40e, 0x411, 0x413, 0x417,
    0x418, 0x41a, 0x421, 0x423, 0x425, 0x428, 0x42a, 0x437, 0x438, 0x43b, 0x43d, 0x440, 0x442, 0x448, 0x44b, 0x44f,
    0x452, 0x455, 0x459, 0x45c, 0x462, 0x469, 0x481, 0x484, 0x487, 0x491, 0x493, 0x498, 0x49f, 0x4a1, 0x4ab, 0x4af,
    0x4b9, 0x4bc, 0x4c0, 0x4c2, 0x4c5, 0x4c9, 0x4d2, 0x4d4, 0x4d9, 0x4db, 0x4e2, 0x4e8, 0x4f6, 0x501, 0x507, 0x510,
    0x513, 0x51a, 0x51d, 0x521, 0x53a, 0x53d, 0x544, 0x549, 0x552, 0x55f, 0x560, 0x56b, 0x578, 0x580, 0x582, 0x587,
    0x591, 0x5ad, 0x5b1, 0x5c5, 0x5c9, 0x5d6, 0x5d8, 0x5e3, 0x5e8, 0x602, 0x609, 0x60b, 0x60d, 0x60f, 0x612, 0x619,
    0x61b, 0x61d, 0x622, 0x624, 0x627, 0x629, 0x633, 0x639, 0x641, 0x643, 0x645, 0x64c, 0x651, 0x653, 0x660, 0x670,
    0x67a, 0x67e, 0x680, 0x68a, 0x690, 0x69a, 0x69c, 0x6a8, 0x6c1, 0x6c8, 0x6cc, 0x6d1, 0x6d3, 0x6d7, 0x6d8, 0x6e1,
    0x6e3, 0x6e7, 0x6ed, 0x6fb, 0x703, 0x709, 0x70e, 0x712, 0x719, 0x72a, 0x730, 0x734, 0x741, 0x748, 0x74a, 0x755,
    0x75a, 0x764, 0x76e, 0x77b, 0x78e, 0x7a1, 0x7c1, 0x7c3, 0x7d0, 0x7d2, 0x7dd, 0x800, 0x804, 0x80a, 0x810, 0x814,
    0x817, 0x81a, 0x821, 0x828, 0x838, 0x842, 0x847, 0x849, 0x84b, 0x852, 0x858, 0x85d, 0x863, 0x869, 0x86d, 0x881,
    0x883, 0x888, 0x88d, 0x891, 0x89b, 0x8a0, 0x8af, 0x8b2, 0x8b8, 0x8c4, 0x8c9, 0x8cb, 0x8d0, 0x8d2, 0x8d9, 0x8dd,
    0x900, 0x902, 0x914, 0x91f, 0x920, 0x939, 0x945, 0x947, 0x951, 0x972, 0x98b, 0x99c, 0x9b0, 0x9c8, 0x9cd, 0x9d8,
    0x9e3, 0x9e9, 0xa02, 0xa08, 0xa0c, 0xa12, 0xa20, 0xa24, 0xa27, 0xa2a, 0xa36, 0xa3c, 0xa41, 0xa43, 0xa45, 0xa4a,
    0xa51, 0xa5a, 0xa7a, 0xa80, 0xa89, 0xa93, 0xa98, 0xa9e, 0xaab, 0xac2, 0xac7, 0xac8, 0xad7, 0xae4, 0xae9, 0xaf5,
    0xafb, 0xb01, 0xb04, 0xb10, 0xb1a, 0xb26, 0xb4a, 0xb56, 0xb69, 0xb6b, 0xba2, 0xbc2, 0xbc4, 0xbd2, 0xc09, 0xc0b,
    0xc0d, 0xc19, 0xc1b, 0xc30, 0xc40, 0xc50, 0xc57, 0xc74, 0xc8a, 0xc9c, 0xca2, 0xcad, 0xcb2, 0xcb8, 0xcc0, 0xccc,
    0xcd1, 0xce0, 0xd15, 0xd23, 0xd32, 0xd40, 0xd43, 0xd5c, 0xd70, 0xd85, 0xda0, 0xdc9, 0xdcb, 0xe00, 0xe04, 0xe07,
    0xe10, 0xe12, 0xe1e, 0xe20, 0xe2c, 0xe32, 0xe42, 0xe49, 0xe54, 0xe63, 0xe65, 0xe81, 0xe84, 0xe88, 0xe8e, 0xe91,
    0xe98, 0xea9, 0xec2, 0xeda, 0xedd, 0xeeb, 0xf01, 0xf05, 0xf0b, 0xf10, 0xf28, 0xf52, 0xf62, 0xf82, 0xf99, 0xfc0,
};

static uint32_t iq3s_entry(int code) {
    const uint32_t c = kIq3sPacked[code];
    uint32_t e = 0;
    for (int t = 0; t < 4; ++t) e |= (2u * ((c >> (3 * t)) & 7u) + 1u) << (8 * t);
    return e;
}

void or_iq3s_grid(uint32_t *out) {
    for (int i = 0; i < 512; ++i) out[i] = iq3s_entry(i);
}

/* One native block of a 32- or 256-element GGUF format to fp32, with the reference decoder's fp32
 * operation order (GgufQuant.swift): Q8_0 :172-175 (d * int8), IQ4_NL :179-185 (d * table, low
 * nibbles first), Q6_K :218-230 ((d * scale) * (code - 32) with the 4 low bits from ql and 2 high
 * from qh), IQ4_XS :261-275 ((d * (scale - 32)) * table). Returns the elements decoded (0 for a
 * type not handled here). */
static int gguf_decode_block(int type, const uint8_t *b, float *out) {
    switch (type) {
        case 8: { /* Q8_0 */
            const float d = half_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            for (int e = 0; e < 32; ++e) out[e] = d * (float)(int8_t)b[2 + e];
            return 32;
        }
        case 20: { /* IQ4_NL */
            const float d = half_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            for (int e = 0; e < 16; ++e) {
                out[e] = d * (float)kIq4Values[b[2 + e] & 15];
                out[16 + e] = d * (float)kIq4Values[b[2 + e] >> 4];
            }
            return 32;
        }
        case 14: { /* Q6_K: ql[128], qh[64], scales[16] (int8), d (fp16) at 208 */
            const float d = half_to_f32((uint16_t)(b[208] | (b[209] << 8)));
            for (int j = 0; j < 8; ++j) {
                const int half = j / 4, quarter = j % 4;
                for (int e = 0; e < 32; ++e) {
                    const int low = (b[64 * half + 32 * (quarter & 1) + e] >> (4 * (quarter >> 1))) & 15;
                    const int high = (b[128 + 32 * half + e] >> (2 * quarter)) & 3;
                    const float code = (float)(low | (high << 4)) - 32.0f;
                    const float scale = (float)(int8_t)b[192 + 2 * j + e / 16];
                    const float ds = d * scale;
                    out[32 * j + e] = ds * code;
                }
            }
            return 256;
        }
        case 23: { /* IQ4_XS: d, scales_h (u16), scales_l[4], qs[128] */
            const float d = half_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            const uint32_t high = (uint32_t)(b[2] | (b[3] << 8));
            for (int j = 0; j < 8; ++j) {
                const uint32_t low = ((uint32_t)b[4 + j / 2] >> (4 * (j % 2))) & 15u;
                const uint32_t scale = low | (((high >> (2 * j)) & 3u) << 4);
                const float scaled = d * ((float)scale - 32.0f);
                for (int e = 0; e < 16; ++e) {
                    const uint8_t byte = b[8 + 16 * j + e];
                    out[32 * j + e] = scaled * (float)kIq4Values[byte & 15];
                    out[32 * j + 16 + e] = scaled * (float)kIq4Values[byte >> 4];
                }
            }
            return 256;
        }
        case 11: { /* Q3_K: hmask[32], qs[64], scales[12], d (fp16) at 108 (GgufQuant.swift:238-256) */
            const float d = half_to_f32((uint16_t)(b[108] | (b[109] << 8)));
            for (int j = 0; j < 8; ++j) {
                const int half = j / 4, shift = 2 * (j % 4);
                for (int e = 0; e < 32; ++e) {
                    const int k = 2 * j + e / 16, word = k / 4, byte = k % 4;
                    const int slow = (b[96 + 4 * (word % 2) + byte] >> (4 * (word / 2))) & 0xF;
                    const int shigh = (b[104 + byte] >> (2 * word)) & 3;
                    const float scale = (float)(slow | (shigh << 4)) - 32.0f;
                    const int low = (b[32 + 32 * half + e] >> shift) & 3;
                    const int high = (b[e] >> j) & 1;
                    const float code = (float)(low | (high << 2)) - 4.0f;
                    const float ds = d * scale;
                    out[32 * j + e] = ds * code;
                }
            }
            return 256;
        }
        case 21: { /* IQ3_S: d, qs[64], qh[8], signs[32], scales[4] (GgufQuant.swift:283-300) */
            const float d = half_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            for (int j = 0; j < 8; ++j) {
                const int scale = (b[106 + j / 2] >> (4 * (j % 2))) & 15;
                const float weight = d * (1.0f + 2.0f * (float)scale);
                const int ninth = b[66 + j];
                for (int k = 0; k < 8; ++k) {
                    const uint32_t entry = iq3s_entry(b[2 + 8 * j + k] | (((ninth >> k) & 1) << 8));
                    for (int t = 0; t < 4; ++t) {
                        const int e = 4 * k + t;
                        const float magnitude = (float)((entry >> (8 * t)) & 0xFFu);
                        const int negative = (b[74 + 4 * j + e / 8] >> (e % 8)) & 1;
                        const float wm = weight * magnitude;
                        out[32 * j + e] = wm * (1.0f - 2.0f * (float)negative);
                    }
                }
            }
            return 256;
        }
        default:
            return 0;
    }
}

int or_gguf_block_bytes(int type) {
    switch (type) {
        case 8: return 34;
        case 20: return 18;
        case 14: return 210;
        case 23: return 136;
        case 11: return 110;
        case 21: return 110;
        case 12: return 144;
        case 13: return 176;
        default: return 0;
    }
}

int or_gguf_decode(int type, const uint8_t *blocks, int64_t nblocks, float *out) {
    if (type == 12 || type == 13) {
        or_q45k_decode(blocks, nblocks, type == 13, out);
        return 0;
    }
    const int size = or_gguf_block_bytes(type);
    if (size == 0) return -1;
    int64_t at = 0;
    for (int64_t i = 0; i < nblocks; ++i) at += gguf_decode_block(type, blocks + i * size, out + at);
    return 0;
}

/* GgufPlanes.slot (GgufPlanes.swift:93-95). */
int or_gguf_slot(int element) { return 8 * ((element >> 2) & 3) + 4 * (element >> 4) + (element & 3); }

/* GgufPlanes.record (GgufPlanes.swift:88-90). */
static inline int64_t plane_record(int64_t row, int64_t block, int64_t blocks) {
    return ((row / 128) * blocks + block) * 128 + row % 128;
}

/* storePairs (GgufPlanes.swift:286-293): word c holds slots 8c..8c+7, slot 8c+i at bit
 * (i & 1) * 16 + 4 * (i >> 1). */
static void store_pairs(const uint8_t *slots, uint8_t *plane) {
    for (int c = 0; c < 4; ++c) {
        uint32_t word = 0;
        for (int i = 0; i < 8; ++i) word |= (uint32_t)slots[8 * c + i] << ((i & 1) * 16 + 4 * (i >> 1));
        memcpy(plane + 4 * c, &word, 4);
    }
}

static void load_pairs(const uint8_t *plane, uint8_t *slots) {
    for (int c = 0; c < 4; ++c) {
        uint32_t word;
        memcpy(&word, plane + 4 * c, 4);
        for (int i = 0; i < 8; ++i) slots[8 * c + i] = (uint8_t)((word >> ((i & 1) * 16 + 4 * (i >> 1))) & 15);
    }
}

/* storeBits width 1 (GgufPlanes.swift:295-304): slot i at bit i of one word. */
static void store_bits1(const uint8_t *slots, uint8_t *plane) {
    uint32_t word = 0;
    for (int i = 0; i < 32; ++i) word |= (uint32_t)slots[i] << i;
    memcpy(plane, &word, 4);
}

static void load_bits1(const uint8_t *plane, uint8_t *slots) {
    uint32_t word;
    memcpy(&word, plane, 4);
    for (int i = 0; i < 32; ++i) slots[i] = (uint8_t)((word >> i) & 1);
}

/* GgufPlanes.repack (GgufPlanes.swift:103-136) with pack for Q4_K/Q5_K (:221-229). */
int or_q45k_repack(const uint8_t *native, int64_t N, int64_t K, int fifth_bit, uint8_t *plane0,
                   uint8_t *plane1, uint8_t *meta) {
    if (N <= 0 || N % 128 || K <= 0 || K % 256) return -1;
    const int64_t block_bytes = fifth_bit ? 176 : 144;
    const int codes = fifth_bit ? 48 : 16;
    const int64_t row_bytes = K / 256 * block_bytes;
    const int64_t groups = K / 32, blocks = groups / 8;
    uint8_t low[32], high[32];
    for (int64_t row = 0; row < N; ++row)
        for (int64_t group = 0; group < groups; ++group) {
            const int64_t block = group / 8;
            const int j = (int)(group % 8);
            const uint8_t *b = native + row * row_bytes + block * block_bytes;
            const int64_t rec = plane_record(row, group, groups);
            for (int e = 0; e < 32; ++e) {
                low[or_gguf_slot(e)] = (uint8_t)((b[codes + 32 * (j / 2) + e] >> (4 * (j % 2))) & 15);
                if (fifth_bit) high[or_gguf_slot(e)] = (uint8_t)((b[16 + e] >> j) & 1);
            }
            store_pairs(low, plane0 + rec * 16);
            if (fifth_bit) store_bits1(high, plane1 + rec * 4);
            if (j == 0) memcpy(meta + plane_record(row, block, blocks) * 16, b, 16);
        }
    return 0;
}

/* GgufPlanes.unpack (GgufPlanes.swift:161-194) with the Q4_K/Q5_K case (:258-267). */
int or_q45k_unpack(const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, int64_t N,
                   int64_t K, int fifth_bit, uint8_t *native) {
    if (N <= 0 || N % 128 || K <= 0 || K % 256) return -1;
    const int64_t block_bytes = fifth_bit ? 176 : 144;
    const int codes = fifth_bit ? 48 : 16;
    const int64_t row_bytes = K / 256 * block_bytes;
    const int64_t groups = K / 32, blocks = groups / 8;
    memset(native, 0, (size_t)(N * row_bytes));
    uint8_t low[32], high[32];
    for (int64_t row = 0; row < N; ++row)
        for (int64_t group = 0; group < groups; ++group) {
            const int64_t block = group / 8;
            const int j = (int)(group % 8);
            uint8_t *b = native + row * row_bytes + block * block_bytes;
            const int64_t rec = plane_record(row, group, groups);
            load_pairs(plane0 + rec * 16, low);
            if (fifth_bit) load_bits1(plane1 + rec * 4, high);
            for (int e = 0; e < 32; ++e) {
                b[codes + 32 * (j / 2) + e] |= (uint8_t)(low[or_gguf_slot(e)] << (4 * (j % 2)));
                if (fifth_bit) b[16 + e] |= (uint8_t)(high[or_gguf_slot(e)] << j);
            }
            if (j == 0) memcpy(b, meta + plane_record(row, block, blocks) * 16, 16);
        }
    return 0;
}

void or_q45k_gemm_native(const uint16_t *a, int64_t lda, const uint8_t *native, int fifth_bit,
                         int64_t M, int64_t N, int64_t K, int64_t n0, int64_t n1, float *out,
                         int threads) {
    const int64_t block_bytes = fifth_bit ? 176 : 144;
    const int64_t row_bytes = K / 256 * block_bytes;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
    {
        float *w = (float *)malloc((size_t)K * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t n = n0; n < n1; ++n) {
            or_q45k_decode(native + n * row_bytes, K / 256, fifth_bit, w);
            for (int64_t m = 0; m < M; ++m) {
                float sum = 0.0f;
                const uint16_t *ar = a + m * lda;
                for (int64_t k = 0; k < K; ++k) {
                    const float p = or_bf16_to_f32(ar[k]) * w[k];
                    sum += p;
                }
                out[m * N + n] = sum;
            }
        }
        free(w);
    }
    (void)threads;
}

/* ---- GGUF conversion: the gated-delta value heads and the float -> Q8_0 requantisation -------- */

/* GgufNames.mlxValueHead (GgufNames.swift:104): the engine's index of file value head i,
 * (value_heads / key_heads) (i % key_heads) + i / key_heads -- 3 (i % 16) + i / 16 for Qwen. */
int or_mlx_value_head(int i, int key_heads, int value_heads) {
    return (value_heads / key_heads) * (i % key_heads) + i / key_heads;
}

/* GgufConvert.HeadOrder.destination (GgufConvert.swift:62-69). */
int64_t or_head_destination(int64_t unit, int64_t first, int64_t span, int key_heads, int value_heads) {
    if (unit < first || (unit - first) / span >= value_heads) return unit;
    const int64_t h = (unit - first) / span;
    return first + (int64_t)or_mlx_value_head((int)h, key_heads, value_heads) * span + (unit - first) % span;
}

/* GgufConvert.ggufPlanes' `order` (GgufConvert.swift:381-395): file row r to row destination(r),
 * rows [rows, stored) zero. span <= 0: no reordering. */
void or_order_rows(const uint8_t *native, int64_t rows, int64_t row_bytes, int64_t first, int64_t span,
                   int key_heads, int value_heads, int64_t stored, uint8_t *out) {
    memset(out, 0, (size_t)(stored * row_bytes));
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t to = span > 0 ? or_head_destination(r, first, span, key_heads, value_heads) : r;
        memcpy(out + to * row_bytes, native + r * row_bytes, (size_t)row_bytes);
    }
}

/* IEEE binary32 -> binary16 bits, round to nearest even (Swift's Float16(Float)): normals,
 * subnormals, overflow to infinity, NaN kept quiet. */
uint16_t or_f32_to_f16_rne(float value) {
    uint32_t x;
    memcpy(&x, &value, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xFFu, mant = x & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    const int e = (int)exp - 127 + 15;  /* binary16 biased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t m = mant | (exp ? 0x800000u : 0u);  /* 24-bit significand */
    int shift;                                    /* bits of m dropped */
    uint32_t he;                                  /* binary16 exponent field of the result */
    if (e >= 1) {
        shift = 13;
        he = (uint32_t)e;
    } else {
        shift = 14 - e;  /* subnormal: value = m 2^(exp-150) = q 2^-24 */
        he = 0;
        if (exp == 0) shift = 24;  /* binary32 subnormals are far below binary16's range */
        if (shift > 25) return (uint16_t)sign;
    }
    const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    uint32_t r = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
    if (e >= 1) {
        /* q holds the implicit bit at 2^10; a carry out of the significand moves the exponent */
        r = (he << 10) + (r - 0x400u);
        if (r >= 0x7C00u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | r);
    }
    return (uint16_t)(sign | r);  /* a subnormal that rounds up to 0x400 is the smallest normal */
}

/* GgufConvert.q8_0Blocks (GgufConvert.swift:236-257), block by block as written there: the largest
 * magnitude, scale = largest / 127 and inverse = 1 / scale in fp32 (0 for a zero scale), the scale
 * stored as fp16, each code (value * inverse) rounded half away from zero and clamped to int8. */
void or_q8_0_blocks(const float *values, int64_t blocks, uint8_t *out) {
    for (int64_t b = 0; b < blocks; ++b) {
        float largest = 0.0f;
        for (int e = 0; e < 32; ++e) {
            const float a = fabsf(values[32 * b + e]);
            largest = a > largest ? a : largest;
        }
        const float scale = largest / 127.0f;
        const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
        const uint16_t stored = or_f32_to_f16_rne(scale);
        out[34 * b] = (uint8_t)(stored & 0xFFu);
        out[34 * b + 1] = (uint8_t)(stored >> 8);
        for (int e = 0; e < 32; ++e) {
            float code = roundf(values[32 * b + e] * inverse);
            code = code < -128.0f ? -128.0f : code > 127.0f ? 127.0f : code;
            out[34 * b + 2 + e] = (uint8_t)(int8_t)code;
        }
    }
}

/* The activations a head-ordered weight meets (engine_gguf.metal:55-72): out[m][k] = a[m][col(k)],
 * col(k) = mlxValueHead(k / 128) 128 + k % 128 -- the weight's inner column k is file head k / 128. */
void or_head_gather(const uint16_t *a, int64_t lda, int64_t m, int64_t inner, int key_heads, uint16_t *out) {
    const int heads = (int)(inner / 128);
    for (int64_t r = 0; r < m; ++r)
        for (int64_t k = 0; k < inner; ++k) {
            const int64_t col = (int64_t)or_mlx_value_head((int)(k / 128), key_heads, heads) * 128 + k % 128;
            out[r * inner + k] = a[r * lda + col];
        }
}
