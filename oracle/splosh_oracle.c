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
