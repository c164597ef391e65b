/*
 * splosh_oracle.h -- CPU restatement of the reference's quantized-matmul algorithms.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker the HIP library is held against; it is never
 * the thing measured or shipped. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. Every function cites the reference file:line it restates
 * (paths are into the ajaxharg/Splosh tree).
 *
 * Arithmetic conventions (all fp32, no FMA contraction: the library is built -ffp-contract=off):
 *   bf16 -> fp32 is a 16-bit shift (Q4BufferLayout.swift:123-125).
 *   MLX affine dequant is scale * q + bias, one rounding (DequantOracle.swift:20-21).
 *   GEMM sums are sequential in k, fp32 (GemmOracle.swift:17-24).
 */
#ifndef SPLOSH_ORACLE_H
#define SPLOSH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 helpers. Q4BufferLayout.bf16 (:123) and bf16Bits (:127, rounds half up in magnitude). */
float or_bf16_to_f32(uint16_t bits);
uint16_t or_f32_to_bf16_halfup(float value);
/* Round-to-nearest-even, the conversion a GPU `bfloat(x)` performs (engine_na.metal:49). */
uint16_t or_f32_to_bf16_rne(float value);
void or_f32_to_bf16_rne_n(const float *src, uint16_t *dst, int64_t count);

/* MLX affine q4, row-major padded: word (row * strideWords + k / 8), nibble 4 * (k % 8),
 * sidecar (row * groupsPerRow + k / 64). Q4BufferLayout.swift:82-117; DequantOracle.swift:11-25.
 * Writes out[row * K + k] for row < N, k < K. */
void or_q4_dequant_rowmajor(const uint32_t *words, int64_t stride_words, const uint16_t *scales,
                            const uint16_t *biases, int64_t N, int64_t K, float *out);

/* The same weight in the 128-row tiled layout that Converter.tile writes (Retile.swift:135-153):
 * codes [N/128][K/64][128][8 words], sidecars [N/128][K/64][128]. Requires N % 128 == 0 and
 * K % 64 == 0. */
void or_q4_dequant_tiled(const uint32_t *words, const uint16_t *scales, const uint16_t *biases,
                         int64_t N, int64_t K, float *out);

/* Converter.tile: [row][group][element] -> [tile][group][row in tile][element]
 * (Retile.swift:135-153). rows % 128 == 0. */
void or_tile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes);
/* Its inverse. */
void or_untile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes);

/* The reference's q4 GEMM semantics (GemmOracleTests.swift:139-148, gemm_q4.metal:44-53):
 * out[m][n] = sum_k bf16(a[m][k]) * w[n][k] in fp32, sequential in k, with w the fp32 dequantized
 * weight [N][K]. a has row stride lda. */
void or_gemm_a_bf16_w_f32(const uint16_t *a, int64_t lda, const float *w, int64_t M, int64_t N,
                          int64_t K, float *out);

/* GemmOracle.bf16 (GemmOracle.swift:6-29): C[M,N] = A[M,K] x B[K,N], both bf16, fp32 sums. */
void or_gemm_bf16(const uint16_t *a, const uint16_t *b, int64_t M, int64_t N, int64_t K, float *out);

/* Fused form used as the CPU baseline: for each output row n, dequantize row n of the
 * row-major q4 weight to fp32 (DequantOracle.dequantize) and take the sequential fp32 dot with
 * each activation row. Same values as or_q4_dequant_rowmajor + or_gemm_a_bf16_w_f32. Output
 * columns [n0, n1) only, so a bounded sample can be timed. threads > 1 uses OpenMP over n. */
void or_q4_gemm_rowmajor(const uint16_t *a, int64_t lda, const uint32_t *words, int64_t stride_words,
                         const uint16_t *scales, const uint16_t *biases, int64_t M, int64_t N, int64_t K,
                         int64_t n0, int64_t n1, float *out, int threads);

/* silu(g) * u with silu(x) = x / (1 + exp(-x)) in fp32 (engine.metal:24, :2050). */
void or_silu_mul(const float *gate, const float *up, int64_t count, float *out);

/* Operand producers (the steps either side of a GEMM). Every "sums" output is per row and per 64
 * consecutive columns, of the values after their bf16 rounding, added in column order.
 * sp_na_prepare (engine_na.metal:38-56): out = RNE(in), sums of out. */
void or_prepare_operand(const float *in, int64_t rows, int64_t inner, uint16_t *out, float *sums);
/* sp_silu_mul_na (engine.metal:200-218): out = RNE(silu(g s) * (u s)) with s = row_inv[row] (1 when
 * row_inv is NULL), silu(x) = x / (1 + exp(-x)) (engine.metal:25); sums of out. */
void or_silu_mul_operand(const float *gate, const float *up, const float *row_inv, int64_t rows, int64_t dim,
                         uint16_t *out, float *sums);
/* The operand a residual projection emits for the next RMSNorm-ed GEMM (engine_na.metal:26-36,
 * 365-411): values = RNE(h * bf16(weight[col])), sums of values, squares = per-64 sums of h * h
 * (h the fp32 hidden state, after the residual add). */
void or_emit_operand(const float *hidden, const uint16_t *norm_weight, int64_t rows, int64_t dim, uint16_t *values,
                     float *sums, float *squares);
/* sp_row_inv (engine.metal:222-233): inv[row] = 1 / sqrt(sum_g squares[row][g] / dim + eps). */
void or_row_inv(const float *squares, int64_t rows, int64_t groups, int64_t dim, float eps, float *inv);

/* GGUF Q4_K (176-byte Q5_K with fifth_bit) block decode, GgufQuant.swift:191-212.
 * blocks: nblocks * (fifth_bit ? 176 : 144) bytes; out: nblocks * 256 floats. */
void or_q45k_decode(const uint8_t *blocks, int64_t nblocks, int fifth_bit, float *out);
/* Native blocks of GGUF type `type` (ggml id: 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K, 20 IQ4_NL,
 * 23 IQ4_XS) to fp32 with the reference decoder's op order (GgufQuant.swift:136-275). Returns -1
 * for another type. or_gguf_block_bytes: the native block size (0: not handled). */
int or_gguf_decode(int type, const uint8_t *blocks, int64_t nblocks, float *out);
int or_gguf_block_bytes(int type);
/* The IQ3_S codebook's 512 entries as the oracle expands them (byte t = magnitude of element t). */
void or_iq3s_grid(uint32_t *out);

/* GgufPlanes for Q4_K / Q5_K (GgufPlanes.swift:62-136, 161-194, 221-229, 288-305).
 * plane0 [N/128][K/32][128][16 B], plane1 [N/128][K/32][128][4 B] (Q5_K only),
 * meta [N/128][K/256][128][16 B]. native: N rows of K/256 blocks. Returns 0, or -1 on a
 * shape with no plane form (N % 128 or K % 256 nonzero). */
int or_q45k_repack(const uint8_t *native, int64_t N, int64_t K, int fifth_bit, uint8_t *plane0,
                   uint8_t *plane1, uint8_t *meta);
int or_q45k_unpack(const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, int64_t N,
                   int64_t K, int fifth_bit, uint8_t *native);
/* Element e (0..31) of a group in chunk order (GgufPlanes.swift:93-95). */
int or_gguf_slot(int element);

/* Fused Q5_K form for the CPU baseline: decode each row's blocks (GgufQuant.decodeQ45K) and take
 * the sequential fp32 dot with each activation row, output columns [n0, n1). */
void or_q45k_gemm_native(const uint16_t *a, int64_t lda, const uint8_t *native, int fifth_bit,
                         int64_t M, int64_t N, int64_t K, int64_t n0, int64_t n1, float *out,
                         int threads);

/* GGUF conversion (GgufNames.swift, GgufConvert.swift): value-head order and Q8_0 requantisation. */
int or_mlx_value_head(int i, int key_heads, int value_heads);
int64_t or_head_destination(int64_t unit, int64_t first, int64_t span, int key_heads, int value_heads);
void or_order_rows(const uint8_t *native, int64_t rows, int64_t row_bytes, int64_t first, int64_t span,
                   int key_heads, int value_heads, int64_t stored, uint8_t *out);
uint16_t or_f32_to_f16_rne(float value);
void or_q8_0_blocks(const float *values, int64_t blocks, uint8_t *out);
void or_head_gather(const uint16_t *a, int64_t lda, int64_t m, int64_t inner, int key_heads, uint16_t *out);

#ifdef __cplusplus
}
#endif
#endif
