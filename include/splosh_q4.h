/*
 * splosh_q4.h -- C ABI of the MI355X (gfx950) quantized-weight matmul library.
 *
 * The library replaces the quantized GEMV/GEMM hot path of Splosh (the SploshQuant format
 * contract and the GEMM entry points of SploshRuntime) with hand-written HIP kernels. Every entry
 * point takes caller-owned device pointers and a hipStream_t, validates its arguments before it
 * launches anything, returns a splosh_status, and is stream-ordered and asynchronous (except the
 * pure host helpers, which touch no device). Nothing is allocated per call: kernels that need
 * scratch memory take a caller workspace sized by splosh_workspace_bytes().
 *
 * Each declaration names the reference interface it stands in for (file:line in the Splosh tree).
 *
 * Formats
 *   MLX affine q4 (SploshQuant/MlxAffine.swift:21-86): w[n][k] = bf16(scale) * q + bf16(bias),
 *     q the 4-bit code at bits 4 (k % 8) of a uint32 word, one scale/bias per group of 64 k.
 *     ROW_MAJOR: word (n * row_stride_words + k / 8), sidecar (n * groups + k / 64)
 *       (Q4BufferLayout.swift:82-104), rows padded to 128 bytes by default.
 *     TILED128: Converter.tile (Model/Retile.swift:135-153): codes
 *       [n / 128][k / 64][n % 128][8 words], sidecars [n / 128][k / 64][n % 128].
 *   GGUF Q5_K (Model/GgufQuant.swift:191-212) in GgufPlanes form (Model/GgufPlanes.swift:8-20):
 *     plane0 [n/128][k/32][128][16 B], plane1 [n/128][k/32][128][4 B], meta [n/128][k/256][128][16 B].
 *
 * GEMM convention (Model/Gemm.swift:7): out[m][n] = sum_k a[m][k] * w[n][k] (+ residual[m][n]),
 * a bf16 [rows][inner] with row stride lda, accumulated in fp32, out fp32 or bf16 (RNE).
 */
#ifndef SPLOSH_Q4_H
#define SPLOSH_Q4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *hipStream_t;

/* Status codes. 1..8 are GemmQ4Error's cases (Model/Gemm.swift:43-52); the rest are
 * Q4BufferLayoutError (Quant/Q4BufferLayout.swift:16-23) and runtime failures
 * (SploshError.capabilityGateFailure, Runtime/Q4Runtime.swift:141-143). */
typedef enum splosh_status {
    SPLOSH_OK = 0,
    SPLOSH_ERR_INVALID_SHAPE = 1,
    SPLOSH_ERR_LAYOUT_MISMATCH = 2,
    SPLOSH_ERR_INVALID_ROW_STRIDE = 3,
    SPLOSH_ERR_ORIENTATION_MISMATCH = 4,
    SPLOSH_ERR_INVALID_GROUP_SIZE = 5,
    SPLOSH_ERR_SIDECAR_GEOMETRY_MISMATCH = 6,
    SPLOSH_ERR_SIDECAR_MISMATCH = 7,
    SPLOSH_ERR_BUFFER_TOO_SMALL = 8,
    SPLOSH_ERR_INVALID_DIMENSIONS = 9,
    SPLOSH_ERR_ARITHMETIC_OVERFLOW = 10,
    SPLOSH_ERR_INVALID_INDEX = 11,
    SPLOSH_ERR_NULL_POINTER = 12,
    SPLOSH_ERR_UNSUPPORTED = 13,
    SPLOSH_ERR_WORKSPACE_TOO_SMALL = 14,
    SPLOSH_ERR_HIP = 15
} splosh_status;

typedef enum splosh_orientation { SPLOSH_ROWS_BY_K = 0, SPLOSH_K_BY_COLUMNS = 1 } splosh_orientation;
typedef enum splosh_q4_order { SPLOSH_Q4_ROW_MAJOR = 0, SPLOSH_Q4_TILED128 = 1 } splosh_q4_order;
typedef enum splosh_dtype { SPLOSH_F32 = 0, SPLOSH_BF16 = 1 } splosh_dtype;

/* Kernel choice (the reference selects kernels through SPLOSH_* environment variables,
 * Runtime/Engine.swift:380-440; here the caller names one, or AUTO picks by rows). */
typedef enum splosh_kernel {
    SPLOSH_KERNEL_AUTO = 0,     /* 1..4 rows of tiled weights whose staged activation rows fit 80 KB
                                   (one or two rows up to K of about 18700, four up to about 9100):
                                   STREAM; else up to 64: DEQUANT (a single weight of at least two
                                   64-column bands a CU as the pair of its column halves); 65..128:
                                   rows 0..63 and the rest as two calls of the above (without the
                                   emit); more: PREFILL for tiled weights with lda % 8 == 0 and
                                   ldc % 4 == 0, else TILE; SCALAR for operands no other kernel
                                   takes */
    SPLOSH_KERNEL_STREAM = 1,   /* weight streaming on raw codes: the every-CU decode kernel for
                                   1-4 rows of tiled weights (with a workspace it splits the last
                                   round of row blocks over K, so every CU gets the same share),
                                   the lane-per-row kernel for row-major ones, the raw-code MFMA
                                   kernel for more rows */
    SPLOSH_KERNEL_DEQUANT = 2,  /* rows <= 64: stream-K MFMA kernel on weights dequantized to bf16 in
                                   registers; uses the workspace for split bands when given one */
    SPLOSH_KERNEL_TILE = 3,     /* any rows: LDS-tiled dequant-to-bf16 MFMA GEMM (prefill) */
    SPLOSH_KERNEL_SCALAR = 4,   /* one thread per output (gemm_q4.metal semantics) */
    SPLOSH_KERNEL_PREFILL = 5   /* TILED128 q4 weights (mlp_in: 128 columns of each a tile,
                                   silu(g) * u in the epilogue) or Q5_K / Q4_K planes:
                                   256 x 256 output tiles, two waves per SIMD, every weight
                                   dequantized once a tile into LDS; uses the workspace to split
                                   the last round of tiles over all CUs */
} splosh_kernel;

/* Q4BufferLayout (Quant/Q4BufferLayout.swift:29-79). */
typedef struct splosh_q4_layout {
    int64_t rows;
    int64_t logical_k;
    int32_t orientation;           /* splosh_orientation */
    int32_t reserved;
    int64_t packed_words_per_row;
    int64_t row_stride_bytes;
    int64_t row_stride_words;
    int64_t padding_words_per_row;
    int64_t groups_per_row;
    int64_t group_stride;
} splosh_q4_layout;

/* A resident q4 weight: the reference's Q4Handle (Runtime/Engine.swift, bound at
 * engine.metal buffers 0..2). rows = outputs N, inner = K. For TILED128, row_stride_words is
 * ignored (the tiled records are 8 words) and rows % 128 == 0, inner % 64 == 0. */
typedef struct splosh_q4_weight {
    const uint32_t *packed;
    const uint16_t *scales;
    const uint16_t *biases;
    int64_t rows;
    int64_t inner;
    int64_t row_stride_words;
    int32_t order;                 /* splosh_q4_order */
    int32_t reserved;
} splosh_q4_weight;

/* A GGUF Q5_K weight in plane form (Model/GgufPlanes.swift:8-20, geometry :62-74). */
typedef struct splosh_q5k_weight {
    const uint8_t *plane0;
    const uint8_t *plane1;
    const uint8_t *meta;
    int64_t rows;
    int64_t inner;
} splosh_q5k_weight;

/* ---- host helpers (no device work) ------------------------------------------------------ */

/* Q4BufferLayout.init (Quant/Q4BufferLayout.swift:43-79). row_stride_bytes 0 = aligned
 * default; row_alignment 0 = 128. */
int splosh_q4_layout_init(int64_t rows, int64_t logical_k, int orientation, int64_t row_stride_bytes,
                          int64_t row_alignment, splosh_q4_layout *out);
/* Q4BufferLayout.wordIndex / nibbleShift / sidecarIndex (Q4BufferLayout.swift:82-104). */
int splosh_q4_layout_word_index(const splosh_q4_layout *layout, int64_t row, int64_t k, int64_t *out);
int splosh_q4_layout_nibble_shift(const splosh_q4_layout *layout, int64_t row, int64_t k, uint32_t *out);
int splosh_q4_layout_sidecar_index(const splosh_q4_layout *layout, int64_t row, int64_t k, int64_t *out);
/* GemmQ4Shape.init + validate(layout:) (Model/Gemm.swift:13-40). */
int splosh_q4_shape_validate(int64_t rows, int64_t columns, int64_t inner, const splosh_q4_layout *layout);

/* Scratch bytes the GEMM entry points can use for `rows` x `columns` x `inner` (0 when none): fp32
 * partial sums of output bands whose K is split across workgroups. The reference's engine owns
 * its scratch (Runtime/Engine.swift:460-486); here the caller does, and the library allocates
 * nothing. Without a workspace (or with a smaller one) the kernels do not split K: the results
 * agree up to the fp32 summation order, with less parallelism. Calls that share one workspace
 * must be ordered on one stream. The workspace must be zero-filled before its first use: its first
 * 16 KiB hold per-band arrival counters that the kernels return to zero before they exit, and no
 * call writes anything else there, so later calls of any shape, row count or entry point reuse it
 * as it is (zero it again after a call that failed or was aborted). */
size_t splosh_workspace_bytes(int64_t rows, int64_t columns, int64_t inner);

const char *splosh_status_string(int status);
/* The message of the last failure on this thread ("" after success). */
const char *splosh_last_error(void);
const char *splosh_version(void);

/* ---- MLX affine q4 ---------------------------------------------------------------------- */

/* Q4GemmRuntime.dispatch (Runtime/Q4Runtime.swift:94-145) running gemm_q4
 * (Shaders/gemm_q4.metal:31-54): c fp32 [rows][columns], one thread per output, either
 * orientation. Validation is GemmQ4Shape.validate (which requires rowsByK). */
int splosh_gemm_q4(const uint16_t *a, const uint32_t *packed, const uint16_t *scales,
                   const uint16_t *biases, float *c, int64_t rows, int64_t columns, int64_t inner,
                   const splosh_q4_layout *layout, hipStream_t stream);

/* Engine.gemm(w, input:, output:, residual:, rows:) (Runtime/Engine.swift:1652-1806): one
 * projection. residual may be NULL or alias out; it has out's dtype and ldc. */
int splosh_q4_gemm(const splosh_q4_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                   int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                   size_t workspace_bytes, hipStream_t stream);

/* Engine.gemm with `emit` (Runtime/Engine.swift:1652-1806; kernels sp_gemm_q4_nat_m32n128s4_emit and
 * sp_gemm_q4_split_tiled_m16n64p4_emit, Shaders/engine_na.metal:322-473, SpNaEmit :26-36): the
 * residual projection out = residual + a w^T (fp32, residual may be NULL or alias out) that also
 * writes the next RMSNorm-ed GEMM's operand from the same values: values = bf16(out * norm_weight)
 * (RNE, [rows][ld_values]), and per row and per 64 columns the sums of those rounded values and of
 * out * out (fp32 [rows][w->rows / 64]), as splosh_emit_operand computes them. w->rows % 64 == 0.
 * The prefill kernel (AUTO for most shapes from 256 rows, or SPLOSH_KERNEL_PREFILL) writes them from
 * its epilogue, and so does the M <= 64 kernel when SPLOSH_KERNEL_DEQUANT is asked for (rows <= 64);
 * otherwise the GEMM is followed by the operand pass (under AUTO at M <= 64 the faster of the two). */
int splosh_q4_gemm_emit(const splosh_q4_weight *w, const uint16_t *a, int64_t lda, float *out, int64_t ldc,
                        const float *residual, int64_t rows, const uint16_t *norm_weight, uint16_t *values,
                        int64_t ld_values, float *sums, float *squares, int kernel, void *workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* No counterpart in the reference: splosh_q4_gemm for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It takes no
 * workspace and allocates nothing: the kernels use a static scratch array in the library's device
 * memory (8 MiB + 16 KiB per GPU, held until the process ends), enough for the M <= 64 kernel's
 * split-K partials on one weight; a call whose split partials would need more runs unsplit (the
 * same results, one workgroup a column band). All calls on one GPU share that scratch: calls that
 * overlap on one GPU (different streams, or host threads without ordering) race and give wrong
 * results. */
int splosh_q4_gemm_noalloc(const splosh_q4_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                           int out_dtype, const void *residual, int64_t rows, int kernel, hipStream_t stream);

/* Several projections of one activation in one launch: the reference encodes a layer's independent
 * projections (q, k and v of an attention layer; qkv and z of a gated-delta layer) into one
 * concurrent encoder so that they overlap (Runtime/Engine.swift:1402, SploshCore/CommandGraph.swift:
 * 57-62; the GEMMs at Engine.swift:1131-1140). out_i = a @ dequant(w_i)^T for i < count
 * (count <= SPLOSH_MAX_GROUP), each into its own output (row stride ldcs[i], out_dtype), no
 * residual. All weights share inner. Up to 64 rows with TILED128 weights (rows % 64 == 0) the
 * group is one launch of the M <= 64 kernel over the weights' joined column bands, split over the
 * CUs as one call (workspace: splosh_workspace_bytes(rows, sum of the weights' rows, inner));
 * otherwise each weight is its own splosh_q4_gemm call, same results to the path's tolerance. */
#define SPLOSH_MAX_GROUP 8
int splosh_q4_gemm_group(const splosh_q4_weight *weights, int count, const uint16_t *a, int64_t lda,
                         void *const *outs, const int64_t *ldcs, int out_dtype, int64_t rows, int kernel,
                         void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Engine.mlpIn(gate:up:input:output:scratch:rows:) (Runtime/Engine.swift:1911-1966) with the
 * fused lane form sp_mlp_in_tiled_* (Shaders/engine.metal:1987-2055): out = silu(gate(a)) * up(a),
 * both weights read in one pass over a. AUTO as splosh_q4_gemm: 65..128 rows as two calls of at most 64,
 * above that tiled weights take the prefill kernel with both weights in each tile. */
int splosh_q4_mlp_in(const splosh_q4_weight *gate, const splosh_q4_weight *up, const uint16_t *a,
                     int64_t lda, void *out, int64_t ldc, int out_dtype, int64_t rows, int kernel,
                     void *workspace, size_t workspace_bytes, hipStream_t stream);

/* DequantOracle.dequantize (Oracle/DequantOracle.swift:11-25) on the device: out fp32
 * [rows][inner], bit-identical to the CPU reference. */
int splosh_q4_dequant(const splosh_q4_weight *w, float *out, hipStream_t stream);

/* sp_embed_q4 (Shaders/engine.metal:39-57), the embedding lookup on a q4 table (either order):
 * out[i][k] = dequant(w)[tokens[i]][k] for i < count, fp32 (bit-identical to DequantOracle) or
 * bf16 (RNE), row stride ldo. tokens: count uint32 ids on the device; an id >= w->rows gives a
 * row of zeros. */
int splosh_q4_embed(const splosh_q4_weight *w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                    int out_dtype, hipStream_t stream);

/* Converter.tile (Model/Retile.swift:135-153) and its inverse on the device:
 * [row][group][element] <-> [row/128][group][row%128][element]. rows % 128 == 0,
 * element_bytes % 2 == 0. src and dst must not overlap. */
int splosh_tile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes,
                   hipStream_t stream);
int splosh_untile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes,
                     hipStream_t stream);

/* ---- GGUF Q5_K ---------------------------------------------------------------------------- */

/* Engine.gemm on a GGUF weight (Runtime/Engine.swift:1671-1697, kernels
 * Shaders/engine_gguf.metal:82-221 instantiated _q5k at :332-349). AUTO: one row takes the
 * every-CU decode kernel; 2..64 rows the dequant-to-bf16 MFMA kernel (DEQUANT; lda % 8 == 0 and
 * 16-byte aligned activations), 65..128 rows two calls of at most 64; more rows the 256 x 256
 * prefill kernel (PREFILL; also ldc % 4 == 0
 * and 16-byte aligned outputs), else the LDS-tiled kernel (TILE), else the streaming kernel
 * (STREAM). DEQUANT and PREFILL use a workspace of splosh_workspace_bytes(rows, w->rows, w->inner)
 * to split K. Odd alignments fall back to SCALAR. */
int splosh_q5k_gemm(const splosh_q5k_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                    int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                    size_t workspace_bytes, hipStream_t stream);

/* The `heads` forms of the GGUF GEMM kernels (Shaders/engine_gguf.metal:55-72,336-338; chosen by
 * Runtime/Engine.swift:765-779 for the weights in ggufHeadOrder): for the gated-delta out
 * projection, whose inner columns a GGUF file keeps in its own order of the value heads (128
 * columns each; GgufConvert.swift:17-23 leaves them so, since moving columns would re-quantise every
 * block). File head h meets the activations of engine head (heads / key_heads) (h mod key_heads) +
 * h / key_heads (GgufNames.mlxValueHead: 3 (h % 16) + h / 16 for Qwen's 48 heads and 16 key
 * heads). key_heads: a power of two dividing inner / 128. Rows the decode or streaming kernel takes
 * read the activations in that order directly; above that the call first writes a permuted copy of
 * the activations to the end of the workspace, which must then hold
 * splosh_heads_workspace_bytes(rows, w->rows, w->inner) (SPLOSH_ERR_WORKSPACE_TOO_SMALL otherwise).
 * splosh_q4k_gemm_heads is the Q4_K form (plane1 not read). */
int splosh_q5k_gemm_heads(const splosh_q5k_weight *w, int key_heads, const uint16_t *a, int64_t lda, void *out,
                          int64_t ldc, int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                          size_t workspace_bytes, hipStream_t stream);
int splosh_q4k_gemm_heads(const splosh_q5k_weight *w, int key_heads, const uint16_t *a, int64_t lda, void *out,
                          int64_t ldc, int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                          size_t workspace_bytes, hipStream_t stream);
/* The workspace a head-ordered call of any form needs: splosh_workspace_bytes plus the permuted
 * activations (rows x inner bf16) and alignment. */
size_t splosh_heads_workspace_bytes(int64_t rows, int64_t columns, int64_t inner);

/* GgufTensorType.decode for Q5_K (Model/GgufQuant.swift:191-212) read from the planes: out fp32
 * [rows][inner], bit-identical to the CPU reference. */
int splosh_q5k_dequant(const splosh_q5k_weight *w, float *out, hipStream_t stream);

/* GgufPlanes.repack / unpack for Q5_K (Model/GgufPlanes.swift:103-194) on the device.
 * native: rows x (inner / 256) blocks of 176 bytes. */
int splosh_q5k_repack(const uint8_t *native, int64_t rows, int64_t inner, uint8_t *plane0,
                      uint8_t *plane1, uint8_t *meta, hipStream_t stream);
int splosh_q5k_unpack(const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, int64_t rows,
                      int64_t inner, uint8_t *native, hipStream_t stream);

/* ---- GGUF Q4_K -----------------------------------------------------------------------------
 *
 * Q4_K (GgufQuant.swift:44,151,191-212: decodeQ45K without fifth bits, 144-byte blocks) in its
 * GgufPlanes form (GgufPlanes.swift:64: plane0 and meta as for Q5_K, no plane1). The weight is a
 * splosh_q5k_weight whose plane1 is not read (pass NULL). The same kernels as Q5_K. */
int splosh_q4k_gemm(const splosh_q5k_weight *w, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                    int out_dtype, const void *residual, int64_t rows, int kernel, void *workspace,
                    size_t workspace_bytes, hipStream_t stream);
int splosh_q4k_dequant(const splosh_q5k_weight *w, float *out, hipStream_t stream);

/* ---- Other GGUF formats, native blocks --------------------------------------------------------
 *
 * Q8_0 (8), Q3_K (11), Q6_K (14), IQ4_NL (20), IQ3_S (21) and IQ4_XS (23), ggml type ids as in the
 * file, in the blocks a
 * GGUF file holds: `rows` rows of `inner` elements, each row inner / block elements native blocks
 * (GgufQuant.swift:13-48), rows back to back. They replace the reference's staged GGUF kernels
 * for these formats (Engine.swift:1673-1694 dispatching sp_gguf_* by format,
 * engine_gguf.metal:332-349) and GgufTensorType.decode (GgufQuant.swift:136-159).
 *
 * Layout. `gguf_type | SPLOSH_GGUF_ROWS32` (every entry point below) names the same blocks in
 * the ROWS32 order that splosh_gguf_repack_rows32 writes: the 256-element units (one super-block,
 * or eight 32-element blocks) of 32 consecutive rows interleaved -- unit u of row n at byte
 * ((n / 32) (inner / 256) 32 + u 32 + n % 32) x unit bytes -- rows padded to a multiple of 32,
 * inner % 256 == 0. The bytes of every block are the file's; only their order differs. It has no
 * counterpart in the reference (whose GgufPlanes repack serves Q5_K only): the 32 lanes of a
 * wave that read one unit of 32 weight rows read one contiguous run, which the row-major file
 * order scatters over 32 rows (at K17408 -> N5120, M=64: Q8_0 44 -> 33 us, IQ4_XS 39 -> 31).
 *
 * splosh_gguf_gemm: out[m][n] = sum_k a[m][k] w[n][k] (+ residual). Up to a few activation rows
 * (IQ4_NL 3, Q3_K 6, the others 4) a streaming kernel reads the weight once. Up to 64 rows
 * (inner % 256 == 0) the stream-K MFMA kernel of splosh_q4_gemm decodes each weight group once,
 * and 65..128 rows run as two such calls but for Q3_K (where it does not fit, the streaming kernel
 * serves up to eight rows). Above that an LDS-tiled
 * MFMA kernel (inner % 64 == 0) decodes each weight group once per 64 or 128 activation rows. From 256
 * rows (rows % 128 == 0, ldc % 4 == 0, 16-byte aligned outputs) the 256 x 256 prefill kernel
 * decodes each group once per 256 rows. The MFMA kernels split K over workgroups when their work
 * is uneven or their tiles few and a workspace of splosh_workspace_bytes(m, rows, inner) is given
 * (zero-filled before first use; the kernels leave their counters zeroed, so one workspace serves
 * every later call; null: no split).
 * splosh_gguf_dequant: the weight as fp32 [rows][inner], bit-exact with the reference decoder.
 * `native` must be 4-byte aligned (GGUF tensor data is 32-byte aligned).
 * Unsupported types return SPLOSH_ERR_UNSUPPORTED. */
#define SPLOSH_GGUF_ROWS32 0x100

/* The ROWS32 order of a native-block weight (layout above): out holds
 * splosh_gguf_rows32_bytes(gguf_type, rows, inner) bytes (the padding rows zero); 0 when the type
 * or shape has no ROWS32 form (inner % 256 != 0). */
size_t splosh_gguf_rows32_bytes(int gguf_type, int64_t rows, int64_t inner);
int splosh_gguf_repack_rows32(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, uint8_t *out,
                              hipStream_t stream);

int splosh_gguf_gemm(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, const uint16_t *a,
                     int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual, int64_t m,
                     void *workspace, size_t workspace_bytes, hipStream_t stream);
/* splosh_gguf_gemm with the weight's inner columns in a GGUF file's value-head order: the `heads`
 * form described at splosh_q5k_gemm_heads. */
int splosh_gguf_gemm_heads(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, int key_heads,
                           const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                           int64_t m, void *workspace, size_t workspace_bytes, hipStream_t stream);
int splosh_gguf_dequant(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, float *out,
                        hipStream_t stream);

/* sp_gguf_embed (Shaders/engine_gguf.metal:302-318, bound at Engine.swift:400 and dispatched at
 * :1612-1625), the embedding lookup on a GGUF table: out[i][k] = decode(w)[tokens[i]][k] for
 * i < count, fp32 (bit-identical to GgufTensorType.decode) or bf16 (RNE), row stride ldo. tokens:
 * count uint32 ids on the device; an id >= rows gives a row of zeros. splosh_q5k_embed /
 * splosh_q4k_embed take the plane form, splosh_gguf_embed the native blocks of the types above. */
int splosh_q5k_embed(const splosh_q5k_weight *w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                     int out_dtype, hipStream_t stream);
int splosh_q4k_embed(const splosh_q5k_weight *w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                     int out_dtype, hipStream_t stream);
int splosh_gguf_embed(int gguf_type, const uint8_t *native, int64_t rows, int64_t inner, const uint32_t *tokens,
                      int64_t count, void *out, int64_t ldo, int out_dtype, hipStream_t stream);
int splosh_q4k_repack(const uint8_t *native, int64_t rows, int64_t inner, uint8_t *plane0, uint8_t *meta,
                      hipStream_t stream);
int splosh_q4k_unpack(const uint8_t *plane0, const uint8_t *meta, int64_t rows, int64_t inner, uint8_t *native,
                      hipStream_t stream);

/* ---- Operand producers: the steps either side of a GEMM -------------------------------------
 *
 * Each writes a GEMM operand as bf16 (RNE) [rows][dim] (row stride ld_out) plus, per row and per
 * 64 columns, the fp32 sum of the rounded values ([rows][dim / 64], dense). dim % 64 == 0; fp32
 * inputs 16-byte aligned with row strides % 4 == 0; the bf16 output 8-byte aligned with
 * ld_out % 4 == 0. */

/* sp_na_prepare (Shaders/engine_na.metal:38-56): fp32 activations -> the bf16 operand and its sums. */
int splosh_prepare_operand(const float *x, int64_t ldx, int64_t rows, int64_t dim, uint16_t *out,
                           int64_t ld_out, float *sums, hipStream_t stream);

/* sp_silu_mul_na (Shaders/engine.metal:200-218): the down projection's operand
 * bf16(silu(gate s) * (up s)) and its sums, s = row_inv[row] (the deferred RMSNorm scale of the
 * norm that fed both projections; NULL: 1). gate and up share the row stride ld. */
int splosh_silu_mul_operand(const float *gate, const float *up, int64_t ld, const float *row_inv, int64_t rows,
                            int64_t dim, uint16_t *out, int64_t ld_out, float *sums, hipStream_t stream);

/* The operand a residual projection emits for the next RMSNorm-ed GEMM (SpNaEmit,
 * Shaders/engine_na.metal:26-36, epilogue :365-411): from the fp32 hidden state h (the projection's
 * output after its residual add) and the norm's bf16 weight: values = bf16(h * weight[col]), their
 * sums, and squares = per-64 sums of h * h. The norm's row scale is applied later (a GEMM is linear
 * in its input), from splosh_row_inv. weight: dim bf16 values, 8-byte aligned. */
int splosh_emit_operand(const float *hidden, int64_t ld_hidden, const uint16_t *norm_weight, int64_t rows,
                        int64_t dim, uint16_t *values, int64_t ld_values, float *sums, float *squares,
                        hipStream_t stream);

/* sp_row_inv (Shaders/engine.metal:222-233): inv[row] = 1 / sqrt(sum(squares[row]) / dim + eps),
 * squares [rows][groups] dense. */
int splosh_row_inv(const float *squares, int64_t rows, int64_t groups, int64_t dim, float eps, float *inv,
                   hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SPLOSH_Q4_H */
