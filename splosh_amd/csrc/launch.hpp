// launch.hpp -- host-side launchers of the kernels, called by the C ABI in api.cpp after it has
// validated every argument. They enqueue on `stream` and return hipGetLastError().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/splosh_q4.h"

namespace splosh {

// Kernel-shape choice of the streaming kernels.
struct StreamPlan {
    int mb;        // 16-row blocks per workgroup (1, 2 or 4)
    int j;         // 16-column blocks per wave (1, 2 or 4)
    int sk;        // waves per workgroup, each a slice of the K groups (1..16)
    int rpl;       // accumulator registers updated per block (1, 2 or 4)
    int row_chunks;
    int col_blocks;
};

hipError_t launch_gemm_q4_scalar(const uint16_t *a, const uint32_t *packed, const uint16_t *scales,
                                 const uint16_t *biases, float *c, int64_t rows, int64_t columns,
                                 int64_t inner, int64_t stride_words, int orientation,
                                 int64_t groups_per_row, hipStream_t stream);

hipError_t launch_q4_dequant(const splosh_q4_weight &w, float *out, hipStream_t stream);

// Rows tokens[i] of the dequantized weight (the q4 embedding lookup).
hipError_t launch_q4_embed(const splosh_q4_weight &w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                           int out_dtype, hipStream_t stream);

hipError_t launch_tile128(const void *src, void *dst, int64_t rows, int64_t groups,
                          int64_t element_bytes, bool inverse, hipStream_t stream);

// Generic q4 GEMM of any shape: one thread per output, weights in either order.
hipError_t launch_q4_gemm_scalar(const splosh_q4_weight &w, const splosh_q4_weight *up,
                                 const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                                 const void *residual, int64_t rows, hipStream_t stream);

// `units` is the number of K slices the waves may split (q4 groups of 64, Q5_K blocks of 256).
StreamPlan plan_stream(int64_t rows, int64_t columns, int64_t units, bool mlp, int max_j);

hipError_t launch_q4_stream(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                            const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                            const void *residual, int64_t rows, hipStream_t stream);

// The lane-per-row decode kernel for one or two rows (lanes.hip).
bool lanes_fit(int64_t rows, int64_t columns, int64_t inner, int64_t stride_words, bool mlp);
StreamPlan plan_lanes(int64_t rows, int64_t columns, int64_t groups, bool mlp);
hipError_t launch_q4_lanes(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                           const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                           const void *residual, int64_t rows, hipStream_t stream);

// The decode kernel on every CU for one to four rows of tiled weights (decode.hip): a workgroup a
// block of 16 or 32 output rows over the whole of K. With a workspace of decode_workspace_bytes
// (zero: not needed) the last round of blocks is split over K so that every CU gets the same work;
// without one every block is whole.
bool decode_fits(int64_t rows, int64_t columns, int64_t inner, int order);
size_t decode_workspace_bytes(int64_t rows, int64_t columns, int64_t inner, int nw);
hipError_t launch_q4_decode(const splosh_q4_weight &w, const splosh_q4_weight *up, const uint16_t *a, int64_t lda,
                            void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                            void *workspace, size_t workspace_bytes, hipStream_t stream);

// The dequant-to-bf16 weight-streaming MFMA kernel for up to 64 rows (mma.hip). Split K over
// workgroups (stream-K) uses a caller workspace of mma_workspace_bytes(); without one every band
// is computed whole by one workgroup.
struct MmaPlan {
    int fm;            // 32-row blocks (1 or 2)
    int bands;         // column bands of 64
    int grid;          // workgroups
    int dp_bands;      // bands computed whole (a multiple of grid)
    int64_t sk_units;  // (band, unit) pairs of the other bands, split evenly over the grid
};
bool mma_fits(int64_t rows, int64_t columns, int64_t inner, int64_t stride_words, int64_t lda);
// `unit_elems`: K elements of one unit (64 for q4 groups, 256 for Q5_K blocks).
MmaPlan plan_mma(int64_t rows, int64_t columns, int64_t groups, bool mlp, size_t workspace_bytes,
                 int64_t unit_elems = 64);
size_t mma_workspace_bytes(int64_t rows, int64_t columns, int64_t groups, bool mlp);
hipError_t launch_q4_mma_group(const MmaPlan &plan, const splosh_q4_weight *w, int count, void *const *outs,
                               const int64_t *ldcs, const uint16_t *a, int64_t lda, int out_dtype, int64_t rows,
                               void *workspace, hipStream_t stream);

// The next RMSNorm's operand a residual projection emits (SpNaEmit, engine_na.metal:26-36).
struct EmitOperand {
    const uint16_t *norm_weight;  // bf16 [n]
    uint16_t *values;             // bf16 [rows][ldv]
    int64_t ldv;
    float *sums, *squares;        // fp32 [rows][n / 64]
};
// emit: null, or the operand to write from the epilogue (single weight, fp32 output, n % 64 == 0).
hipError_t launch_q4_mma(const MmaPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                         const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                         int64_t rows, void *workspace, hipStream_t stream, const EmitOperand *emit = nullptr);

// GGUF Q8_0 / Q6_K / IQ4_NL / IQ4_XS in native blocks (gguf_native.hip). The launchers below
// take the type id with the layout flag (SPLOSH_GGUF_ROWS32) and split it with gguf_layout.
int gguf_native_block(int type, int *elems, int *bytes);
inline bool gguf_layout(int &type) {
    const bool rows32 = (type & SPLOSH_GGUF_ROWS32) != 0;
    type &= 0xFF;
    return rows32;
}
hipError_t launch_gguf_repack_rows32(int type, const uint8_t *native, int64_t rows, int64_t inner, uint8_t *out,
                                     hipStream_t stream);
hipError_t launch_gguf_dequant(int type, const uint8_t *w, int64_t rows, int64_t inner, float *dense,
                               hipStream_t stream);
hipError_t launch_gguf_embed(int type, const uint8_t *w, int64_t rows, int64_t inner, const uint32_t *tokens,
                             int64_t count, void *out, int64_t ldo, int out_dtype, hipStream_t stream);
// The embedding lookup on Q5_K / Q4_K planes (plane1 null: Q4_K).
hipError_t launch_q5k_embed(const splosh_q5k_weight &w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                            int out_dtype, hipStream_t stream);
// The LDS-tiled MFMA GEMM for GGUF weights (gguf_tile.hip): type a native-block ggml id, or 13 / 12
// for Q5_K / Q4_K planes (w = plane0). Needs inner % 64 == 0 and lda % 8 == 0. With a workspace
// (zero-filled before first use, left zeroed) it splits K over workgroups when the tiles are few.
bool gguf_tile_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda);
hipError_t launch_gguf_tile(int type, const uint8_t *w, const uint8_t *plane1, const uint8_t *meta, int64_t rows_w,
                            int64_t inner, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                            const void *residual, int64_t m, void *workspace, size_t workspace_bytes,
                            hipStream_t stream);
// Workspace that lets the tiled kernel split K (0: it would not split): arrival counters in the
// first 16 KiB, fp32 partials after.
size_t gguf_tile_workspace_bytes(int64_t rows, int64_t n, int64_t inner);
// dst[m][k] = a[m][column of k in the engine's value-head order] (head_group), m rows of `inner`
// elements: the activations of a head-ordered weight for the kernels that read them unpermuted.
hipError_t launch_head_gather(const uint16_t *a, int64_t lda, int64_t m, int64_t inner, int hs, int vph,
                              uint16_t *dst, hipStream_t stream);
hipError_t launch_gguf_gemv(int type, const uint8_t *w, int64_t rows, int64_t inner, const uint16_t *a, int64_t lda,
                            void *out, int64_t ldc, int out_dtype, const void *residual, int64_t m,
                            hipStream_t stream, int hs = -1, int vph = 0);

// One wide weight as the pair of its column halves (plan: columns / 2, mlp = true), where
// mma_split says it pays.
bool mma_split(const splosh_q4_weight &w);
hipError_t launch_q4_mma_split(const MmaPlan &plan, const splosh_q4_weight &w, const uint16_t *a, int64_t lda,
                               void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                               void *workspace, hipStream_t stream);

// The same kernel over Q5_K planes; the plan's units are 256-element blocks.
bool q5k_mma_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda);
hipError_t launch_q5k_mma(const MmaPlan &plan, const splosh_q5k_weight &w, const uint16_t *a, int64_t lda, void *out,
                          int64_t ldc, int out_dtype, const void *residual, int64_t rows, void *workspace,
                          hipStream_t stream);

// The same kernel over GGUF native blocks (Q8_0, IQ4_NL, Q6_K, Q3_K, IQ3_S, IQ4_XS); the plan's
// units are 256 elements of K.
bool gguf_mma_fits(int type, int64_t rows, int64_t columns, int64_t inner, int64_t lda);
hipError_t launch_gguf_mma(const MmaPlan &plan, int type, const uint8_t *native, int64_t columns, int64_t inner,
                           const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                           int64_t rows, void *workspace, hipStream_t stream);

// Sums split-K partials [splits][nw][rows][n] in slice order and applies the epilogue
// (silu(g) * u for nw = 2, then the optional residual, then the output conversion).
hipError_t launch_splitk_finish(const float *partial, int splits, int nw, int64_t rows, int64_t n, void *out,
                                int64_t ldc, int out_dtype, const void *residual, hipStream_t stream);

// The LDS-tiled dequant-to-bf16 MFMA GEMM for any rows (tile.hip). Split K uses a caller workspace
// of tile_workspace_bytes(); without one (or a smaller one) the plan does not split.
struct TilePlan {
    int kind;     // tile shape: 0 = 64 x 64, 1 = 256 x 256, 2 = 128 x 128
    int grid_m, grid_n;
    int splits;   // K slices (1 = no workspace use)
};
bool tile_fits(int64_t rows, int64_t columns, int64_t lda, int64_t stride_words);
TilePlan plan_tile(int64_t rows, int64_t columns, int64_t groups, bool mlp, size_t workspace_bytes);
size_t tile_workspace_bytes(int64_t rows, int64_t columns, int64_t groups, bool mlp);
hipError_t launch_q4_tile(const TilePlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                          const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                          int64_t rows, void *workspace, hipStream_t stream);

// The prefill kernel for one tiled weight (prefill.hip): 256 x 256 tiles, two waves per SIMD,
// weights dequantized once a workgroup into LDS; stream-K over a caller workspace of prefill_workspace_bytes().
struct PrefillPlan {
    int mblocks;       // row blocks of 256
    int tiles;
    int grid;
    int dp_tiles;      // tiles computed whole (a multiple of grid)
    int64_t sk_units;  // (tile, group) pairs of the other tiles, split evenly over the grid
};
bool prefill_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda, int64_t ldc);
PrefillPlan plan_prefill(int64_t rows, int64_t columns, int64_t groups, size_t workspace_bytes);
size_t prefill_workspace_bytes(int64_t rows, int64_t columns, int64_t groups);
// emit: null, or the operand to write from the epilogue (fp32 output, n % 64 == 0).
hipError_t launch_q4_prefill(const PrefillPlan &plan, const splosh_q4_weight &w, const uint16_t *a, int64_t lda,
                             void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                             void *workspace, hipStream_t stream, const EmitOperand *emit = nullptr);
// Fused gate+up (silu(g) * u) over two TILED128 weights of one geometry: tiles of 128 columns of
// each; plan with plan_prefill(rows, 2 * columns, groups, ...).
hipError_t launch_q4_prefill_mlp(const PrefillPlan &plan, const splosh_q4_weight &gate, const splosh_q4_weight &up,
                                 const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, int64_t rows,
                                 void *workspace, hipStream_t stream);
// The same kernel over Q5_K (fifth) or Q4_K planes: K a multiple of 256.
bool q5k_prefill_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda, int64_t ldc);
hipError_t launch_q5k_prefill(const PrefillPlan &plan, const splosh_q5k_weight &w, bool fifth, const uint16_t *a,
                              int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                              void *workspace, hipStream_t stream);
// And over the GGUF native blocks (ggml type ids 8, 11, 14, 20, 21, 23): K a multiple of 64 and of
// the block.
bool gguf_prefill_fits(int type, int64_t rows, int64_t columns, int64_t inner, int64_t lda, int64_t ldc);
hipError_t launch_gguf_prefill(const PrefillPlan &plan, int type, const uint8_t *native, int64_t rows_w,
                               int64_t inner, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                               const void *residual, int64_t rows, void *workspace, hipStream_t stream);

// The decode kernel for one activation row of Q5_K planes (q5k_decode.hip).
bool q5k_decode_fits(int64_t rows, int64_t columns, int64_t inner);
size_t q5k_decode_workspace_bytes(int64_t rows, int64_t columns, int64_t inner);
hipError_t launch_q5k_decode(const splosh_q5k_weight &w, const uint16_t *a, void *out, int out_dtype,
                             const void *residual, void *workspace, size_t workspace_bytes, hipStream_t stream,
                             int hs = -1, int vph = 0);

// Operand producers (operand.hip).
hipError_t launch_prepare_operand(const float *x, int64_t ldx, int64_t rows, int64_t dim, uint16_t *out, int64_t ldo,
                                  float *sums, hipStream_t stream);
hipError_t launch_silu_mul_operand(const float *gate, const float *up, int64_t ld, const float *row_inv, int64_t rows,
                                   int64_t dim, uint16_t *out, int64_t ldo, float *sums, hipStream_t stream);
hipError_t launch_emit_operand(const float *hidden, int64_t ldh, const uint16_t *weight, int64_t rows, int64_t dim,
                               uint16_t *values, int64_t ldv, float *sums, float *squares, hipStream_t stream);
hipError_t launch_row_inv(const float *squares, int64_t rows, int64_t groups, int64_t dim, float eps, float *inv,
                          hipStream_t stream);

hipError_t launch_q5k_dequant(const splosh_q5k_weight &w, float *out, hipStream_t stream);
// fifth = false: Q4_K (144-byte blocks, no plane1).
hipError_t launch_q5k_repack(const uint8_t *native, int64_t rows, int64_t inner, uint8_t *p0,
                             uint8_t *p1, uint8_t *meta, bool inverse, hipStream_t stream, bool fifth = true);
hipError_t launch_q5k_stream(const StreamPlan &plan, const splosh_q5k_weight &w, const uint16_t *a,
                             int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                             int64_t rows, hipStream_t stream);
hipError_t launch_q5k_gemm_scalar(const splosh_q5k_weight &w, const uint16_t *a, int64_t lda, void *out,
                                  int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                                  hipStream_t stream);

}  // namespace splosh
