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

// The 32x32x16 MFMA streaming kernel for rows <= 32 (stream32.hip).
StreamPlan plan_stream32(int64_t rows, int64_t columns, int64_t groups, bool mlp);
hipError_t launch_q4_stream32(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                              const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                              const void *residual, int64_t rows, hipStream_t stream);

// The decode kernel for rows <= 8 with activations staged in LDS (gemv.hip).
bool gemv_fits(int64_t rows, int64_t inner);
StreamPlan plan_gemv(int64_t rows, int64_t columns, int64_t groups, bool mlp);
hipError_t launch_q4_gemv(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                          const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                          const void *residual, int64_t rows, hipStream_t stream);

// The lane-per-row decode kernel for one or two rows (lanes.hip).
bool lanes_fit(int64_t rows, int64_t columns, int64_t inner, int64_t stride_words, bool mlp);
StreamPlan plan_lanes(int64_t rows, int64_t columns, int64_t groups, bool mlp);
hipError_t launch_q4_lanes(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                           const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                           const void *residual, int64_t rows, hipStream_t stream);

hipError_t launch_q5k_dequant(const splosh_q5k_weight &w, float *out, hipStream_t stream);
hipError_t launch_q5k_repack(const uint8_t *native, int64_t rows, int64_t inner, uint8_t *p0,
                             uint8_t *p1, uint8_t *meta, bool inverse, hipStream_t stream);
hipError_t launch_q5k_stream(const StreamPlan &plan, const splosh_q5k_weight &w, const uint16_t *a,
                             int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                             int64_t rows, hipStream_t stream);
hipError_t launch_q5k_gemm_scalar(const splosh_q5k_weight &w, const uint16_t *a, int64_t lda, void *out,
                                  int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                                  hipStream_t stream);

}  // namespace splosh
