// q4_basic.hip -- the simple q4 kernels: the oracle-grade one-thread-per-output GEMM, the
// fp32 dequantizer, the 128-row retile and a generic scalar GEMM used for shapes the streaming
// kernels do not take. None of these is on the measured path; they are exact references on the
// device and fallbacks for odd shapes.
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

// gemm_q4 (Shaders/gemm_q4.metal:31-54): c[row][col] = sum_k bf16(a) * (s * q + b), fp32,
// sequential in k. orientation 0 = rowsByK, 1 = kByColumns (gemm_q4.metal:21-29).
__global__ void __launch_bounds__(256)
gemm_q4_scalar_kernel(const uint16_t *__restrict__ a, const uint32_t *__restrict__ packed,
                      const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases,
                      float *__restrict__ c, int64_t rows, int64_t columns, int64_t inner,
                      int64_t stride_words, int orientation, int64_t groups_per_row) {
    const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t row = blockIdx.y;
    if (col >= columns || row >= rows) return;
    float sum = 0.0f;
    for (int64_t k = 0; k < inner; ++k) {
        const int64_t wi = orientation == 0 ? col * stride_words + k / 8 : k * stride_words + col / 8;
        const uint32_t shift = orientation == 0 ? (uint32_t)(k % 8) * 4u : (uint32_t)(col % 8) * 4u;
        const uint32_t q = (packed[wi] >> shift) & 0xfu;
        const int64_t sc = col * groups_per_row + k / kGroup;
        const float weight = bf16_bits_to_f32(scales[sc]) * (float)q + bf16_bits_to_f32(biases[sc]);
        sum += bf16_bits_to_f32(a[row * inner + k]) * weight;
    }
    c[row * columns + col] = sum;
}

hipError_t launch_gemm_q4_scalar(const uint16_t *a, const uint32_t *packed, const uint16_t *scales,
                                 const uint16_t *biases, float *c, int64_t rows, int64_t columns,
                                 int64_t inner, int64_t stride_words, int orientation,
                                 int64_t groups_per_row, hipStream_t stream) {
    dim3 grid((unsigned)((columns + 255) / 256), (unsigned)rows);
    hipLaunchKernelGGL(gemm_q4_scalar_kernel, grid, dim3(256), 0, stream, a, packed, scales, biases, c,
                       rows, columns, inner, stride_words, orientation, groups_per_row);
    return hipGetLastError();
}

// Word index and sidecar index of (row n, word wi = k / 8) in either order.
__device__ __forceinline__ void q4_address(const splosh_q4_weight &w, int64_t n, int64_t wi, int64_t groups,
                                           int64_t *word, int64_t *sidecar) {
    const int64_t g = wi / 8;
    if (w.order == SPLOSH_Q4_TILED128) {
        const int64_t rec = tiled_record(n, g, groups);
        *word = rec * 8 + (wi % 8);
        *sidecar = rec;
    } else {
        *word = n * w.row_stride_words + wi;
        *sidecar = n * groups + g;
    }
}

// DequantOracle.dequantize (Oracle/DequantOracle.swift:11-25): one thread per packed word,
// eight fp32 values s * q + b. s * q is exact, so the one rounding equals the CPU's.
__global__ void __launch_bounds__(256)
q4_dequant_kernel(splosh_q4_weight w, float *__restrict__ out) {
    const int64_t words_per_row = (w.inner + 7) / 8;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= w.rows * words_per_row) return;
    const int64_t n = idx / words_per_row, wi = idx % words_per_row;
    const int64_t groups = (w.inner + kGroup - 1) / kGroup;
    int64_t word_index, sidecar;
    q4_address(w, n, wi, groups, &word_index, &sidecar);
    const uint32_t word = w.packed[word_index];
    const float s = bf16_bits_to_f32(w.scales[sidecar]);
    const float b = bf16_bits_to_f32(w.biases[sidecar]);
    float *dst = out + n * w.inner + wi * 8;
    const int64_t count = w.inner - wi * 8 < 8 ? w.inner - wi * 8 : 8;
    for (int i = 0; i < count; ++i) dst[i] = __builtin_fmaf(s, (float)((word >> (4 * i)) & 0xfu), b);
}

hipError_t launch_q4_dequant(const splosh_q4_weight &w, float *out, hipStream_t stream) {
    const int64_t total = w.rows * ((w.inner + 7) / 8);
    hipLaunchKernelGGL(q4_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, w, out);
    return hipGetLastError();
}

// sp_embed_q4 (engine.metal:39-57): out[i] = dequant(w)[tokens[i]] for each token, thread per
// (token, code word); the same one-rounding s * q + b as the dequant above. A token past the
// weight's rows gives a row of zeros (nothing is read out of bounds).
__global__ void __launch_bounds__(256)
q4_embed_kernel(splosh_q4_weight w, const uint32_t *__restrict__ tokens, int64_t count, void *__restrict__ out,
                int64_t ldo, int out_dtype) {
    const int64_t words_per_row = (w.inner + 7) / 8;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= count * words_per_row) return;
    const int64_t i = idx / words_per_row, wi = idx % words_per_row;
    const int64_t token = tokens[i];
    const bool live = token < w.rows;
    const int64_t groups = (w.inner + kGroup - 1) / kGroup;
    float v[8];
    if (live) {
        int64_t word_index, sidecar;
        q4_address(w, token, wi, groups, &word_index, &sidecar);
        const uint32_t word = w.packed[word_index];
        const float s = bf16_bits_to_f32(w.scales[sidecar]);
        const float b = bf16_bits_to_f32(w.biases[sidecar]);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(s, (float)((word >> (4 * e)) & 0xfu), b);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    }
    const int64_t n = w.inner - wi * 8 < 8 ? w.inner - wi * 8 : 8;
    if (out_dtype == SPLOSH_F32) {
        float *dst = (float *)out + i * ldo + wi * 8;
        for (int e = 0; e < n; ++e) dst[e] = v[e];
    } else {
        uint16_t *dst = (uint16_t *)out + i * ldo + wi * 8;
        for (int e = 0; e < n; ++e) dst[e] = f32_to_bf16(v[e]);
    }
}

hipError_t launch_q4_embed(const splosh_q4_weight &w, const uint32_t *tokens, int64_t count, void *out, int64_t ldo,
                           int out_dtype, hipStream_t stream) {
    const int64_t total = count * ((w.inner + 7) / 8);
    hipLaunchKernelGGL(q4_embed_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, w, tokens, count,
                       out, ldo, out_dtype);
    return hipGetLastError();
}

// Converter.tile (Model/Retile.swift:135-153) moving 16-bit units: thread per destination unit.
__global__ void __launch_bounds__(256)
tile128_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst, int64_t rows, int64_t groups,
               int64_t units, int inverse) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = rows * groups * units;
    if (idx >= total) return;
    const int64_t u = idx % units;
    const int64_t rec = idx / units;             // tiled record index
    const int64_t n_in_tile = rec % kTileRows;
    const int64_t g = (rec / kTileRows) % groups;
    const int64_t tile = rec / (kTileRows * groups);
    const int64_t row = tile * kTileRows + n_in_tile;
    const int64_t row_major = (row * groups + g) * units + u;
    if (inverse) dst[row_major] = src[idx];
    else dst[idx] = src[row_major];
}

hipError_t launch_tile128(const void *src, void *dst, int64_t rows, int64_t groups, int64_t element_bytes,
                          bool inverse, hipStream_t stream) {
    const int64_t units = element_bytes / 2;
    const int64_t total = rows * groups * units;
    hipLaunchKernelGGL(tile128_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       (const uint16_t *)src, (uint16_t *)dst, rows, groups, units, inverse ? 1 : 0);
    return hipGetLastError();
}

// Write one output element in the caller's dtype, adding the residual first when given.
__device__ __forceinline__ void store_out(void *out, int64_t index, int out_dtype, const void *residual, float v) {
    if (out_dtype == SPLOSH_F32) {
        if (residual) v += ((const float *)residual)[index];
        ((float *)out)[index] = v;
    } else {
        if (residual) v += bf16_bits_to_f32(((const uint16_t *)residual)[index]);
        ((uint16_t *)out)[index] = f32_to_bf16(v);
    }
}

__device__ float q4_dot_scalar(const splosh_q4_weight &w, const uint16_t *a_row, int64_t n) {
    const int64_t groups = (w.inner + kGroup - 1) / kGroup;
    float sum = 0.0f;
    for (int64_t k = 0; k < w.inner; ++k) {
        int64_t word_index, sidecar;
        q4_address(w, n, k / 8, groups, &word_index, &sidecar);
        const uint32_t q = (w.packed[word_index] >> (4 * (k % 8))) & 0xfu;
        const float weight = bf16_bits_to_f32(w.scales[sidecar]) * (float)q + bf16_bits_to_f32(w.biases[sidecar]);
        sum += bf16_bits_to_f32(a_row[k]) * weight;
    }
    return sum;
}

// Generic q4 GEMM / fused gate+up for shapes outside the streaming kernels' domain.
__global__ void __launch_bounds__(256)
q4_gemm_scalar_kernel(splosh_q4_weight w, splosh_q4_weight up, int has_up, const uint16_t *__restrict__ a,
                      int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows) {
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (n >= w.rows || m >= rows) return;
    const uint16_t *a_row = a + m * lda;
    float v = q4_dot_scalar(w, a_row, n);
    if (has_up) v = silu(v) * q4_dot_scalar(up, a_row, n);
    store_out(out, m * ldc + n, out_dtype, residual, v);
}

hipError_t launch_q4_gemm_scalar(const splosh_q4_weight &w, const splosh_q4_weight *up, const uint16_t *a,
                                 int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                                 int64_t rows, hipStream_t stream) {
    dim3 grid((unsigned)((w.rows + 255) / 256), (unsigned)rows);
    hipLaunchKernelGGL(q4_gemm_scalar_kernel, grid, dim3(256), 0, stream, w, up ? *up : w, up ? 1 : 0, a, lda,
                       out, ldc, out_dtype, residual, rows);
    return hipGetLastError();
}

}  // namespace splosh
