// operand.hip -- the steps either side of a q4 GEMM that produce its bf16 operand.
//
// The reference feeds every projection a bf16 activation operand together with the per-64 sums
// of its rounded values (the affine term of a q4 group is bias * sum(a)): sp_na_prepare turns an
// fp32 activation into that form (engine_na.metal:38-56), sp_silu_mul_na turns the gate and up
// projections into the down projection's operand (engine.metal:200-218), a residual projection
// emits the next RMSNorm-ed operand -- hidden * norm weight as bf16, its sums, and the per-64 sums
// of hidden^2 the norm's row scale comes from (engine_na.metal:26-36, 365-411) -- and sp_row_inv
// turns those squares into the row scale (engine.metal:222-233).
//
// All four are elementwise passes bound by HBM. A thread takes four consecutive columns (one
// 16-byte fp32 load per input, one 8-byte bf16 store), sixteen threads a 64-column group; the
// group's sums meet in four xor shuffles. Rows are contiguous runs of whole groups, so a group
// never straddles two rows.
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

constexpr int kOperandThreads = 256;

// Sum over the 16 lanes of a group (lanes 16 i .. 16 i + 15 of the wave).
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m, 16);
    return v;
}

__device__ __forceinline__ float rounded(uint32_t bits16) { return bf16_bits_to_f32(bits16 & 0xffffu); }

// x / (1 + exp(-x)) with a true division (engine.metal:25): these passes are memory bound, so
// the exact form costs nothing.
__device__ __forceinline__ float silu_exact(float x) { return x / (1.0f + expf(-x)); }

struct OperandArgs {
    const float *a;          // prepare: input; silu: gate; emit: hidden
    const float *b;          // silu: up
    const float *row_inv;    // silu: per-row scale or null
    const uint16_t *weight;  // emit: norm weight (bf16)
    int64_t lda, ldb, ldo;   // row strides (elements) of a, b and the bf16 output
    int64_t rows, dim;
    uint16_t *out;
    float *sums, *squares;   // [rows][dim / 64]
};

// MODE 0: prepare, 1: silu * mul, 2: emit.
template <int MODE>
__global__ void __launch_bounds__(kOperandThreads)
operand_kernel(OperandArgs args) {
    const int64_t quads = args.dim / 4;
    const int64_t q = (int64_t)blockIdx.x * kOperandThreads + threadIdx.x;
    const bool live = q < args.rows * quads;
    const int64_t row = live ? q / quads : 0, col = live ? (q % quads) * 4 : 0;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f}, sq = 0.0f;
    if (live) {
        const f32x4 x = *(const f32x4 *)(args.a + row * args.lda + col);
        if constexpr (MODE == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = x[e];
        } else if constexpr (MODE == 1) {
            const f32x4 u = *(const f32x4 *)(args.b + row * args.ldb + col);
            const float s = args.row_inv ? args.row_inv[row] : 1.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = silu_exact(x[e] * s) * (u[e] * s);
        } else {
            const u32x2 w = *(const u32x2 *)(args.weight + col);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t wb = (e & 1) ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu;
                v[e] = x[e] * bf16_bits_to_f32(wb);
                sq = __builtin_fmaf(x[e], x[e], sq);
            }
        }
    }
    const uint32_t lo = f32x2_to_bf16x2(v[0], v[1]), hi = f32x2_to_bf16x2(v[2], v[3]);
    float s = (rounded(lo) + rounded(lo >> 16)) + (rounded(hi) + rounded(hi >> 16));
    s = group16_sum(s);
    if constexpr (MODE == 2) sq = group16_sum(sq);
    if (!live) return;
    *(u32x2 *)(args.out + row * args.ldo + col) = u32x2{lo, hi};
    if ((threadIdx.x & 15) == 0) {
        const int64_t index = row * (args.dim / 64) + col / 64;
        args.sums[index] = s;
        if constexpr (MODE == 2) args.squares[index] = sq;
    }
}

// One wave a row: the row's group squares summed, then 1 / sqrt(mean + eps).
__global__ void __launch_bounds__(64)
row_inv_kernel(const float *__restrict__ squares, int64_t groups, int64_t dim, float eps, float *__restrict__ inv) {
    const int64_t row = blockIdx.x;
    float t = 0.0f;
    for (int64_t g = threadIdx.x; g < groups; g += 64) t += squares[row * groups + g];
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) t += __shfl_xor(t, m, 64);
    if (threadIdx.x == 0) inv[row] = 1.0f / sqrtf(t / (float)dim + eps);
}

template <int MODE>
static hipError_t launch_operand_mode(const OperandArgs &args, hipStream_t stream) {
    const int64_t threads = args.rows * (args.dim / 4);
    const int64_t blocks = (threads + kOperandThreads - 1) / kOperandThreads;
    hipLaunchKernelGGL(operand_kernel<MODE>, dim3((unsigned)blocks), dim3(kOperandThreads), 0, stream, args);
    return hipGetLastError();
}

hipError_t launch_prepare_operand(const float *x, int64_t ldx, int64_t rows, int64_t dim, uint16_t *out, int64_t ldo,
                                  float *sums, hipStream_t stream) {
    OperandArgs a{x, nullptr, nullptr, nullptr, ldx, 0, ldo, rows, dim, out, sums, nullptr};
    return launch_operand_mode<0>(a, stream);
}

hipError_t launch_silu_mul_operand(const float *gate, const float *up, int64_t ld, const float *row_inv, int64_t rows,
                                   int64_t dim, uint16_t *out, int64_t ldo, float *sums, hipStream_t stream) {
    OperandArgs a{gate, up, row_inv, nullptr, ld, ld, ldo, rows, dim, out, sums, nullptr};
    return launch_operand_mode<1>(a, stream);
}

hipError_t launch_emit_operand(const float *hidden, int64_t ldh, const uint16_t *weight, int64_t rows, int64_t dim,
                               uint16_t *values, int64_t ldv, float *sums, float *squares, hipStream_t stream) {
    OperandArgs a{hidden, nullptr, nullptr, weight, ldh, 0, ldv, rows, dim, values, sums, squares};
    return launch_operand_mode<2>(a, stream);
}

hipError_t launch_row_inv(const float *squares, int64_t rows, int64_t groups, int64_t dim, float eps, float *inv,
                          hipStream_t stream) {
    hipLaunchKernelGGL(row_inv_kernel, dim3((unsigned)rows), dim3(64), 0, stream, squares, groups, dim, eps, inv);
    return hipGetLastError();
}

}  // namespace splosh
