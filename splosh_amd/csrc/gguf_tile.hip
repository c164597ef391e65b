// gguf_tile.hip -- LDS-tiled GEMM on v_mfma_f32_32x32x16_bf16 for GGUF weights at row counts the
// streaming kernels do not serve well: every native-block format (Q8_0, Q3_K, Q6_K, IQ4_NL, IQ3_S,
// IQ4_XS) above decode row counts, and Q5_K / Q4_K planes above 64 rows (the reference's
// sp_gguf_split / sp_gguf_wide, engine_gguf.metal:82-221, which stage a weight tile through
// threadgroup memory for every format).
//
// A workgroup of four waves (2 x 2) computes a BM x BN block of outputs, BM = 64 FM, BN = 64 FN,
// walking K 64 elements at a time. Per step:
//   * the activation tile A[BM][64] (bf16) is copied to LDS;
//   * each of the block's BN columns has its two 32-element groups decoded once, in registers,
//     by the format's reference-order decoder (gguf_decode.hpp), rounded to bf16 (RNE) and
//     written to LDS as B[BN][64];
//   * every wave multiplies its (32 FM) x (32 FN) sub-block from LDS fragments (row stride 144
//     bytes: the 16-byte operand reads do not conflict).
// Two barriers a step; no prefetch: several workgroups a CU (small tiles, few registers) hide the
// decode's load latency behind each other's MFMAs.
//
// Numerics: the weight is the decoder's fp32 value rounded to bf16 (RNE), products exact in fp32,
// fp32 accumulation -- as the q4 MFMA kernels.
#include "common.hpp"
#include "gguf_decode.hpp"
#include "launch.hpp"

namespace splosh {

constexpr int kGtStride = 72;  // bf16 elements per LDS row: 64 + 8 padding (144 bytes)

struct GgufTileArgs {
    const uint8_t *w;          // native blocks (rows back to back), or plane0 for Q5_K / Q4_K
    const uint8_t *plane1, *meta;
    uint32_t w_bytes, row_bytes;
    int64_t n, inner;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
};

// TYPE: a ggml type id; 13 / 12 = Q5_K / Q4_K planes.
template <int TYPE, int FM, int FN>
__global__ void __launch_bounds__(256) gguf_tile_kernel(GgufTileArgs args) {
    constexpr int BM = 64 * FM, BN = 64 * FN;
    constexpr int kAChunks = BM * 8;        // 16-byte chunks of the A tile
    constexpr int kAPer = kAChunks / 256;
    constexpr int kDecodes = 2 * BN;        // 32-element groups of the B tile
    constexpr int kDPer = (kDecodes + 255) / 256;
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t *sA = lds, *sB = lds + BM * kGtStride;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r = lane & 31, h = lane >> 5;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int steps = (int)(args.inner / 64);
    const rsrc_t wr = make_rsrc(args.w, args.w_bytes);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    for (int s = 0; s < steps; ++s) {
#pragma unroll
        for (int p = 0; p < kAPer; ++p) {
            const int c = p * 256 + tid, row = c >> 3, chunk = c & 7;
            const int64_t m = m0 + row;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (m < args.rows) v = *(const u32x4 *)(args.a + m * args.lda + (int64_t)s * 64 + chunk * 8);
            *(u32x4 *)(sA + row * kGtStride + chunk * 8) = v;
        }
#pragma unroll
        for (int p = 0; p < kDPer; ++p) {
            const int c = p * 256 + tid;
            if (c >= kDecodes) continue;
            const int col = c >> 1, half = c & 1;
            const int64_t n = n0 + col < args.n ? n0 + col : args.n - 1;
            const int64_t g = (int64_t)s * 2 + half;
            float v[32];
            if constexpr (TYPE == 13 || TYPE == 12)
                decode_plane_group(args.w, TYPE == 13 ? args.plane1 : nullptr, args.meta, args.inner, n, g, v);
            else
                decode_group<TYPE>(wr, (uint32_t)(n * args.row_bytes), (int)g, v);
            uint16_t *dst = sB + col * kGtStride + 32 * half;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x4 d;
#pragma unroll
                for (int e = 0; e < 4; ++e) d[e] = f32x2_to_bf16x2(v[8 * q + 2 * e], v[8 * q + 2 * e + 1]);
                *(u32x4 *)(dst + 8 * q) = d;
            }
        }
        __syncthreads();
        const uint16_t *A = sA + (wm * FM * 32 + r) * kGtStride + 8 * h;
        const uint16_t *B = sB + (wn * FN * 32 + r) * kGtStride + 8 * h;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 af[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = as_bf16x8(*(const u32x4 *)(A + i * 32 * kGtStride + 16 * ks));
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const bf16x8 bf = as_bf16x8(*(const u32x4 *)(B + j * 32 * kGtStride + 16 * ks));
#pragma unroll
                for (int i = 0; i < FM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf, acc[i][j], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // Element (row 8 (e / 4) + 4 h + e % 4 of tile i, column r of tile j).
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t n = n0 + wn * FN * 32 + j * 32 + r;
            if (n >= args.n) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t m = m0 + wm * FM * 32 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (m >= args.rows) continue;
                float value = acc[i][j][e];
                const int64_t index = m * args.ldc + n;
                if (args.out_dtype == SPLOSH_F32) {
                    if (args.residual) value += ((const float *)args.residual)[index];
                    ((float *)args.out)[index] = value;
                } else {
                    if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                    ((uint16_t *)args.out)[index] = f32_to_bf16(value);
                }
            }
        }
}

template <int TYPE, int FM, int FN>
static hipError_t launch_gt(const GgufTileArgs &args, hipStream_t stream) {
    constexpr int BM = 64 * FM, BN = 64 * FN;
    const size_t lds = (size_t)(BM + BN) * kGtStride * sizeof(uint16_t);
    const dim3 grid((unsigned)((args.n + BN - 1) / BN), (unsigned)((args.rows + BM - 1) / BM));
    hipLaunchKernelGGL((gguf_tile_kernel<TYPE, FM, FN>), grid, dim3(256), lds, stream, args);
    return hipGetLastError();
}

// Tile shape: 128 x 128 when that still gives two workgroups a CU, else 64 x 64.
template <int TYPE>
static hipError_t launch_gt_rows(const GgufTileArgs &args, hipStream_t stream) {
    const int64_t big = ((args.n + 127) / 128) * ((args.rows + 127) / 128);
    if (big >= 512) return launch_gt<TYPE, 2, 2>(args, stream);
    return launch_gt<TYPE, 1, 1>(args, stream);
}

bool gguf_tile_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda) {
    const int64_t limit = ((int64_t)1 << 31);
    return rows >= 1 && rows <= 65535LL * 64 && columns > 0 && inner % 64 == 0 && lda % 8 == 0 &&
           rows * lda < limit;
}

hipError_t launch_gguf_tile(int type, const uint8_t *w, const uint8_t *plane1, const uint8_t *meta, int64_t rows_w,
                            int64_t inner, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                            const void *residual, int64_t m, hipStream_t stream) {
    GgufTileArgs args = {};
    args.w = w;
    args.plane1 = plane1;
    args.meta = meta;
    args.n = rows_w;
    args.inner = inner;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = m;
    args.out_dtype = out_dtype;
    if (type != 13 && type != 12) {
        int elems = 0, bytes = 0;
        gguf_native_block(type, &elems, &bytes);
        args.row_bytes = (uint32_t)(inner / elems * bytes);
        args.w_bytes = (uint32_t)(rows_w * (int64_t)args.row_bytes);
    }
    switch (type) {
        case 8: return launch_gt_rows<8>(args, stream);
        case 11: return launch_gt_rows<11>(args, stream);
        case 14: return launch_gt_rows<14>(args, stream);
        case 20: return launch_gt_rows<20>(args, stream);
        case 21: return launch_gt_rows<21>(args, stream);
        case 23: return launch_gt_rows<23>(args, stream);
        case 12: return launch_gt_rows<12>(args, stream);
        default: return launch_gt_rows<13>(args, stream);
    }
}

}  // namespace splosh
