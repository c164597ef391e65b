// tile.hip -- LDS-tiled q4 GEMM on v_mfma_f32_32x32x16_bf16: draft-verify (M = 64) and prefill
// (M >= 512).
//
// A workgroup computes a BM x BN block of outputs (for NW = 2, of both the gate and the up
// weight) walking K one 64-group at a time. Per group:
//   * the activation tile A[BM][64] (bf16) is copied to LDS;
//   * the weight tile is dequantized exactly once: each thread loads 16 bytes of codes (half of a
//     32-byte tiled record: BN consecutive records are contiguous), turns its 32 codes into bf16
//     weights RNE(s q + b) (v_cvt_f32_ubyte, v_fma_f32, v_cvt_pk_bf16_f32: 22 VALU per 8 weights)
//     and writes them to LDS as B[BN][64];
//   * every wave multiplies its (32 FM) x (32 FN) sub-block from LDS fragments: the A operand of an
//     MFMA step is row r, k = 16 i + 8 h .. + 7 and the B operand column r, the same k -- one
//     ds_read_b128 each (row stride 144 bytes: conflict-free).
// The next group's codes, sidecars and activations are loaded into registers while the current
// group is multiplied; LDS is double-buffered, one barrier per group.
//
// Split K. When a shape has too few output blocks to fill the GPU (the 64-row down projection has
// 80), gridDim.z workgroups share one block over K slices and write fp32 partials to a caller
// workspace; a second kernel sums them in a fixed order (deterministic) and applies the epilogue.
//
// Numerics as mma.hip: fp32 dequantized weight rounded to bf16, exact products, fp32 sums.
#include "common.hpp"
#include "launch.hpp"

#include <cstdlib>

namespace splosh {

struct TileArgs {
    const uint32_t *packed[2];
    const uint16_t *scales[2];
    const uint16_t *biases[2];
    int64_t stride_words;
    int64_t n;
    int64_t groups;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
    float *partial;      // split-K workspace [splits][NW][rows][n], or null
};

constexpr int kLdsStride = 72;  // bf16 elements per LDS row: 64 + 8 padding (144 bytes)

__device__ __forceinline__ float cvt_ubyte(uint32_t x, int j) {
    float r;
    switch (j) {
        case 0: asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x)); break;
        case 1: asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x)); break;
        case 2: asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x)); break;
        default: asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x)); break;
    }
    return r;
}

// Eight weights of one code word (k order), RNE(s q + b) as bf16.
__device__ __forceinline__ u32x4 tile_dequant(uint32_t w, float s, float b) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    u32x4 d;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        d[j] = f32x2_to_bf16x2(__builtin_fmaf(s, cvt_ubyte(lo, j), b), __builtin_fmaf(s, cvt_ubyte(hi, j), b));
    return d;
}

// WM x WN waves, each FM x FN MFMA tiles of 32 x 32; NW weights.
template <int WM, int WN, int FM, int FN, int NW, bool TILED>
__global__ void __launch_bounds__(WM * WN * 64)
q4_tile_kernel(TileArgs args) {
    constexpr int kThreads = WM * WN * 64;
    constexpr int BM = WM * FM * 32, BN = WN * FN * 32;
    constexpr int kAChunks = BM * 8;                  // 16-byte chunks of the A tile
    constexpr int kAPer = (kAChunks + kThreads - 1) / kThreads;
    constexpr int kBHalves = NW * BN * 2;             // 16-byte halves of code records
    constexpr int kBPer = (kBHalves + kThreads - 1) / kThreads;
    constexpr int kAStage = BM * kLdsStride;          // bf16 elements
    constexpr int kBStage = NW * BN * kLdsStride;
    extern __shared__ __align__(16) uint16_t lds[];
    auto sA = [&](int buf) { return lds + buf * (kAStage + kBStage); };
    auto sB = [&](int buf) { return lds + buf * (kAStage + kBStage) + kAStage; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int r = lane & 31, h = lane >> 5;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;
    const int64_t G = args.groups;
    const int splits = gridDim.z;
    const int64_t g0 = G * blockIdx.z / splits, g1 = G * (blockIdx.z + 1) / splits;
    const uint32_t G32 = (uint32_t)G;

    // Per-thread load assignments.
    uint32_t a_off[kAPer];
    bool a_ok[kAPer];
    uint32_t a_lds[kAPer];
#pragma unroll
    for (int p = 0; p < kAPer; ++p) {
        const int c = p * kThreads + tid;
        const int row = c >> 3, chunk = c & 7;
        const int64_t m = m0 + row;
        a_ok[p] = c < kAChunks && m < args.rows;
        a_off[p] = (uint32_t)((a_ok[p] ? m : 0) * args.lda + chunk * 8);
        a_lds[p] = (uint32_t)(row * kLdsStride + chunk * 8);
    }
    uint32_t b_col[kBPer];
    int b_w[kBPer], b_half[kBPer];
    bool b_ok[kBPer];
#pragma unroll
    for (int p = 0; p < kBPer; ++p) {
        const int c = p * kThreads + tid;
        const int w = c / (BN * 2), rem = c % (BN * 2);
        const int col = rem >> 1;
        b_w[p] = w < NW ? w : 0;
        b_half[p] = rem & 1;
        b_ok[p] = c < kBHalves;
        const int64_t n = n0 + col;
        b_col[p] = (uint32_t)(n < args.n ? n : args.n - 1);
    }

    u32x4 ra[kAPer], rb[kBPer];
    uint32_t rs[kBPer], rbias[kBPer];
    auto load_group = [&](int64_t g) {
        const uint32_t g32 = (uint32_t)g;
#pragma unroll
        for (int p = 0; p < kAPer; ++p) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (a_ok[p]) v = *(const u32x4 *)(args.a + a_off[p] + g32 * 64u);
            ra[p] = v;
        }
#pragma unroll
        for (int p = 0; p < kBPer; ++p) {
            if (!b_ok[p]) continue;
            uint32_t word, sidx;
            const uint32_t col = b_col[p];
            if (TILED) {
                const uint32_t rec = ((col >> 7) * G32 + g32) * 128u + (col & 127u);
                word = rec * 8u + 4u * b_half[p];
                sidx = rec;
            } else {
                word = col * (uint32_t)args.stride_words + g32 * 8u + 4u * b_half[p];
                sidx = col * G32 + g32;
            }
            const int w = b_w[p];
            rb[p] = *(const u32x4 *)(args.packed[w] + word);
            rs[p] = args.scales[w][sidx];
            rbias[p] = args.biases[w][sidx];
        }
    };
    auto store_group = [&](int buf) {
#pragma unroll
        for (int p = 0; p < kAPer; ++p)
            if (p * kThreads + tid < kAChunks) *(u32x4 *)(sA(buf) + a_lds[p]) = ra[p];
#pragma unroll
        for (int p = 0; p < kBPer; ++p) {
            if (!b_ok[p]) continue;
            const int c = p * kThreads + tid;
            const int w = c / (BN * 2), col = (c % (BN * 2)) >> 1;
            const float s = bf16_bits_to_f32(rs[p]), b = bf16_bits_to_f32(rbias[p]);
            uint16_t *dst = sB(buf) + (w * BN + col) * kLdsStride + 32 * b_half[p];
#pragma unroll
            for (int i = 0; i < 4; ++i) *(u32x4 *)(dst + 8 * i) = tile_dequant(rb[p][i], s, b);
        }
    };

    f32x16 acc[NW][FM][FN];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[w][i][j][e] = 0.0f;

    if (g0 < g1) {
        load_group(g0);
        store_group(0);
    }
    __syncthreads();
    int buf = 0;
    for (int64_t g = g0; g < g1; ++g) {
        if (g + 1 < g1) load_group(g + 1);
        const uint16_t *A = sA(buf) + (wm * FM * 32 + r) * kLdsStride + 8 * h;
        const uint16_t *B = sB(buf) + (wn * FN * 32 + r) * kLdsStride + 8 * h;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 af[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = as_bf16x8(*(const u32x4 *)(A + i * 32 * kLdsStride + 16 * ks));
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const bf16x8 bf =
                        as_bf16x8(*(const u32x4 *)(B + (w * BN + j * 32) * kLdsStride + 16 * ks));
#pragma unroll
                    for (int i = 0; i < FM; ++i)
                        acc[w][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf, acc[w][i][j], 0, 0, 0);
                }
        }
        if (g + 1 < g1) store_group(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // Epilogue: element (row 8 (e / 4) + 4 h + e % 4 of tile i, column r of tile j).
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
                if (args.partial) {
#pragma unroll
                    for (int w = 0; w < NW; ++w)
                        args.partial[(((int64_t)blockIdx.z * NW + w) * args.rows + m) * args.n + n] = acc[w][i][j][e];
                    continue;
                }
                float value = acc[0][i][j][e];
                if constexpr (NW == 2) value = silu(value) * acc[NW - 1][i][j][e];
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

// Sum the split-K partials in slice order and apply the epilogue.
__global__ void __launch_bounds__(256)
tile_splitk_finish(const float *__restrict__ partial, int splits, int nw, int64_t rows, int64_t n, void *out,
                   int64_t ldc, int out_dtype, const void *residual) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * n) return;
    const int64_t m = idx / n, col = idx % n;
    float v[2] = {0.0f, 0.0f};
    for (int w = 0; w < nw; ++w)
        for (int s = 0; s < splits; ++s) v[w] += partial[((int64_t)s * nw + w) * rows * n + idx];
    float value = nw == 2 ? silu(v[0]) * v[1] : v[0];
    const int64_t index = m * ldc + col;
    if (out_dtype == SPLOSH_F32) {
        if (residual) value += ((const float *)residual)[index];
        ((float *)out)[index] = value;
    } else {
        if (residual) value += bf16_bits_to_f32(((const uint16_t *)residual)[index]);
        ((uint16_t *)out)[index] = f32_to_bf16(value);
    }
}

// Tile shapes: 0 = 64 x 64 (4 waves, 2 x 2 of 32 x 32), 1 = 256 x 256 (8 waves of 128 x 64),
// 2 = 128 x 128 (4 waves of 64 x 64).
struct TileShape {
    int bm, bn;
};
static TileShape tile_shape(int kind) {
    switch (kind) {
        case 1: return {256, 256};
        case 2: return {128, 128};
        default: return {64, 64};
    }
}

static int tile_kind(int64_t rows, bool mlp) {
    int kind = rows <= 64 ? 0 : (rows >= 1024 && !mlp ? 1 : 2);
    // A development override of the tile shape, read from the environment once per process.
    static const int kind_override = [] { const char *e = getenv("SPLOSH_TILE_KIND"); return e ? atoi(e) : -1; }();
    if (kind_override >= 0) kind = kind_override;
    if (mlp && kind == 1) kind = 2;
    return kind;
}

// The kernel addresses activations and code words with 32-bit element offsets.
bool tile_fits(int64_t rows, int64_t columns, int64_t lda, int64_t stride_words) {
    const int64_t limit = (int64_t)1 << 32;
    return rows > 0 && columns > 0 && rows * lda < limit && columns * stride_words < limit && rows <= 65535 * 64LL;
}

// Arrival counters of the other kernels sit in the first 16 KiB of a shared workspace.
constexpr size_t kTileCounterBytes = 16384;

TilePlan plan_tile(int64_t rows, int64_t columns, int64_t groups, bool mlp, size_t workspace_bytes) {
    TilePlan p;
    p.kind = tile_kind(rows, mlp);
    const TileShape t = tile_shape(p.kind);
    p.grid_m = (int)((rows + t.bm - 1) / t.bm);
    p.grid_n = (int)((columns + t.bn - 1) / t.bn);
    // Split K when the blocks cannot give every CU a workgroup, if the workspace allows.
    int splits = 1;
    const int64_t blocks = (int64_t)p.grid_m * p.grid_n;
    while (splits < 8 && blocks * splits < 256 && groups / (splits * 2) >= 8) splits *= 2;
    static const int splits_override = [] { const char *e = getenv("SPLOSH_TILE_SPLITS"); return e ? atoi(e) : 0; }();
    if (splits_override > 0) splits = splits_override;
    const size_t need = kTileCounterBytes + (size_t)splits * (mlp ? 2 : 1) * rows * columns * sizeof(float);
    if (splits > 1 && need > workspace_bytes) splits = 1;
    p.splits = splits;
    return p;
}

size_t tile_workspace_bytes(int64_t rows, int64_t columns, int64_t groups, bool mlp) {
    const TilePlan p = plan_tile(rows, columns, groups, mlp, (size_t)-1);
    return p.splits > 1 ? kTileCounterBytes + (size_t)p.splits * (mlp ? 2 : 1) * rows * columns * sizeof(float) : 0;
}

template <int WM, int WN, int FM, int FN, int NW>
static hipError_t launch_tile_v(const TilePlan &p, bool tiled, const TileArgs &args, hipStream_t stream) {
    constexpr int BM = WM * FM * 32, BN = WN * FN * 32;
    const size_t lds = (size_t)2 * (BM + NW * BN) * kLdsStride * sizeof(uint16_t);
    dim3 grid((unsigned)p.grid_n, (unsigned)p.grid_m, (unsigned)p.splits);
    dim3 block(WM * WN * 64);
    if (tiled) {
        static bool once = [] {
            (void)hipFuncSetAttribute((const void *)q4_tile_kernel<WM, WN, FM, FN, NW, true>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            return true;
        }();
        (void)once;
        hipLaunchKernelGGL((q4_tile_kernel<WM, WN, FM, FN, NW, true>), grid, block, lds, stream, args);
    } else {
        static bool once = [] {
            (void)hipFuncSetAttribute((const void *)q4_tile_kernel<WM, WN, FM, FN, NW, false>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            return true;
        }();
        (void)once;
        hipLaunchKernelGGL((q4_tile_kernel<WM, WN, FM, FN, NW, false>), grid, block, lds, stream, args);
    }
    return hipGetLastError();
}

template <int NW>
static hipError_t launch_tile_nw(const TilePlan &p, bool tiled, const TileArgs &args, hipStream_t stream) {
    switch (p.kind) {
        case 1:
            if constexpr (NW == 1) return launch_tile_v<2, 4, 4, 2, NW>(p, tiled, args, stream);
            return hipErrorInvalidValue;  // plan_tile never picks it for two weights
        case 2: return launch_tile_v<2, 2, 2, 2, NW>(p, tiled, args, stream);
        default: return launch_tile_v<2, 2, 1, 1, NW>(p, tiled, args, stream);
    }
}

hipError_t launch_q4_tile(const TilePlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                          const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                          int64_t rows, void *workspace, hipStream_t stream) {
    TileArgs args;
    args.packed[0] = w.packed;
    args.scales[0] = w.scales;
    args.biases[0] = w.biases;
    args.packed[1] = up ? up->packed : w.packed;
    args.scales[1] = up ? up->scales : w.scales;
    args.biases[1] = up ? up->biases : w.biases;
    args.stride_words = w.row_stride_words;
    args.n = w.rows;
    args.groups = w.inner / kGroup;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = rows;
    args.out_dtype = out_dtype;
    // The partials follow the 16 KiB of arrival counters the other kernels keep at the start of the
    // workspace (zero between calls), which this kernel never touches.
    float *partial = plan.splits > 1 ? (float *)((char *)workspace + kTileCounterBytes) : nullptr;
    args.partial = partial;
    const bool tiled = w.order == SPLOSH_Q4_TILED128;
    hipError_t err = up ? launch_tile_nw<2>(plan, tiled, args, stream) : launch_tile_nw<1>(plan, tiled, args, stream);
    if (err != hipSuccess || plan.splits == 1) return err;
    return launch_splitk_finish(partial, plan.splits, up ? 2 : 1, rows, w.rows, out, ldc, out_dtype,
                                residual, stream);
}

hipError_t launch_splitk_finish(const float *partial, int splits, int nw, int64_t rows, int64_t n, void *out,
                                int64_t ldc, int out_dtype, const void *residual, hipStream_t stream) {
    const int64_t total = rows * n;
    hipLaunchKernelGGL(tile_splitk_finish, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, partial,
                       splits, nw, rows, n, out, ldc, out_dtype, residual);
    return hipGetLastError();
}

}  // namespace splosh
