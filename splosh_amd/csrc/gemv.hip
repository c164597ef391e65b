// gemv.hip -- decode GEMV / very narrow GEMM (rows <= 8) over q4 weights.
//
// At one to eight activation rows the whole call is one pass over the weight (50 MB for
// K=5120, N=17408: about six HBM latencies at 8 TB/s), so what limits it is how much of the
// weight is in flight, not arithmetic. The kernel is built around that:
//
// * Every wave issues the code and sidecar loads of its whole K slice in two register stages;
//   stage 0 is issued before anything else, so its latency overlaps the prologue.
// * The activation rows are staged once per workgroup into LDS, already in the nibble-pair order
//   of the code operand (x0 x4 x1 x5 x2 x6 x3 x7 per 8 k), together with sum(a) of every 64-group.
//   The MFMA A operand is then one ds_read_b128 per 16 k, and the sums need no MFMA.
// * Arithmetic is stream32.hip's: P = sum a (128 + q) on v_mfma_f32_32x32x16_bf16 from raw codes,
//   acc += s P + (b - 128 s) S.
// The SK waves of a workgroup split K and meet in LDS.
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

struct GemvArgs {
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
};

constexpr int kGemvMaxRows = 8;

__device__ __forceinline__ bf16x8 gemv_codes(uint32_t w) {
    u32x4 d;
    d.x = (w & 0x000F000Fu) | 0x43004300u;
    d.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
    d.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
    d.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
    return as_bf16x8(d);
}

__device__ __forceinline__ u32x4 gemv_act_pairs(u32x4 v) {
    u32x4 o;
    o.x = perm_bytes(v.z, v.x, 0x05040100u);
    o.y = perm_bytes(v.z, v.x, 0x07060302u);
    o.z = perm_bytes(v.w, v.y, 0x05040100u);
    o.w = perm_bytes(v.w, v.y, 0x07060302u);
    return o;
}

// LDS row stride of the staged activations, in bf16 elements: K plus 8 so that consecutive rows
// start 16 bytes apart modulo the bank width.
__host__ __device__ inline int64_t gemv_a_stride(int64_t k) { return k + 8; }

template <int J, int RPL, int NW, bool TILED, int U>
__global__ void __launch_bounds__(512)
q4_gemv_kernel(GemvArgs args) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sk = blockDim.x / kWave;
    const int r = lane & 31, h = lane >> 5;
    const int64_t n0 = (int64_t)blockIdx.x * 32 * J;
    const int64_t m0 = (int64_t)blockIdx.y * kGemvMaxRows;
    const int64_t G = args.groups;
    const int64_t K = G * kGroup;
    const int mb = (int)(args.rows - m0 < kGemvMaxRows ? args.rows - m0 : kGemvMaxRows);
    const int64_t g0 = G * wave / sk, g1 = G * (wave + 1) / sk;
    const int64_t astride = gemv_a_stride(K);
    uint16_t *sa = (uint16_t *)lds;
    float *ssx = (float *)(lds + (size_t)mb * astride * 2);   // [kGemvMaxRows][G]

    int64_t col[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t n = n0 + 32 * j + r;
        col[j] = n < args.n ? n : args.n - 1;
    }

    struct Stage {
        u32x4 wq[U][NW][J];
        uint16_t side[U][NW][J];
    };
    auto load_stage = [&](Stage &st, int64_t gbase) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t g = gbase + u < g1 ? gbase + u : g1 - 1;
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    int64_t word, side;
                    if (TILED) {
                        const int64_t rec = tiled_record(col[j], g, G);
                        word = rec * 8 + 4 * h;
                        side = rec;
                    } else {
                        word = col[j] * args.stride_words + g * 8 + 4 * h;
                        side = col[j] * G + g;
                    }
                    st.wq[u][w][j] = *(const u32x4 *)(args.packed[w] + word);
                    st.side[u][w][j] = (h == 0 ? args.scales[w] : args.biases[w])[side];
                }
        }
    };

    Stage st0, st1;
    if (g0 < g1) load_stage(st0, g0);

    // Prologue: stage the rows' activations (pair-permuted) and their per-group sums.
    for (int64_t item = threadIdx.x; item < (int64_t)kGemvMaxRows * G; item += blockDim.x) {
        const int row = (int)(item / G);
        const int64_t g = item % G;
        float sum = 0.0f;
        if (row < mb) {
            const u32x4 *src = (const u32x4 *)(args.a + (m0 + row) * args.lda + g * kGroup);
            u32x4 *dst = (u32x4 *)(sa + row * astride + g * kGroup);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const u32x4 v = src[c];
                dst[c] = gemv_act_pairs(v);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    sum += bf16_bits_to_f32(v[e] & 0xffffu) + bf16_bits_to_f32(v[e] >> 16);
            }
        }
        ssx[row * G + g] = sum;
    }
    __syncthreads();

    float acc[NW][J][RPL];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < RPL; ++i) acc[w][j][i] = 0.0f;
    f32x16 zero;
#pragma unroll
    for (int i = 0; i < 16; ++i) zero[i] = 0.0f;
    const bool arow_valid = r < mb;
    const uint16_t *arow = sa + (arow_valid ? r : 0) * astride + 32 * h;

    auto use_stage = [&](const Stage &st, int64_t gbase) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t g = gbase + u;
            if (g >= g1) break;
            bf16x8 a[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (arow_valid) v = *(const u32x4 *)(arow + g * kGroup + 8 * i);
                a[i] = as_bf16x8(v);
            }
            float sx[RPL];
#pragma unroll
            for (int i = 0; i < RPL; ++i) sx[i] = ssx[(8 * (i >> 2) + 4 * h + (i & 3)) * G + g];
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint32_t mine = st.side[u][w][j];
                    const uint32_t other = (uint32_t)__shfl_xor((int)mine, 32);
                    const float s = bf16_bits_to_f32(h == 0 ? mine : other);
                    const float b = bf16_bits_to_f32(h == 0 ? other : mine);
                    const float bp = __builtin_fmaf(-128.0f, s, b);
                    f32x16 p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], gemv_codes(st.wq[u][w][j].x), zero, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], gemv_codes(st.wq[u][w][j].y), p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], gemv_codes(st.wq[u][w][j].z), p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[3], gemv_codes(st.wq[u][w][j].w), p, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < RPL; ++i)
                        acc[w][j][i] = __builtin_fmaf(s, p[i], __builtin_fmaf(bp, sx[i], acc[w][j][i]));
                }
        }
    };

    for (int64_t g = g0; g < g1; g += 2 * U) {
        if (g + U < g1) load_stage(st1, g + U);
        use_stage(st0, g);
        if (g + U >= g1) break;
        if (g + 2 * U < g1) load_stage(st0, g + 2 * U);
        use_stage(st1, g + U);
    }

    // Split-K partials meet in LDS (the activation stage is dead now).
    __syncthreads();
    float *red = (float *)lds;
    constexpr int kPerWeight = J * RPL * kWave;
    constexpr int kPerWave = NW * kPerWeight;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < RPL; ++i) red[wave * kPerWave + ((w * J + j) * RPL + i) * kWave + lane] = acc[w][j][i];
    __syncthreads();
    for (int e = threadIdx.x; e < kPerWeight; e += blockDim.x) {
        const int ln = e % kWave;
        const int i = (e / kWave) % RPL;
        const int j = e / (kWave * RPL);
        const int64_t mm = m0 + 8 * (i >> 2) + 4 * (ln >> 5) + (i & 3);
        const int64_t n = n0 + 32 * j + (ln & 31);
        if (mm >= args.rows || n >= args.n) continue;
        float v[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            float sum = 0.0f;
            for (int s = 0; s < sk; ++s) sum += red[s * kPerWave + w * kPerWeight + e];
            v[w] = sum;
        }
        float value = NW == 2 ? silu(v[0]) * v[1] : v[0];
        const int64_t index = mm * args.ldc + n;
        if (args.out_dtype == SPLOSH_F32) {
            if (args.residual) value += ((const float *)args.residual)[index];
            ((float *)args.out)[index] = value;
        } else {
            if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
            ((uint16_t *)args.out)[index] = f32_to_bf16(value);
        }
    }
}

bool gemv_fits(int64_t rows, int64_t inner) {
    const int64_t mb = rows < kGemvMaxRows ? rows : kGemvMaxRows;
    return rows <= kGemvMaxRows && inner % kGroup == 0 &&
           mb * gemv_a_stride(inner) * 2 + (int64_t)kGemvMaxRows * (inner / kGroup) * 4 <= 64 * 1024;
}

StreamPlan plan_gemv(int64_t rows, int64_t columns, int64_t groups, bool mlp) {
    StreamPlan p;
    p.mb = 1;
    p.row_chunks = 1;
    p.rpl = rows == 1 ? 1 : rows == 2 ? 2 : 4;
    // Two 32-column blocks a wave (four stage words of codes per group) unless that leaves fewer
    // than 256 workgroups or the fused pair would need too many registers.
    p.j = mlp ? 1 : 2;
    if (p.j == 2 && (columns + 63) / 64 < 256) p.j = 1;
    p.col_blocks = (int)((columns + 32 * p.j - 1) / (32 * p.j));
    // Waves per workgroup: about eight groups a wave, at most eight waves.
    int64_t sk = (groups + 7) / 8;
    if (sk > 8) sk = 8;
    if (sk < 1) sk = 1;
    p.sk = (int)sk;
    return p;
}

template <int J, int RPL, int NW, int U>
static hipError_t launch_gemv_v(const StreamPlan &p, bool tiled, const GemvArgs &args, int64_t inner,
                                hipStream_t stream) {
    dim3 grid((unsigned)p.col_blocks, 1);
    dim3 block((unsigned)(p.sk * kWave));
    const int64_t mb = args.rows < kGemvMaxRows ? args.rows : kGemvMaxRows;
    size_t stage = (size_t)(mb * gemv_a_stride(inner) * 2 + (int64_t)kGemvMaxRows * (inner / kGroup) * 4);
    const size_t red = (size_t)p.sk * NW * J * RPL * kWave * sizeof(float);
    const size_t lds = stage > red ? stage : red;
    if (tiled)
        hipLaunchKernelGGL((q4_gemv_kernel<J, RPL, NW, true, U>), grid, block, lds, stream, args);
    else
        hipLaunchKernelGGL((q4_gemv_kernel<J, RPL, NW, false, U>), grid, block, lds, stream, args);
    return hipGetLastError();
}

template <int NW>
static hipError_t launch_gemv_nw(const StreamPlan &p, bool tiled, const GemvArgs &args, int64_t inner, int64_t gpw,
                                 hipStream_t stream) {
    // Stage size: half a wave's groups (so that two stages cover it) where registers allow.
    const int64_t half = (gpw + 1) / 2;
#define SPLOSH_GEMV_CASE(J_, RPL_)                                                             \
    if (p.j == J_ && p.rpl == RPL_)                                                            \
        return half <= 4 ? launch_gemv_v<J_, RPL_, NW, 4>(p, tiled, args, inner, stream)       \
             : half <= 5 ? launch_gemv_v<J_, RPL_, NW, 5>(p, tiled, args, inner, stream)       \
                         : launch_gemv_v<J_, RPL_, NW, 8>(p, tiled, args, inner, stream);
    SPLOSH_GEMV_CASE(1, 1) SPLOSH_GEMV_CASE(1, 2) SPLOSH_GEMV_CASE(1, 4)
    if constexpr (NW == 1) {
        SPLOSH_GEMV_CASE(2, 1) SPLOSH_GEMV_CASE(2, 2) SPLOSH_GEMV_CASE(2, 4)
    }
#undef SPLOSH_GEMV_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_q4_gemv(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                          const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                          int64_t rows, hipStream_t stream) {
    GemvArgs args;
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
    const bool tiled = w.order == SPLOSH_Q4_TILED128;
    const int64_t gpw = (args.groups + plan.sk - 1) / plan.sk;
    return up ? launch_gemv_nw<2>(plan, tiled, args, w.inner, gpw, stream)
              : launch_gemv_nw<1>(plan, tiled, args, w.inner, gpw, stream);
}

}  // namespace splosh
