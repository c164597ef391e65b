// stream32.hip -- the decode / narrow-batch q4 streaming kernel (rows <= 32) on
// v_mfma_f32_32x32x16_bf16.
//
// Arithmetic as in stream.hip: codes become bf16 128 + q (one AND-OR per pair of nibbles j, j+4),
// P = sum a (128 + q) per group from four chained MFMAs, S = sum a from four MFMAs against ones,
// acc += s P + (b - 128 s) S.
//
// Why 32x32x16. Its B operand gives lane (r, h) = (lane & 31, lane >> 5) one word of column r per
// MFMA, so over a group's four MFMAs the lane uses words 4h..4h+3 of its row's 32-byte record:
// one 16-byte load. The 64 lanes of a wave then read 32 consecutive records -- a contiguous
// kilobyte of the tiled layout -- with one instruction, and each column's bf16 scale and bias
// come from one 2-byte load (lanes h = 0 load scales, h = 1 biases, swapped across halves with
// one ds_bpermute).
//
// Pipelining. A wave walks its K slice in stages of U groups; every load of a stage (codes,
// sidecars and the activation words) is issued before the previous stage is consumed, so the
// wait before an MFMA only covers loads issued a whole stage earlier.
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

struct Q4Stream32Args {
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

__device__ __forceinline__ bf16x8 codes_pairs(uint32_t w) {
    u32x4 d;
    d.x = (w & 0x000F000Fu) | 0x43004300u;
    d.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
    d.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
    d.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
    return as_bf16x8(d);
}

__device__ __forceinline__ bf16x8 act_pairs(u32x4 v) {
    u32x4 o;
    o.x = perm_bytes(v.z, v.x, 0x05040100u);
    o.y = perm_bytes(v.z, v.x, 0x07060302u);
    o.z = perm_bytes(v.w, v.y, 0x05040100u);
    o.w = perm_bytes(v.w, v.y, 0x07060302u);
    return as_bf16x8(o);
}

// Row of accumulator register i of lane half h in the 32x32 output block.
__device__ __forceinline__ int row_of(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

template <int J, int RPL, int NW, bool TILED, int U>
__global__ void __launch_bounds__(512)
q4_stream32_kernel(Q4Stream32Args args) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sk = blockDim.x / kWave;
    const int r = lane & 31, h = lane >> 5;
    const int64_t n0 = (int64_t)blockIdx.x * 32 * J;
    const int64_t m0 = (int64_t)blockIdx.y * 32;
    const int64_t G = args.groups;
    const int64_t g0 = G * wave / sk, g1 = G * (wave + 1) / sk;

    int64_t col[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t n = n0 + 32 * j + r;
        col[j] = n < args.n ? n : args.n - 1;
    }
    const int64_t m = m0 + r;
    const bool mvalid = m < args.rows;
    const uint16_t *arow = args.a + (mvalid ? m : 0) * args.lda + 32 * h;

    float acc[NW][J][RPL];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < RPL; ++i) acc[w][j][i] = 0.0f;

    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    f32x16 zero;
#pragma unroll
    for (int i = 0; i < 16; ++i) zero[i] = 0.0f;

    struct Stage {
        u32x4 wq[U][NW][J];
        uint16_t side[U][NW][J];
        u32x4 av[U][4];
    };
    auto load_stage = [&](Stage &st, int64_t gbase) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t g = gbase + u;
            if (g < g1) {
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
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    u32x4 v = {0u, 0u, 0u, 0u};
                    if (mvalid) v = *(const u32x4 *)(arow + g * kGroup + 8 * i);
                    st.av[u][i] = v;
                }
            }
        }
    };
    auto use_stage = [&](const Stage &st, int64_t gbase) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (gbase + u >= g1) break;
            bf16x8 a[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = act_pairs(st.av[u][i]);
            f32x16 sx = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], ones, zero, 0, 0, 0);
#pragma unroll
            for (int i = 1; i < 4; ++i) sx = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], ones, sx, 0, 0, 0);
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint32_t mine = st.side[u][w][j];
                    const uint32_t other = (uint32_t)__shfl_xor((int)mine, 32);
                    const float s = bf16_bits_to_f32(h == 0 ? mine : other);
                    const float b = bf16_bits_to_f32(h == 0 ? other : mine);
                    const float bp = __builtin_fmaf(-128.0f, s, b);
                    f32x16 p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], codes_pairs(st.wq[u][w][j].x), zero, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], codes_pairs(st.wq[u][w][j].y), p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], codes_pairs(st.wq[u][w][j].z), p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[3], codes_pairs(st.wq[u][w][j].w), p, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < RPL; ++i)
                        acc[w][j][i] = __builtin_fmaf(s, p[i], __builtin_fmaf(bp, sx[i], acc[w][j][i]));
                }
        }
    };

    Stage st0, st1;
    if (g0 < g1) load_stage(st0, g0);
    for (int64_t g = g0; g < g1; g += 2 * U) {
        if (g + U < g1) load_stage(st1, g + U);
        use_stage(st0, g);
        if (g + U >= g1) break;
        if (g + 2 * U < g1) load_stage(st0, g + 2 * U);
        use_stage(st1, g + U);
    }

    // Split-K partials meet in LDS: red[wave][weight][j][reg][lane].
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
        float v[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            float sum = 0.0f;
            for (int s = 0; s < sk; ++s) sum += red[s * kPerWave + w * kPerWeight + e];
            v[w] = sum;
        }
        const int ln = e % kWave;
        const int i = (e / kWave) % RPL;
        const int j = e / (kWave * RPL);
        const int64_t mm = m0 + row_of(i, ln >> 5);
        const int64_t n = n0 + 32 * j + (ln & 31);
        if (mm < args.rows && n < args.n) {
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
}

StreamPlan plan_stream32(int64_t rows, int64_t columns, int64_t groups, bool mlp) {
    StreamPlan p;
    p.mb = 1;
    p.row_chunks = (int)((rows + 31) / 32);
    p.rpl = rows == 1 ? 1 : rows == 2 ? 2 : rows <= 8 ? 4 : 16;
    p.j = p.rpl == 16 ? 1 : 2;
    while (p.j > 1 && ((columns + 32 * p.j - 1) / (32 * p.j)) * p.row_chunks < 256) p.j /= 2;
    p.col_blocks = (int)((columns + 32 * p.j - 1) / (32 * p.j));
    const int64_t wgs = (int64_t)p.col_blocks * p.row_chunks;
    int64_t sk = (2048 + wgs - 1) / wgs;
    if (sk > 8) sk = 8;
    if (sk > groups / 2) sk = groups / 2;
    if (sk < 1) sk = 1;
    const int64_t per_wave = (int64_t)(mlp ? 2 : 1) * p.j * p.rpl * kWave * 4;
    while (sk > 1 && sk * per_wave > 65536) --sk;
    p.sk = (int)sk;
    return p;
}

template <int J, int RPL, int NW>
static hipError_t launch32(const StreamPlan &p, bool tiled, const Q4Stream32Args &args, hipStream_t stream) {
    constexpr int U = 2;
    dim3 grid((unsigned)p.col_blocks, (unsigned)p.row_chunks);
    dim3 block((unsigned)(p.sk * kWave));
    const size_t lds = (size_t)p.sk * NW * J * RPL * kWave * sizeof(float);
    if (tiled)
        hipLaunchKernelGGL((q4_stream32_kernel<J, RPL, NW, true, U>), grid, block, lds, stream, args);
    else
        hipLaunchKernelGGL((q4_stream32_kernel<J, RPL, NW, false, U>), grid, block, lds, stream, args);
    return hipGetLastError();
}

template <int NW>
static hipError_t launch32_nw(const StreamPlan &p, bool tiled, const Q4Stream32Args &args, hipStream_t stream) {
#define SPLOSH_CASE32(J_, RPL_) \
    if (p.j == J_ && p.rpl == RPL_) return launch32<J_, RPL_, NW>(p, tiled, args, stream);
    SPLOSH_CASE32(2, 1) SPLOSH_CASE32(1, 1)
    SPLOSH_CASE32(2, 2) SPLOSH_CASE32(1, 2)
    SPLOSH_CASE32(2, 4) SPLOSH_CASE32(1, 4)
    SPLOSH_CASE32(1, 16)
#undef SPLOSH_CASE32
    return hipErrorInvalidValue;
}

hipError_t launch_q4_stream32(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                              const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                              const void *residual, int64_t rows, hipStream_t stream) {
    Q4Stream32Args args;
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
    return up ? launch32_nw<2>(plan, tiled, args, stream) : launch32_nw<1>(plan, tiled, args, stream);
}

}  // namespace splosh
