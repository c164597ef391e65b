// stream.hip -- weight-streaming GEMV/GEMM for small row counts (decode M=1, draft-verify M<=64).
//
// The path is bound by reading the weight once from HBM, so the kernel's job is to turn packed
// codes into MFMA operands with as few VALU instructions per weight as possible and to keep many
// loads in flight.
//
// Arithmetic. Per 64-element group g of output n the reference computes
//   sum_k a[m][k] * (s * q[k] + b)          (Oracle/DequantOracle.swift:20, gemm_q4.metal:50-51)
// which is s * sum(a q) + b * sum(a) (the per-group identity of engine_na.metal:8-20). A 4-bit code
// becomes the bf16 value 128 + q with one AND-OR ((w >> 4j) & 0x000F000F | 0x43004300 turns
// nibbles j and j+4 of a word into two bf16 lanes), so one v_mfma_f32_16x16x32_bf16 on raw codes
// gives P = 128 * sum(a) + sum(a q) exactly (bf16 x bf16 products are exact in fp32), and a
// second MFMA against a ones operand gives S = sum(a). The epilogue is
//   acc += s * P + (b - 128 s) * S.
// The activation operand is permuted (x0 x4 x1 x5 x2 x6 x3 x7) with v_perm_b32 to match the
// nibble-pair order of the codes.
//
// Shape. A wave owns 16*J consecutive outputs and all 16*MB rows of its row chunk, over a slice of
// the K groups; the SK waves of a workgroup split K and meet in LDS. In MFMA terms the weight
// rows are the B columns (lane & 15) and the activation rows the A rows (lane & 15); lane >> 4
// picks which 16 of a group's 64 k the lane feeds: words 2c and 2c+1 of the group's record, 8
// bytes, so the 64 lanes of a wave read the 16 records of a 16-row block (512 contiguous bytes in
// the tiled layout) with one load.
#include "common.hpp"
#include "launch.hpp"

namespace splosh {

struct Q4StreamArgs {
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

// Nibbles j and j + 4 of w as the bf16 pair (128 + q_j, 128 + q_{j+4}), j = 0..3.
__device__ __forceinline__ bf16x8 q4_codes_operand(uint32_t w) {
    u32x4 d;
    d.x = (w & 0x000F000Fu) | 0x43004300u;
    d.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
    d.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
    d.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
    return as_bf16x8(d);
}

// Eight bf16 activations x0..x7 (four words) reordered to x0 x4 x1 x5 x2 x6 x3 x7.
__device__ __forceinline__ bf16x8 q4_act_operand(u32x4 v) {
    u32x4 o;
    o.x = perm_bytes(v.z, v.x, 0x05040100u);
    o.y = perm_bytes(v.z, v.x, 0x07060302u);
    o.z = perm_bytes(v.w, v.y, 0x05040100u);
    o.w = perm_bytes(v.w, v.y, 0x07060302u);
    return as_bf16x8(o);
}

__device__ __forceinline__ bf16x8 ones_operand() {
    u32x4 d = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    return as_bf16x8(d);
}

__device__ __forceinline__ void store_value(void *out, int64_t index, int out_dtype, const void *residual, float v) {
    if (out_dtype == SPLOSH_F32) {
        if (residual) v += ((const float *)residual)[index];
        ((float *)out)[index] = v;
    } else {
        if (residual) v += bf16_bits_to_f32(((const uint16_t *)residual)[index]);
        ((uint16_t *)out)[index] = f32_to_bf16(v);
    }
}

// Sum the SK waves' partials held in LDS and write the outputs of the workgroup.
// red layout: [wave][weight][j][mb][reg][lane].
template <int MB, int J, int RPL, int NW>
__device__ __forceinline__ void stream_finish(const float *red, int sk, int64_t n0, int64_t m0, int64_t n_total,
                                              int64_t rows, void *out, int64_t ldc, int out_dtype,
                                              const void *residual) {
    constexpr int kPerWeight = J * MB * RPL * kWave;
    constexpr int kPerWave = NW * kPerWeight;
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
        const int mb = (e / (kWave * RPL)) % MB;
        const int j = e / (kWave * RPL * MB);
        const int64_t m = m0 + 16 * mb + 4 * (ln >> 4) + i;
        const int64_t n = n0 + 16 * j + (ln & 15);
        if (m < rows && n < n_total) {
            const float value = NW == 2 ? silu(v[0]) * v[1] : v[0];
            store_value(out, m * ldc + n, out_dtype, residual, value);
        }
    }
}

template <int MB, int J, int RPL, int NW, bool TILED>
__global__ void __launch_bounds__(512)
q4_stream_kernel(Q4StreamArgs args) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sk = blockDim.x / kWave;
    const int r = lane & 15, c = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 16 * J;
    const int64_t m0 = (int64_t)blockIdx.y * 16 * MB;
    const int64_t G = args.groups;
    const int64_t g0 = G * wave / sk, g1 = G * (wave + 1) / sk;

    int64_t col[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t n = n0 + 16 * j + r;
        col[j] = n < args.n ? n : args.n - 1;
    }
    const uint16_t *arow[MB];
    bool mvalid[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int64_t m = m0 + 16 * mb + r;
        mvalid[mb] = m < args.rows;
        arow[mb] = args.a + (mvalid[mb] ? m : 0) * args.lda + 16 * c;
    }

    float acc[NW][J][MB][RPL];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < RPL; ++i) acc[w][j][mb][i] = 0.0f;

    const bf16x8 ones = ones_operand();
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

    // Register double buffer: the codes and sidecars of the next group are loaded while the
    // current one is used. Two named buffers keep every register index static.
    struct Stage {
        u32x2 wq[NW][J];
        uint16_t sv[NW][J], bv[NW][J];
    };
    auto load_group = [&](Stage &st, int64_t g) {
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int j = 0; j < J; ++j) {
                int64_t word, side;
                if (TILED) {
                    const int64_t rec = tiled_record(col[j], g, G);
                    word = rec * 8 + 2 * c;
                    side = rec;
                } else {
                    word = col[j] * args.stride_words + g * 8 + 2 * c;
                    side = col[j] * G + g;
                }
                st.wq[w][j] = *(const u32x2 *)(args.packed[w] + word);
                st.sv[w][j] = args.scales[w][side];
                st.bv[w][j] = args.biases[w][side];
            }
    };
    auto use_group = [&](const Stage &st, int64_t g) {
        bf16x8 a0[MB], a1[MB];
        f32x4 sx[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            u32x4 v0 = {0u, 0u, 0u, 0u}, v1 = {0u, 0u, 0u, 0u};
            if (mvalid[mb]) {
                const u32x4 *p = (const u32x4 *)(arow[mb] + g * kGroup);
                v0 = p[0];
                v1 = p[1];
            }
            a0[mb] = q4_act_operand(v0);
            a1[mb] = q4_act_operand(v1);
            sx[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[mb], ones, zero, 0, 0, 0);
            sx[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mb], ones, sx[mb], 0, 0, 0);
        }
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const bf16x8 b0 = q4_codes_operand(st.wq[w][j].x);
                const bf16x8 b1 = q4_codes_operand(st.wq[w][j].y);
                const float s = bf16_bits_to_f32(st.sv[w][j]);
                const float bp = __builtin_fmaf(-128.0f, s, bf16_bits_to_f32(st.bv[w][j]));
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[mb], b0, zero, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mb], b1, p, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < RPL; ++i)
                        acc[w][j][mb][i] = __builtin_fmaf(s, p[i], __builtin_fmaf(bp, sx[mb][i], acc[w][j][mb][i]));
                }
            }
    };

    Stage st0, st1;
    if (g0 < g1) load_group(st0, g0);
    for (int64_t g = g0; g < g1; g += 2) {
        if (g + 1 < g1) load_group(st1, g + 1);
        use_group(st0, g);
        if (g + 1 >= g1) break;
        if (g + 2 < g1) load_group(st0, g + 2);
        use_group(st1, g + 1);
    }

    constexpr int kPerWave = NW * J * MB * RPL * kWave;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < RPL; ++i)
                    red[wave * kPerWave + (((w * J + j) * MB + mb) * RPL + i) * kWave + lane] = acc[w][j][mb][i];
    __syncthreads();
    stream_finish<MB, J, RPL, NW>(red, sk, n0, m0, args.n, args.rows, args.out, args.ldc, args.out_dtype,
                                  args.residual);
}

StreamPlan plan_stream(int64_t rows, int64_t columns, int64_t groups, bool mlp, int max_j) {
    StreamPlan p;
    p.mb = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
    p.row_chunks = (int)((rows + 16 * p.mb - 1) / (16 * p.mb));
    p.rpl = rows == 1 ? 1 : rows == 2 ? 2 : 4;
    p.j = p.mb == 1 ? 4 : 2;
    if (p.j > max_j) p.j = max_j;
    while (p.j > 1 && ((columns + 16 * p.j - 1) / (16 * p.j)) * p.row_chunks < 256) p.j /= 2;
    p.col_blocks = (int)((columns + 16 * p.j - 1) / (16 * p.j));
    const int64_t wgs = (int64_t)p.col_blocks * p.row_chunks;
    int64_t sk = (4096 + wgs - 1) / wgs;
    if (sk > 8) sk = 8;
    if (sk > groups) sk = groups;
    if (sk < 1) sk = 1;
    const int64_t per_wave = (int64_t)(mlp ? 2 : 1) * p.j * p.mb * p.rpl * kWave * 4;
    while (sk > 1 && sk * per_wave > 65536) --sk;
    p.sk = (int)sk;
    return p;
}

template <int MB, int J, int RPL, int NW>
static hipError_t launch_q4_variant(const StreamPlan &plan, bool tiled, const Q4StreamArgs &args,
                                    hipStream_t stream) {
    dim3 grid((unsigned)plan.col_blocks, (unsigned)plan.row_chunks);
    dim3 block((unsigned)(plan.sk * kWave));
    const size_t lds = (size_t)plan.sk * NW * J * MB * RPL * kWave * sizeof(float);
    if (tiled)
        hipLaunchKernelGGL((q4_stream_kernel<MB, J, RPL, NW, true>), grid, block, lds, stream, args);
    else
        hipLaunchKernelGGL((q4_stream_kernel<MB, J, RPL, NW, false>), grid, block, lds, stream, args);
    return hipGetLastError();
}

template <int NW>
static hipError_t launch_q4_nw(const StreamPlan &p, bool tiled, const Q4StreamArgs &args, hipStream_t stream) {
#define SPLOSH_Q4_CASE(MB_, J_, RPL_)                                         \
    if (p.mb == MB_ && p.j == J_ && p.rpl == RPL_)                            \
        return launch_q4_variant<MB_, J_, RPL_, NW>(p, tiled, args, stream);
    SPLOSH_Q4_CASE(1, 4, 1) SPLOSH_Q4_CASE(1, 2, 1) SPLOSH_Q4_CASE(1, 1, 1)
    SPLOSH_Q4_CASE(1, 4, 2) SPLOSH_Q4_CASE(1, 2, 2) SPLOSH_Q4_CASE(1, 1, 2)
    SPLOSH_Q4_CASE(1, 4, 4) SPLOSH_Q4_CASE(1, 2, 4) SPLOSH_Q4_CASE(1, 1, 4)
    SPLOSH_Q4_CASE(2, 2, 4) SPLOSH_Q4_CASE(2, 1, 4)
    SPLOSH_Q4_CASE(4, 2, 4) SPLOSH_Q4_CASE(4, 1, 4)
#undef SPLOSH_Q4_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_q4_stream(const StreamPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                            const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                            const void *residual, int64_t rows, hipStream_t stream) {
    Q4StreamArgs args;
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
    return up ? launch_q4_nw<2>(plan, tiled, args, stream) : launch_q4_nw<1>(plan, tiled, args, stream);
}

}  // namespace splosh
