// prefill.hip -- q4 GEMM for prefill (hundreds to thousands of activation rows) on
// v_mfma_f32_32x32x16_bf16, two waves per SIMD.
//
// A workgroup of eight waves computes a 256 x 256 output tile; wave (wm, wn) = (wave / 4,
// wave % 4) owns rows 128 wm .. 128 wm + 127 of columns 64 wn .. 64 wn + 63 (4 x 2 MFMA tiles of
// 32 x 32: 128 fp32 accumulators a lane, in AGPRs). Per 64-group of K:
//  * the activations A[256][64] go straight into LDS (buffer loads with the LDS modifier), rows of
//    128 bytes whose 16-byte pieces are swizzled: piece P of row R sits at slot P ^ ((R / 2) mod 8),
//    so that a wave's writes are contiguous and the operand reads of 16 consecutive rows hit 16
//    different bank groups;
//  * every thread loads a 16-byte piece of one column's codes with that column's scale and bias,
//    dequantizes its four code words into bf16 (dequant_word_fp8, 19 instructions per 8 weights) and writes
//    them into the group's weight buffer ([256 columns][64 k], rows of 144 bytes: the operand reads
//    of 32 consecutive columns do not conflict). Every weight is dequantized once a workgroup.
//  * MFMA step i uses k = 32 h + 8 i .. + 7 for both operands, piece 4 h + i of a row or column.
// Two buffers: in step t the waves multiply out of buffer t mod 2 while group t + 1 fills buffer
// t + 1 mod 2 (its activations loaded at the start of the step, its codes loaded a step earlier and
// dequantized during the step) and group t + 2's codes are loaded; one barrier ends the step. With
// two waves on a SIMD one wave's dequantization and LDS traffic run while the other's MFMAs keep
// the matrix core busy.
//
// Work split. Tiles are numbered row block first (tile t: row block t mod MB, column block t / MB),
// so that with eight row blocks every XCD (workgroup id mod 8) works on one row block and keeps
// its activations in its L2. As in mma.hip, whole tiles go round-robin over the grid and the
// remaining tiles' (tile, group) pairs are split evenly over all workgroups (stream-K); a tile
// covered in part is summed by prefill_finish from fp32 partials in the caller's workspace.
//
// Numerics as mma.hip: fp32 dequantized weight rounded to bf16, exact products, fp32 sums.
#include "common.hpp"
#include "launch.hpp"
#include "gguf_decode.hpp"
#include "mix.hpp"

#include <cstdlib>

namespace splosh {

struct PrefillArgs {
    // q4: codes, scales, biases; Q5_K / Q4_K: plane0, plane1 (none for Q4_K), meta.
    const void *w[3];
    const void *u[3];   // fused gate+up: the up weight (same geometry as w)
    uint32_t w_bytes[3];
    int rows32;         // GGUF native blocks in the ROWS32 order (gguf_row)
    int64_t n;          // weight rows = output columns
    int64_t groups;     // 64-element groups of K
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
    int mblocks;        // row blocks of 256
    float *partial;     // stream-K partial tiles [gridDim.x][2][256][256]
    int dp_tiles;       // tiles computed whole (a multiple of gridDim.x)
    int64_t sk_units;   // (tile, group) pairs of the remaining tiles
    uint32_t a_bytes;
    // The next RMSNorm's operand, written from the epilogue (one weight, fp32 output, N % 64 == 0;
    // null norm_weight: none).
    EmitOperand emit;
};

constexpr int kPB = 256;                       // tile rows and columns
constexpr int kPRow = 144;                     // LDS bytes per weight column (128 + 16)
constexpr int kPABuf = kPB * kPRow;            // one weight buffer
constexpr int kPEpiRow = 68;                   // floats per row of a wave's epilogue staging
constexpr int kPEpi = 32 * kPEpiRow * 4;       // bytes of a wave's epilogue staging (32 rows)
constexpr int kPFinishMax = 1024;              // contributors prefill_finish can list

// Four output elements of row m, columns n .. n + 3, with the residual added; returns the values
// before the output's rounding.
__device__ __forceinline__ f32x4 prefill_out4(void *out, int64_t ldc, int out_dtype, const void *residual, int64_t m,
                                              int64_t n, f32x4 v) {
    const int64_t index = m * ldc + n;
    if (out_dtype == SPLOSH_F32) {
        if (residual) v += *(const f32x4 *)((const float *)residual + index);
        *(f32x4 *)((float *)out + index) = v;
    } else {
        if (residual) {
            const u32x2 rb = *(const u32x2 *)((const uint16_t *)residual + index);
            v[0] += bf16_bits_to_f32(rb[0] & 0xffffu);
            v[1] += bf16_bits_to_f32(rb[0] >> 16);
            v[2] += bf16_bits_to_f32(rb[1] & 0xffffu);
            v[3] += bf16_bits_to_f32(rb[1] >> 16);
        }
        const u32x2 pk = {f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
        *(u32x2 *)((uint16_t *)out + index) = pk;
    }
    return v;
}

// Emit (engine_na.metal:365-411 restated) for four fp32 outputs h of row m, columns n .. n + 3:
// values bf16(h w_norm) (RNE), and the row's sums over its 64-column band n / 64 of those rounded
// values and of h^2. The band's 64 columns are the four-column pieces of 16 consecutive lanes
// (lane % 16 = piece), summed by a shuffle tree; every lane of the wave calls it (`live` false
// past the rows or columns).
__device__ __forceinline__ void prefill_emit_band(const EmitOperand &e, int64_t n_total, int64_t m, int64_t n, f32x4 h,
                                                  bool live, int lane) {
    float sv = 0.0f, sq = 0.0f;
    if (live) {
        const u32x2 wb = *(const u32x2 *)(e.norm_weight + n);
        const float wn[4] = {bf16_bits_to_f32(wb[0] & 0xffffu), bf16_bits_to_f32(wb[0] >> 16),
                             bf16_bits_to_f32(wb[1] & 0xffffu), bf16_bits_to_f32(wb[1] >> 16)};
        uint32_t vb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vb[i] = f32_to_bf16(h[i] * wn[i]);
            sv += bf16_bits_to_f32(vb[i]);
            sq += h[i] * h[i];
        }
        const u32x2 pk = {vb[0] | (vb[1] << 16), vb[2] | (vb[3] << 16)};
        *(u32x2 *)(e.values + m * e.ldv + n) = pk;
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        sv += __shfl_xor(sv, o, 64);
        sq += __shfl_xor(sq, o, 64);
    }
    if (live && (lane & 15) == 0) {
        const int64_t at = m * (n_total / 64) + n / 64;
        e.sums[at] = sv;
        e.squares[at] = sq;
    }
}

// A wave's share of a finished tile: rows tr0 .. tr0 + 32 FM - 1 of columns tc0 .. tc0 + 63, one
// 32-row block at a time through the wave's own LDS area `epi` (over the operand buffers, once
// every wave is done with them): lane (r, h) holds row 8 (e / 4) + 4 h + e % 4, column 32 j + r;
// the rows are then written 16 bytes (4 columns) a lane, to the output (slot < 0) or to this
// workgroup's partial tile `slot`.
template <int FM, bool EMIT>
__device__ __forceinline__ void prefill_store_tile(const PrefillArgs &args, const f32x16 (&acc)[FM][2], char *epi,
                                                   int64_t m0, int64_t ncol, int tc0, int tr0, int lane, int slot) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int f = 0; f < FM; ++f) {
        const int tr = tr0 + 32 * f;  // the block's first row in the tile
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = 8 * (e >> 2) + 4 * h + (e & 3);
                *(float *)(epi + (row * kPEpiRow + 32 * j + r) * 4) = acc[f][j][e];
            }
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int idx = p * 64 + lane, row = idx >> 4, c4 = (idx & 15) * 4;
            const f32x4 v = *(const f32x4 *)(epi + (row * kPEpiRow + c4) * 4);
            const int64_t m = m0 + tr + row, n = ncol + c4;
            const bool live = m < args.rows && n < args.n;
            if (EMIT && slot < 0 && args.emit.norm_weight) {  // fp32 output, whole 64-column bands
                const f32x4 h = live ? prefill_out4(args.out, args.ldc, SPLOSH_F32, args.residual, m, n, v) : v;
                prefill_emit_band(args.emit, args.n, m, n, h, live, lane);
                continue;
            }
            if (!live) continue;
            if (slot >= 0) {
                float *dst = args.partial + ((int64_t)(blockIdx.x * 2 + slot) * kPB + tr + row) * kPB + tc0 + c4;
                *(f32x4 *)dst = v;
                continue;
            }
            prefill_out4(args.out, args.ldc, args.out_dtype, args.residual, m, n, v);
        }
    }
}

// The fused gate+up epilogue of a whole tile: the waves with wn = 0, 1 hold the gate's columns
// 64 wn .. + 63 of the tile, the waves with wn = 2, 3 the up weight's same columns. One 32-row
// block at a time every wave parks its block in its LDS area; then the gate waves read their own
// and their partner's (wave + 2) and write silu(g) * u. Every wave passes the same barriers.
template <int FM>
__device__ __forceinline__ void prefill_store_mlp(const PrefillArgs &args, const f32x16 (&acc)[FM][2], char *lds,
                                                  int wave, int64_t m0, int64_t ncol, int tr0, int lane) {
    const int r = lane & 31, h = lane >> 5;
    char *epi = lds + wave * kPEpi;
    const char *partner = lds + (wave + 2) * kPEpi;
    const bool gate = (wave & 3) < 2;
#pragma unroll
    for (int f = 0; f < FM; ++f) {
        const int tr = tr0 + 32 * f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = 8 * (e >> 2) + 4 * h + (e & 3);
                *(float *)(epi + (row * kPEpiRow + 32 * j + r) * 4) = acc[f][j][e];
            }
        lds_barrier();
        if (gate) {
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const int idx = p * 64 + lane, row = idx >> 4, c4 = (idx & 15) * 4;
                const f32x4 g = *(const f32x4 *)(epi + (row * kPEpiRow + c4) * 4);
                const f32x4 u = *(const f32x4 *)(partner + (row * kPEpiRow + c4) * 4);
                const int64_t m = m0 + tr + row, n = ncol + c4;
                if (m >= args.rows || n >= args.n) continue;
                const float o[4] = {silu(g[0]) * u[0], silu(g[1]) * u[1], silu(g[2]) * u[2], silu(g[3]) * u[3]};
                const int64_t index = m * args.ldc + n;
                if (args.out_dtype == SPLOSH_F32) {
                    const f32x4 v = {o[0], o[1], o[2], o[3]};
                    *(f32x4 *)((float *)args.out + index) = v;
                } else {
                    const u32x2 pk = {f32x2_to_bf16x2(o[0], o[1]), f32x2_to_bf16x2(o[2], o[3])};
                    *(u32x2 *)((uint16_t *)args.out + index) = pk;
                }
            }
        }
        lds_barrier();
    }
}

// The weights of one 64-element group of K for the tile's 256 columns: thread t loads the part
// of column t / 2 that covers k = 32 (t % 2) .. + 31 of the group, dequantizes it and writes the
// 64 bytes of bf16 weights into the weight buffer (four 16-byte pieces, `dst` = the first). Loads
// go to one of two register sets; kLoads loads a thread and group.

// MLX affine q4, TILED128: the thread's 16 bytes of the column's record (words 4 (t % 2) .. + 3)
// and the column's scale and bias (Retile.swift:135-153), dequantized by dequant_word_fp8.
struct Q4Stage {
    static constexpr int kLoads = 3, kNW = 1;
    static constexpr bool kEmit = true;  // the epilogue can write the next norm's operand
    rsrc_t q_rsrc, s_rsrc, b_rsrc;
    uint32_t c_src, s_src;
    u32x4 cr[2];
    uint32_t sr[2], br[2];
    __device__ Q4Stage(const PrefillArgs &args, bool up = false) {
        const void *const *w = up ? args.u : args.w;
        q_rsrc = make_rsrc(w[0], args.w_bytes[0]);
        s_rsrc = make_rsrc(w[1], args.w_bytes[1]);
        b_rsrc = make_rsrc(w[2], args.w_bytes[2]);
    }
    __device__ void begin(const PrefillArgs &args, uint32_t col, int hh) {
        const uint32_t rec = (col >> 7) * (uint32_t)args.groups * 128u + (col & 127u);
        c_src = rec * 32u + 16u * hh;
        s_src = rec * 2u;
    }
    __device__ void load(uint32_t g, int set) {
        cr[set] = buffer_load16_cp<2>(q_rsrc, c_src + g * (128u * 32u), 0);
        sr[set] = buffer_load_u16(s_rsrc, s_src + g * 256u, 0);
        br[set] = buffer_load_u16(b_rsrc, s_src + g * 256u, 0);
    }
    // Words q0 and q0 + 1, pieces q0 and q0 + 1.
    __device__ void store(char *dst, int set, uint32_t, bool on, int q0) {
        const float s = on ? bf16_bits_to_f32(sr[set]) : 0.0f, b = on ? bf16_bits_to_f32(br[set]) : 0.0f;
#pragma unroll
        for (int q = q0; q < q0 + 2; ++q) *(bf16x8 *)(dst + 16 * q) = dequant_word_fp8(cr[set][q], s, b);
    }
};

// Fused gate+up over two tiled q4 weights: the tile's 256 columns are 128 of the gate (threads
// 0 .. 255) and the same 128 of the up weight (threads 256 .. 511).
struct Q4PairStage : Q4Stage {
    static constexpr int kNW = 2;
    static constexpr bool kEmit = false;
    __device__ Q4PairStage(const PrefillArgs &args)
        : Q4Stage(args, __builtin_amdgcn_readfirstlane(threadIdx.x >> 8) != 0) {}
};

// GGUF Q5_K / Q4_K planes (GgufPlanes.swift:8-20, 62-74): the thread's 32-element group j of its
// 256-element block is one 16-byte plane0 record (nibbles in chunk order), one 4-byte plane1
// record (fifth bits; none for Q4_K) and the block's 16-byte meta record (fp16 d, dmin, packed
// 6-bit scales and minimums). In chunk order (gguf_formats.h:17-21) word c of the plane0 record
// holds elements 4c .. 4c + 3 and 16 + 4c .. 16 + 4c + 3: w & 0x0F0F0F0F has the codes of elements
// (4c, 16+4c, 4c+1, 16+4c+1) in its bytes and (w >> 4) & 0x0F0F0F0F those of (4c+2, 16+4c+2, 4c+3,
// 16+4c+3); the fifth bits reach bit 4 of those bytes by one multiply ((x & 0x33) * 0x880110 moves
// bits 0, 4, 1, 5 of plane1 byte c to bits 4, 12, 20, 28). Words 0 and 1 so give elements 0..7
// (bytes 0 and 2) and 16..23 (bytes 1 and 3), words 2 and 3 elements 8..15 and 24..31. The weight
// is code * (d sc) - dmin mn in one fma (both products exact in fp32, GgufQuant.swift:191-212),
// then RNE to bf16.
template <bool FIFTH>
struct Q5Stage {
    static constexpr int kLoads = FIFTH ? 3 : 2, kNW = 1;
    static constexpr bool kEmit = false;
    rsrc_t p0_rsrc, p1_rsrc, m_rsrc;
    uint32_t p0_src, p1_src, m_src;
    int hh;
    u32x4 p0[2], mr[2];
    uint32_t p1[2];
    __device__ Q5Stage(const PrefillArgs &args) {
        p0_rsrc = make_rsrc(args.w[0], args.w_bytes[0]);
        p1_rsrc = make_rsrc(FIFTH ? args.w[1] : args.w[0], FIFTH ? args.w_bytes[1] : 0u);
        m_rsrc = make_rsrc(args.w[2], args.w_bytes[2]);
    }
    __device__ void begin(const PrefillArgs &args, uint32_t col, int hh_) {
        hh = hh_;
        const uint32_t g32 = 2u * (uint32_t)args.groups, blocks = (uint32_t)args.groups / 4u;
        const uint32_t rec = ((col >> 7) * g32 + (uint32_t)hh) * 128u + (col & 127u);  // 32-group hh of group 0
        p0_src = rec * 16u;
        p1_src = rec * 4u;
        m_src = ((col >> 7) * blocks * 128u + (col & 127u)) * 16u;
    }
    // 64-group g: 32-groups 2 g and 2 g + 1, block g / 4.
    __device__ void load(uint32_t g, int set) {
        p0[set] = buffer_load16_cp<2>(p0_rsrc, p0_src + g * (2u * 128u * 16u), 0);
        if constexpr (FIFTH) p1[set] = buffer_load_u32(p1_rsrc, p1_src + g * (2u * 128u * 4u), 0);
        else p1[set] = 0u;
        mr[set] = buffer_load16(m_rsrc, m_src + (g >> 2) * (128u * 16u), 0);
    }
    // Words q0 and q0 + 1: pieces q0 / 2 (elements 8 (q0 / 2) .. + 7) and 2 + q0 / 2.
    __device__ void store(char *dst, int set, uint32_t g, bool on, int q0) {
        // Scale and minimum of 32-group j = (2 g + hh) mod 8 (GgufQuant.swift:196-203): packed byte
        // k is meta byte 4 + k; for j < 4 the low six bits of bytes 4 + j and 8 + j, else the
        // nibbles of byte 12 + (j - 4) joined with the top two bits of bytes 4 + (j - 4) and
        // 8 + (j - 4). j >= 4 is uniform (g & 2); the byte within its word is 2 (g & 1) + hh.
        const u32x4 m = mr[set];
        const uint32_t sh = 8u * (2u * (g & 1u) + (uint32_t)hh);
        uint32_t sc, mn;
        if ((g & 2u) == 0u) {
            sc = __builtin_amdgcn_ubfe(m[1], sh, 6);
            mn = __builtin_amdgcn_ubfe(m[2], sh, 6);
        } else {
            sc = __builtin_amdgcn_ubfe(m[3], sh, 4) | (__builtin_amdgcn_ubfe(m[1], sh + 6, 2) << 4);
            mn = __builtin_amdgcn_ubfe(m[3], sh + 4, 4) | (__builtin_amdgcn_ubfe(m[2], sh + 6, 2) << 4);
        }
        const float d = half_bits_to_f32(m[0]), dmin = half_bits_to_f32(m[0] >> 16);
        const float scaled = on ? d * (float)sc : 0.0f, offset = on ? -(dmin * (float)mn) : 0.0f;
        uint32_t lo[2], hi[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int c = q0 + e;
            const uint32_t w = p0[set][c];
            lo[e] = w & 0x0F0F0F0Fu;
            hi[e] = (w >> 4) & 0x0F0F0F0Fu;
            if constexpr (FIFTH) {
                const uint32_t x = __builtin_amdgcn_ubfe(p1[set], 8 * c, 8);
                lo[e] |= ((x & 0x33u) * 0x880110u) & 0x10101010u;
                hi[e] |= (((x >> 2) & 0x33u) * 0x880110u) & 0x10101010u;
            }
        }
        auto wt = [&](uint32_t codes, int j) { return __builtin_fmaf(cvt_byte(codes, j), scaled, offset); };
#pragma unroll
        for (int b = 0; b < 2; ++b) {  // bytes b and b + 2 of each word: the lower or upper elements
            u32x4 v;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                v[2 * e] = f32x2_to_bf16x2(wt(lo[e], b), wt(lo[e], b + 2));
                v[2 * e + 1] = f32x2_to_bf16x2(wt(hi[e], b), wt(hi[e], b + 2));
            }
            *(u32x4 *)(dst + 16 * (2 * b + q0 / 2)) = v;
        }
    }
};

// GGUF native blocks (Q8_0, Q3_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS; rows back to back): the thread's
// 32-element group 2 g + t % 2 of its column, fetched by gguf_fetch and decoded by gguf_decode in
// the reference's fp32 order (GgufQuant.swift), then rounded to bf16. The number of loads a group
// takes differs by format, so kLoads = 0: the step's wait takes every load.
template <int TYPE>
struct GgufStage {
    static constexpr int kLoads = 0, kNW = 1;
    static constexpr bool kEmit = false;
    rsrc_t r;
    GgufRow row;
    int hh;
    GgufRaw<TYPE> raw[2];
    __device__ GgufStage(const PrefillArgs &args) { r = make_rsrc(args.w[0], args.w_bytes[0]); }
    __device__ void begin(const PrefillArgs &args, uint32_t col, int hh_) {
        hh = hh_;
        const uint32_t row_bytes = (uint32_t)(args.groups * 64 / GgufGeom<TYPE>::kElems * GgufGeom<TYPE>::kBytes);
        row = gguf_row<TYPE>(col, row_bytes, args.rows32);
    }
    __device__ void load(uint32_t g, int set) { raw[set] = gguf_fetch<TYPE>(r, row, (int)(2u * g) + hh); }
    // The whole part at q0 = 0 (the decoders produce all 32 values at once), nothing at q0 = 2.
    __device__ void store(char *dst, int set, uint32_t, bool on, int q0) {
        if (q0 != 0) return;
        float v[32];
        gguf_decode<TYPE>(raw[set], v);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = on ? f32x2_to_bf16x2(v[8 * q + 2 * e], v[8 * q + 2 * e + 1]) : 0u;
            *(u32x4 *)(dst + 16 * q) = o;
        }
    }
};

// The kernel's buffers (see the top of the file).
constexpr int kSA = kPB * 128;                 // swizzled activations of a group
constexpr int kSBuf = kSA + kPABuf;            // activations and bf16 weights of a group
constexpr size_t kSLds = 2 * (size_t)kSBuf;
constexpr int kSALoads = 4;                    // activation loads (into LDS) of a wave and group
static_assert(8 * kPEpi <= (int)kSLds, "eight waves' epilogue staging fits the buffers");

template <class W>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
prefill_kernel(PrefillArgs args) {
    constexpr int kSCodeLoads = W::kLoads;
    constexpr int NW = W::kNW;          // 2: fused gate+up, 128 columns of each weight a tile
    constexpr int kTileCols = kPB / NW; // output columns a tile
    constexpr int FM = 4, kAPer = 4;
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / 4, wn = wave % 4;
    const int r = lane & 31, h = lane >> 5;
    const int G = (int)args.groups;
    const rsrc_t a_rsrc = make_rsrc(args.a, args.a_bytes);
    W wst(args);
    {
        // An AGPR operand makes the compiler select the AGPR form of the MFMAs: the accumulators
        // then live in AGPRs, beside a full set of 128 VGPRs.
        float agpr_use;
        asm volatile("v_accvgpr_write_b32 %0, 0" : "=a"(agpr_use));
        (void)agpr_use;
    }
    char *epi = lds + wave * kPEpi;
    // The operand slot of piece 4 h + i for this lane's rows (32-row blocks start at multiples of
    // 16 rows, so the swizzle only depends on r).
    const int swz = (r >> 1) & 7;

    auto run_job = [&](int tile, int ga, int gb, int slot) {
        const int mb = tile % args.mblocks, nb = tile / args.mblocks;
        const int64_t m0 = (int64_t)mb * kPB, n0 = (int64_t)nb * kTileCols;
        const int T = gb - ga;
        // Activation load p of this wave writes LDS bytes [8192 p + 1024 wave, + 1024): lane l takes
        // row 64 p + 8 wave + l / 8, slot l % 8, i.e. piece (l % 8) ^ ((row / 2) mod 8) (rows past
        // the last clamped).
        uint32_t a_src[kAPer];
#pragma unroll
        for (int p = 0; p < kAPer; ++p) {
            const int row = 64 * p + 8 * wave + (lane >> 3);
            const int piece = (lane & 7) ^ ((row >> 1) & 7);
            const int64_t m = m0 + row;
            a_src[p] = (uint32_t)(((m < args.rows ? m : args.rows - 1) * args.lda + piece * 8) * 2);
        }
        // The weights of column tid / 2, k = 32 (tid % 2) .. + 31 of each group (columns past the
        // last clamped).
        const int hh = tid & 1, sc = tid >> 1;
        {
            const int64_t nc = n0 + (sc & (kTileCols - 1));
            wst.begin(args, (uint32_t)(nc < args.n ? nc : args.n - 1), hh);
        }
        const uint32_t b_dst = (uint32_t)(kSA + sc * kPRow + 64 * hh);
        auto clampg = [&](int t) {
            const int g = ga + t < gb ? ga + t : gb - 1;
            return (uint32_t)__builtin_amdgcn_readfirstlane(g);
        };
        auto load_a = [&](int t, int buf) {
            const uint32_t g = clampg(t);
#pragma unroll
            for (int p = 0; p < kAPer; ++p)
                buffer_load_lds16(a_rsrc, lds + buf * kSBuf + 8192 * p + 1024 * wave, a_src[p] + g * 128u);
        };
        // Group t's weights in register set t mod 2.
        auto load_codes = [&](int t, int set) { wst.load(clampg(t), set); };
        // Group t's weights (half q0 / 2 of this thread's part) into buffer `buf`; zero weights
        // past the job (the step count is padded to even).
        auto store_b = [&](int buf, int set, int t, int q0) {
            wst.store(lds + buf * kSBuf + b_dst, set, clampg(t), t < T, q0);
        };
        // Operands of MFMA step i (k = 32 h + 8 i .. + 7 of the group, piece 4 h + i of a row).
        auto read_ops = [&](bf16x8 *af, bf16x8 *bw, int buf, int i) {
            const char *pa = lds + buf * kSBuf + (128 * wm + r) * 128 + (((4 * h + i) ^ swz) << 4);
#pragma unroll
            for (int f = 0; f < FM; ++f) af[f] = as_bf16x8(*(const u32x4 *)(pa + f * 32 * 128));
            const char *pb = lds + buf * kSBuf + kSA + (64 * wn + r) * kPRow + (4 * h + i) * 16;
#pragma unroll
            for (int j = 0; j < 2; ++j) bw[j] = as_bf16x8(*(const u32x4 *)(pb + j * 32 * kPRow));
        };

        f32x16 acc[FM][2];
#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[f][j][e] = 0.0f;

        // Prologue: group 0 into buffer 0, group 1's codes in flight.
        load_a(0, 0);
        load_codes(0, 0);
        store_b(0, 0, 0, 0);
        store_b(0, 0, 0, 2);
        __builtin_amdgcn_sched_barrier(0);
        load_codes(1, 1);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<kSCodeLoads>();  // group 0's activations have landed; group 1's codes may not
        lds_barrier_staged<0>();

        // Step t: buffer and code set d = t mod 2.
        auto step = [&](int t, int d) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // Group t + 1's activations into the other buffer and group t + 2's codes, a step
                // ahead of their use (pinned here, or the scheduler sinks them to the end of the
                // step); group t + 1's weights over MFMA steps 1 and 2.
                if (i == 0) {
                    load_a(t + 1, d ^ 1);
                    load_codes(t + 2, d);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // No operand prefetch: the other wave on the SIMD covers the read latency.
                bf16x8 af[FM], bw[2];
                read_ops(af, bw, d, i);
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int f = 0; f < FM; ++f)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[f], bw[j], acc[f][j], 0, 0, 0);
                if (i == 1 || i == 2) store_b(d ^ 1, d ^ 1, t + 1, 2 * (i - 1));
            }
            // Group t + 1's activations have landed (only group t + 2's code loads, issued after
            // them, may be outstanding), and every wave is done with buffer t mod 2.
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<kSCodeLoads>();
            lds_barrier_staged<0>();
        };
        const int Tp = (T + 1) / 2 * 2;
        for (int t0 = 0; t0 < Tp; t0 += 2) {
            step(t0, 0);
            step(t0 + 1, 1);
        }
        const int64_t ncol = n0 + ((64 * wn) & (kTileCols - 1));  // the wave's first output column
        if (NW == 2 && slot < 0)
            prefill_store_mlp<FM>(args, acc, lds, wave, m0, ncol, 32 * FM * wm, lane);
        else
            prefill_store_tile<FM, W::kEmit>(args, acc, epi, m0, ncol, 64 * wn, 32 * FM * wm, lane, slot);
    };

    const int P = gridDim.x;
    int dp_tile = blockIdx.x;
    int64_t u = args.sk_units * blockIdx.x / P;
    const int64_t u_end = args.sk_units * (blockIdx.x + 1) / P;
    int slot = 0;
    for (;;) {
        int tile, ga, gb, job_slot;
        if (dp_tile < args.dp_tiles) {
            tile = dp_tile;
            ga = 0;
            gb = G;
            job_slot = -1;
            dp_tile += P;
        } else if (u < u_end) {
            tile = args.dp_tiles + (int)(u / G);
            ga = (int)(u % G);
            gb = (int)((int64_t)ga + (u_end - u) < G ? ga + (u_end - u) : G);
            job_slot = (ga == 0 && gb == G) ? -1 : slot;
            u += gb - ga;
            slot = 1;
        } else {
            break;
        }
        run_job(tile, ga, gb, job_slot);
        lds_barrier();  // the next job stores into buffer 0, which slow waves may still read
    }
}

// Sums the stream-K partials of the remainder tiles in workgroup order and applies the epilogue.
// Block (rt, y) covers elements [1024 y, 1024 y + 1024) of remainder tile rt, four a thread; its
// first thread lists the tile's contributing workgroups once (see q4_mma_finish).
__global__ void __launch_bounds__(256)
prefill_finish(const float *__restrict__ partial, int dp_tiles, int64_t sk_units, int P, int64_t groups,
                  int mblocks, int64_t rows, int64_t n, void *out, int64_t ldc, int out_dtype, const void *residual,
                  int nw, EmitOperand emit) {
    __shared__ int wg[kPFinishMax];
    __shared__ int slot_of[kPFinishMax];
    __shared__ int count;
    const int64_t rt = blockIdx.x;
    const int64_t lo = rt * groups, hi = lo + groups;
    if (threadIdx.x == 0) {
        const int i_lo = (int)(((lo + 1) * P - 1) / sk_units), i_hi = (int)((hi * P - 1) / sk_units);
        int c = 0;
        for (int i = i_lo; i <= i_hi && c < kPFinishMax; ++i) {
            const int64_t s = sk_units * i / P, e = sk_units * (i + 1) / P;
            if (s == e) continue;
            wg[c] = i;
            slot_of[c] = s < lo ? 1 : 0;
            ++c;
        }
        count = c;
    }
    __syncthreads();
    const int contributors = count;
    if (contributors <= 1) return;  // one workgroup covered the tile and wrote it
    const int tile = dp_tiles + (int)rt;
    const int cols = kPB / nw;  // output columns a tile (nw = 2: gate at tc, up at tc + 128)
    const int64_t m0 = (int64_t)(tile % mblocks) * kPB, n0 = (int64_t)(tile / mblocks) * cols;
    const int e0 = (blockIdx.y * 256 + threadIdx.x) * 4;  // element of the tile
    const int tr = e0 / cols, tc = e0 % cols;
    const int64_t m = m0 + tr, col = n0 + tc;
    const bool live = m < rows && col < n;
    if (!live && !emit.norm_weight) return;
    auto sum_at = [&](int c) {
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j0 = 0; j0 < contributors; j0 += 8) {
            f32x4 x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int jj = j0 + j < contributors ? j0 + j : contributors - 1;
                x[j] = *(const f32x4 *)(partial + ((int64_t)(wg[jj] * 2 + slot_of[jj]) * kPB + tr) * kPB + c);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j0 + j < contributors) v += x[j];
        }
        return v;
    };
    f32x4 v = sum_at(tc);
    if (nw == 2) {
        const f32x4 u = sum_at(tc + cols);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = silu(v[e]) * u[e];
    }
    if (emit.norm_weight) {
        // One weight, fp32 output: a row's 256 columns are the 64 lanes of one wave, a 64-column
        // band 16 consecutive lanes.
        const f32x4 h = live ? prefill_out4(out, ldc, SPLOSH_F32, residual, m, col, v) : v;
        prefill_emit_band(emit, n, m, col, h, live, (int)threadIdx.x & 63);
        return;
    }
    prefill_out4(out, ldc, out_dtype, residual, m, col, v);
}

// One tiled weight, 16-byte aligned rows of activations and outputs (vector epilogue), 32-bit
// byte offsets.
bool prefill_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda, int64_t ldc) {
    const int64_t limit = ((int64_t)1 << 32) - 256;
    return rows >= 1 && columns > 0 && columns % 128 == 0 && inner >= 64 && lda % 8 == 0 && ldc % 4 == 0 &&
           (rows * lda + inner) * 2 < limit && columns * (inner / 64) * 32 < limit;
}

static int prefill_grid() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    // A development override of the grid, read from the environment once per process.
    static const int grid_override = [] { const char *e = getenv("SPLOSH_PREFILL_GRID"); return e ? atoi(e) : 0; }();
    if (grid_override > 0) cus = grid_override;
    return cus < kPFinishMax ? cus : kPFinishMax;
}

// The workspace's first 16 KiB hold the other kernels' arrival counters (left at zero between
// calls); the partial tiles follow them.
constexpr size_t kPCounterBytes = 16384;
static size_t prefill_sk_bytes(int grid) { return kPCounterBytes + (size_t)grid * 2 * kPB * kPB * sizeof(float); }

PrefillPlan plan_prefill(int64_t rows, int64_t columns, int64_t groups, size_t workspace_bytes) {
    PrefillPlan p;
    p.mblocks = (int)((rows + kPB - 1) / kPB);
    p.tiles = p.mblocks * (int)((columns + kPB - 1) / kPB);
    p.grid = prefill_grid();
    p.dp_tiles = (p.tiles / p.grid) * p.grid;
    p.sk_units = (int64_t)(p.tiles - p.dp_tiles) * groups;
    if (p.sk_units > 0 && prefill_sk_bytes(p.grid) > workspace_bytes) {
        // No room for partials: every tile whole, one workgroup each.
        p.grid = p.tiles;
        p.dp_tiles = p.tiles;
        p.sk_units = 0;
    }
    return p;
}

size_t prefill_workspace_bytes(int64_t rows, int64_t columns, int64_t groups) {
    const PrefillPlan p = plan_prefill(rows, columns, groups, (size_t)-1);
    return p.sk_units > 0 ? prefill_sk_bytes(p.grid) : 0;
}

template <class W>
static hipError_t launch_prefill(const PrefillPlan &plan, PrefillArgs &args, int64_t n, int64_t inner,
                                 const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                                 const void *residual, int64_t rows, void *workspace, hipStream_t stream) {
    args.n = n;
    args.groups = inner / kGroup;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = rows;
    args.out_dtype = out_dtype;
    args.mblocks = plan.mblocks;
    args.partial = plan.sk_units > 0 ? (float *)((char *)workspace + kPCounterBytes) : nullptr;
    args.dp_tiles = plan.dp_tiles;
    args.sk_units = plan.sk_units;
    args.a_bytes = (uint32_t)(((rows - 1) * lda + inner) * 2);
    static bool once = [] {
        (void)hipFuncSetAttribute((const void *)prefill_kernel<W>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)kSLds);
        return true;
    }();
    (void)once;
    hipLaunchKernelGGL(prefill_kernel<W>, dim3((unsigned)plan.grid), dim3(512), kSLds, stream, args);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || plan.sk_units == 0) return err;
    const int remainder = plan.tiles - plan.dp_tiles;
    hipLaunchKernelGGL(prefill_finish, dim3((unsigned)remainder, kPB * kPB / 1024 / W::kNW), dim3(256), 0, stream,
                       (const float *)args.partial, plan.dp_tiles, plan.sk_units, plan.grid, args.groups, plan.mblocks,
                       rows, n, out, ldc, out_dtype, residual, W::kNW, args.emit);
    return hipGetLastError();
}

hipError_t launch_q4_prefill(const PrefillPlan &plan, const splosh_q4_weight &w, const uint16_t *a, int64_t lda,
                             void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                             void *workspace, hipStream_t stream, const EmitOperand *emit) {
    PrefillArgs args = {};
    if (emit) args.emit = *emit;
    const int64_t groups = w.inner / kGroup;
    args.w[0] = w.packed;
    args.w[1] = w.scales;
    args.w[2] = w.biases;
    args.w_bytes[0] = (uint32_t)(w.rows * groups * 32);
    args.w_bytes[1] = args.w_bytes[2] = (uint32_t)(w.rows * groups * 2);
    return launch_prefill<Q4Stage>(plan, args, w.rows, w.inner, a, lda, out, ldc, out_dtype, residual, rows,
                                   workspace, stream);
}

hipError_t launch_q4_prefill_mlp(const PrefillPlan &plan, const splosh_q4_weight &gate, const splosh_q4_weight &up,
                                 const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, int64_t rows,
                                 void *workspace, hipStream_t stream) {
    PrefillArgs args = {};
    const int64_t groups = gate.inner / kGroup;
    args.w[0] = gate.packed;
    args.w[1] = gate.scales;
    args.w[2] = gate.biases;
    args.u[0] = up.packed;
    args.u[1] = up.scales;
    args.u[2] = up.biases;
    args.w_bytes[0] = (uint32_t)(gate.rows * groups * 32);
    args.w_bytes[1] = args.w_bytes[2] = (uint32_t)(gate.rows * groups * 2);
    return launch_prefill<Q4PairStage>(plan, args, gate.rows, gate.inner, a, lda, out, ldc, out_dtype, nullptr, rows,
                                       workspace, stream);
}

bool q5k_prefill_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda, int64_t ldc) {
    const int64_t limit = ((int64_t)1 << 32) - 256;
    return inner % 256 == 0 && prefill_fits(rows, columns, inner, lda, ldc) && columns * (inner / 32) * 16 < limit;
}

hipError_t launch_q5k_prefill(const PrefillPlan &plan, const splosh_q5k_weight &w, bool fifth, const uint16_t *a,
                              int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                              void *workspace, hipStream_t stream) {
    PrefillArgs args = {};
    args.w[0] = w.plane0;
    args.w[1] = fifth ? (const void *)w.plane1 : nullptr;
    args.w[2] = w.meta;
    args.w_bytes[0] = (uint32_t)(w.rows * (w.inner / 32) * 16);
    args.w_bytes[1] = fifth ? (uint32_t)(w.rows * (w.inner / 32) * 4) : 0u;
    args.w_bytes[2] = (uint32_t)(w.rows * (w.inner / 256) * 16);
    if (fifth)
        return launch_prefill<Q5Stage<true>>(plan, args, w.rows, w.inner, a, lda, out, ldc, out_dtype, residual,
                                             rows, workspace, stream);
    return launch_prefill<Q5Stage<false>>(plan, args, w.rows, w.inner, a, lda, out, ldc, out_dtype, residual, rows,
                                          workspace, stream);
}

bool gguf_prefill_fits(int type, int64_t rows, int64_t columns, int64_t inner, int64_t lda, int64_t ldc) {
    int elems = 0, bytes = 0;
    if (!gguf_native_block(type, &elems, &bytes)) return false;
    return inner % 64 == 0 && inner % elems == 0 && prefill_fits(rows, columns, inner, lda, ldc) &&
           (columns + 31) * (inner / elems) * bytes < ((int64_t)1 << 32) - 256;
}

hipError_t launch_gguf_prefill(const PrefillPlan &plan, int type, const uint8_t *native, int64_t rows_w,
                               int64_t inner, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                               const void *residual, int64_t rows, void *workspace, hipStream_t stream) {
    int elems = 0, bytes = 0;
    if (!gguf_native_block(type, &elems, &bytes)) return hipErrorInvalidValue;
    PrefillArgs args = {};
    args.rows32 = gguf_layout(type);
    args.w[0] = native;
    args.w_bytes[0] = (uint32_t)((args.rows32 ? (rows_w + 31) / 32 * 32 : rows_w) * (inner / elems) * bytes);
#define SPLOSH_GGUF_PREFILL(T) \
    launch_prefill<GgufStage<T>>(plan, args, rows_w, inner, a, lda, out, ldc, out_dtype, residual, rows, workspace, stream)
    switch (type) {
        case 8: return SPLOSH_GGUF_PREFILL(8);
        case 11: return SPLOSH_GGUF_PREFILL(11);
        case 14: return SPLOSH_GGUF_PREFILL(14);
        case 20: return SPLOSH_GGUF_PREFILL(20);
        case 21: return SPLOSH_GGUF_PREFILL(21);
        default: return SPLOSH_GGUF_PREFILL(23);
    }
#undef SPLOSH_GGUF_PREFILL
}

}  // namespace splosh
