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
// Two barriers a step; a step's global reads go out one step ahead. With few tiles K is split over
// workgroups, whose fp32 partials a second pass (gguf_tile_finish) sums in slice order.
//
// Numerics: the weight is the decoder's fp32 value rounded to bf16 (RNE), products exact in fp32,
// fp32 accumulation -- as the q4 MFMA kernels.
#include "common.hpp"
#include "gguf_decode.hpp"
#include "launch.hpp"

#include <type_traits>

namespace splosh {

constexpr int kGtStride = 72;       // bf16 elements per LDS row: 64 + 8 padding (144 bytes)
constexpr int kGtCounterBytes = 16384;  // reserved at the start of the workspace (partials follow)
constexpr int kGtMaxSplitTiles = kGtCounterBytes / 4;
constexpr int kGtMaxSplits = 32;        // K slices at most
constexpr int kGtCpol = 1 | 16;         // partials written through to memory (sc0 sc1)
constexpr int kGtSqStride = 36;         // floats a row of a wave's 32 x 32 epilogue square

struct GgufTileArgs {
    const uint8_t *w;          // native blocks (rows back to back), or plane0 for Q5_K / Q4_K
    const uint8_t *plane1, *meta;
    uint32_t w_bytes, row_bytes;
    int rows32;                // native blocks in the ROWS32 order (gguf_row)
    int64_t n, inner;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
    int vector_out;            // out / residual 16-byte aligned and ldc % 8 == 0: 16-byte stores
    int splits;                // K slices (gridDim.z); > 1 needs the workspace
    char *partial;             // [tiles][splits][256 threads][FM FN 16] fp32
    uint32_t partial_bytes;
};

// TYPE: a ggml type id; 13 / 12 = Q5_K / Q4_K planes.
template <int TYPE, int FM, int FN, bool SPLIT, int KH>
__global__ void __launch_bounds__(256 * KH) gguf_tile_kernel(GgufTileArgs args) {
    constexpr int BM = 64 * FM, BN = 64 * FN;
    constexpr int kAChunks = BM * 8;        // 16-byte chunks of the A tile
    constexpr int kAPer = kAChunks / 256;
    static_assert(BN == 128, "one 32-element weight group a thread");
    extern __shared__ __align__(16) uint16_t lds[];
    // KH K-halves: half kh (threads 256 kh ..) takes the 64-element steps s with s % KH == kh of
    // the slice into operand tiles of its own; the halves' sums meet in LDS at the end.
    const int kh = KH > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8) : 0;
    uint16_t *sA = lds + kh * (BM + BN) * kGtStride, *sB = sA + BM * kGtStride;

    const int tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r = lane & 31, h = lane >> 5;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int steps = (int)(args.inner / 64);
    // This workgroup's K slice: steps [s_lo, s_hi).
    const int z = blockIdx.z, S = args.splits;
    const int s_lo = (int)((int64_t)steps * z / S), s_hi = (int)((int64_t)steps * (z + 1) / S);
    const rsrc_t wr = make_rsrc(args.w, args.w_bytes);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // One step's global reads, held in registers: this thread's pieces of the activation tile and
    // the raw bytes of its weight group (column tid / 2, half tid % 2 of the 64 elements). They are
    // fetched a step ahead, so that their latency overlaps the previous step's decode and MFMAs.
    constexpr bool kPlanes = TYPE == 13 || TYPE == 12;
    using Raw = typename std::conditional<kPlanes, PlaneRaw, GgufRaw<kPlanes ? 8 : TYPE>>::type;
    struct Stage {
        u32x4 a[kAPer];
        Raw w;
    };
    const int col = tid >> 1, half = tid & 1;
    const int64_t wcol = n0 + col < args.n ? n0 + col : args.n - 1;
    auto fetch = [&](Stage &st, int step) {
#pragma unroll
        for (int p = 0; p < kAPer; ++p) {
            const int c = p * 256 + tid, row = c >> 3, chunk = c & 7;
            const int64_t m = m0 + row;
            st.a[p] = u32x4{0u, 0u, 0u, 0u};
            if (m < args.rows) st.a[p] = *(const u32x4 *)(args.a + m * args.lda + (int64_t)step * 64 + chunk * 8);
        }
        const int64_t g = (int64_t)step * 2 + half;
        if constexpr (kPlanes)
            st.w = fetch_plane_group(args.w, TYPE == 13 ? args.plane1 : nullptr, args.meta, args.inner, wcol, g);
        else
            st.w = gguf_fetch<TYPE>(wr, gguf_row<TYPE>((uint32_t)wcol, args.row_bytes, args.rows32), (int)g);
    };
    auto commit = [&](const Stage &st) {
#pragma unroll
        for (int p = 0; p < kAPer; ++p) {
            const int c = p * 256 + tid, row = c >> 3, chunk = c & 7;
            *(u32x4 *)(sA + row * kGtStride + chunk * 8) = st.a[p];
        }
        float v[32];
        if constexpr (kPlanes)
            decode_plane(st.w, v);
        else
            gguf_decode<TYPE>(st.w, v);
        uint16_t *dst = sB + col * kGtStride + 32 * half;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4 d;
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e] = f32x2_to_bf16x2(v[8 * q + 2 * e], v[8 * q + 2 * e + 1]);
            *(u32x4 *)(dst + 8 * q) = d;
        }
    };
    const uint16_t *A = sA + (wm * FM * 32 + r) * kGtStride + 8 * h;
    const uint16_t *B = sB + (wn * FN * 32 + r) * kGtStride + 8 * h;
    auto multiply = [&] {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 af[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = as_bf16x8(*(const u32x4 *)(A + i * 32 * kGtStride + 16 * ks));
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const bf16x8 bf = as_bf16x8(*(const u32x4 *)(B + j * 32 * kGtStride + 16 * ks));
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf, acc[i][j], 0, 0, 0);
            }
        }
    };

    Stage cur, nxt;
    if (s_lo + kh < s_hi) fetch(cur, s_lo + kh);
    for (int s = s_lo + kh; s - kh < s_hi; s += KH) {
        const bool on = s < s_hi;  // wave-uniform: a half whose last step is past the slice idles
        if (s + KH < s_hi) fetch(nxt, s + KH);
        if (on) commit(cur);
        __syncthreads();
        if (on) multiply();
        __syncthreads();
        cur = nxt;
    }
    if constexpr (KH > 1) {
        // Half 1 hands its sums to half 0 (thread for thread) through LDS; half 0 goes on alone.
        float *sx = (float *)lds;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (kh == 1)
                        *(f32x4 *)(sx + (((i * FN + j) * 4 + q) * 256 + tid) * 4) =
                            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        __syncthreads();
        if (kh == 1) return;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 t = *(const f32x4 *)(sx + (((i * FN + j) * 4 + q) * 256 + tid) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += t[e];
                }
    }

    // The epilogue takes one 32 x 32 block of a wave at a time through a wave-private LDS
    // square (the operand tiles are no longer read): element e of lane (r, h) -- row
    // 8 (e / 4) + 4 h + e % 4, column r -- goes in, and lane l takes out row l / 2, columns
    // 16 (l % 2) .. + 16, so that the stores to the output (and the residual loads) are 64 or 32
    // contiguous bytes a lane.
    float *sq = (float *)lds + (KH > 1 ? FM * FN * 4 * 256 * 4 : 0) + wave * 32 * kGtSqStride;
    auto store_block = [&](int i, int j, const f32x16 &v) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sq[(8 * (e >> 2) + 4 * h + (e & 3)) * kGtSqStride + r] = v[e];
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's writes are done
        __builtin_amdgcn_wave_barrier();
        float o[16];
        const int orow = lane >> 1, ocol = 16 * (lane & 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x4 t = *(const f32x4 *)(sq + orow * kGtSqStride + ocol + 4 * c);
            o[4 * c] = t[0], o[4 * c + 1] = t[1], o[4 * c + 2] = t[2], o[4 * c + 3] = t[3];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();  // the square is read before the next block writes it
        const int64_t m = m0 + wm * FM * 32 + i * 32 + orow;
        const int64_t n = n0 + wn * FN * 32 + j * 32 + ocol;
        if (m >= args.rows) return;
        const int64_t index = m * args.ldc + n;
        const int valid = args.n - n >= 16 ? 16 : (int)(args.n - n);
        if (valid == 16 && args.vector_out) {
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) {
                    const f32x4 *res = (const f32x4 *)((const float *)args.residual + index);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const f32x4 t = res[c];
                        o[4 * c] += t[0], o[4 * c + 1] += t[1], o[4 * c + 2] += t[2], o[4 * c + 3] += t[3];
                    }
                }
                f32x4 *dst = (f32x4 *)((float *)args.out + index);
#pragma unroll
                for (int c = 0; c < 4; ++c) dst[c] = f32x4{o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]};
            } else {
                if (args.residual) {
                    const u32x4 *res = (const u32x4 *)((const uint16_t *)args.residual + index);
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const u32x4 t = res[c];
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            o[8 * c + 2 * k] += bf16_bits_to_f32(t[k] & 0xffffu);
                            o[8 * c + 2 * k + 1] += bf16_bits_to_f32(t[k] >> 16);
                        }
                    }
                }
                u32x4 *dst = (u32x4 *)((uint16_t *)args.out + index);
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    u32x4 t;
#pragma unroll
                    for (int k = 0; k < 4; ++k) t[k] = f32x2_to_bf16x2(o[8 * c + 2 * k], o[8 * c + 2 * k + 1]);
                    dst[c] = t;
                }
            }
            return;
        }
        for (int c = 0; c < valid; ++c) {
            float value = o[0];
#pragma unroll
            for (int k = 1; k < 16; ++k) value = c == k ? o[k] : value;
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) value += ((const float *)args.residual)[index + c];
                ((float *)args.out)[index + c] = value;
            } else {
                if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index + c]);
                ((uint16_t *)args.out)[index + c] = f32_to_bf16(value);
            }
        }
    };
    if constexpr (!SPLIT) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) store_block(i, j, acc[i][j]);
        return;
    } else {

    // Split K: every slice writes its accumulators (16-byte pieces, [tile][slice][thread] order,
    // coalesced); gguf_tile_finish sums them.
    constexpr int kPer = FM * FN * 16;  // floats a thread
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const rsrc_t pr = make_rsrc(args.partial, args.partial_bytes);
    auto off = [&](int slice, int piece) {
        return (uint32_t)((((int64_t)tile * S + slice) * 256 + tid) * kPer + 4 * piece) * 4u;
    };
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), pr, off(z, (i * FN + j) * 4 + q),
                                                       0, kGtCpol);
            }
    }
}

// Split K, second pass: sums the slices' partials of every tile in slice order (so the result does
// not depend on timing) and writes the outputs. Block (tile, p) takes accumulator quarter p of all
// 256 threads of the split kernel: thread t's quarter holds rows 8 (e / 4) + 4 h + e % 4 of one
// column, in the MFMA output layout the split kernel wrote them in.
template <int FM, int FN>
__global__ void __launch_bounds__(256) gguf_tile_finish(GgufTileArgs args) {
    constexpr int kPer = FM * FN * 16;
    const int tile = blockIdx.x, p = blockIdx.y;  // p: (i FN + j) 4 + q
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, r = lane & 31, h = lane >> 5;
    const int S = args.splits;
    const int tiles_n = (int)((args.n + 64 * FN - 1) / (64 * FN));
    const int64_t m0 = (int64_t)(tile / tiles_n) * 64 * FM, n0 = (int64_t)(tile % tiles_n) * 64 * FN;
    const rsrc_t pr = make_rsrc(args.partial, args.partial_bytes);
    auto off = [&](int slice) { return (uint32_t)((((int64_t)tile * S + slice) * 256 + tid) * kPer + 4 * p) * 4u; };
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < S; s0 += 4) {
        f32x4 part[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            part[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off(s0 + k < S ? s0 + k : 0), 0, kGtCpol));
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (s0 + k < S) sum += part[k];
    }
    const int i = p / (FN * 4), j = (p / 4) % FN, q = p % 4;
    const int64_t n = n0 + wn * FN * 32 + j * 32 + r;
    if (n >= args.n) return;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm * FM * 32 + i * 32 + 8 * q + 4 * h + e;
        if (m >= args.rows) continue;
        const int64_t index = m * args.ldc + n;
        float value = sum[e];
        if (args.out_dtype == SPLOSH_F32) {
            if (args.residual) value += ((const float *)args.residual)[index];
            ((float *)args.out)[index] = value;
        } else {
            if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
            ((uint16_t *)args.out)[index] = f32_to_bf16(value);
        }
    }
}

// Tile shapes (BM x 128 columns): 64 rows up to 64 activation rows, 128 up to 128, 256 above.
// K-halves a workgroup at 64-row tiles (two: eight waves, two a SIMD instead of about one).
static int gt_kh() {
    static const int kh = [] {
        const char *e = getenv("SPLOSH_GGUF_TILE_KH");
        return e && atoi(e) == 1 ? 1 : 2;
    }();
    return kh;
}

static int gt_fm(int64_t rows) {
    static const int forced = [] {
        const char *e = getenv("SPLOSH_GGUF_TILE_FM");
        return e ? atoi(e) : 0;
    }();
    if (forced == 1 || forced == 2) return forced;
    return rows <= 64 ? 1 : 2;
}

// K slices: enough workgroups for about 1.5 a CU (measured best among 1.25, 1.5, 2, 2.5, 4 and 8
// a CU at K17408 -> N5120, M=16 and 64, for Q8_0, Q6_K, IQ3_S and Q5_K at M=128), at least four
// 64-element steps a slice, and only with room in the workspace.
static int gt_splits(int64_t rows, int64_t n, int64_t inner, size_t workspace_bytes) {
    const int fm = gt_fm(rows);
    const int64_t tiles = ((rows + 64 * fm - 1) / (64 * fm)) * ((n + 127) / 128);
    static const int target = [] {
        const char *e = getenv("SPLOSH_GGUF_TILE_WGS");
        if (e && atoi(e) > 0) return atoi(e);
        int dev = 0, cus = 256;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        return cus * 25 / 16;
    }();
    int64_t s = (target + tiles - 1) / tiles;
    const int64_t most = inner / 64 / 4;
    if (s > most) s = most;
    if (s > kGtMaxSplits) s = kGtMaxSplits;
    if (s <= 1 || tiles > kGtMaxSplitTiles) return 1;
    auto need = [&](int64_t k) { return (size_t)kGtCounterBytes + (size_t)(tiles * k * 256 * fm * 2 * 16 * 4); };
    while (s > 1 && (need(s) > workspace_bytes || need(s) >= ((size_t)1 << 31))) --s;
    return (int)s;
}

size_t gguf_tile_workspace_bytes(int64_t rows, int64_t n, int64_t inner) {
    const int s = gt_splits(rows, n, inner, (size_t)-1);
    if (s <= 1) return 0;
    const int fm = gt_fm(rows);
    const int64_t tiles = ((rows + 64 * fm - 1) / (64 * fm)) * ((n + 127) / 128);
    return (size_t)kGtCounterBytes + (size_t)tiles * s * 256 * fm * 2 * 16 * 4;
}

// LDS of one launch: KH pairs of operand tiles; with two K-halves also the hand-over of half 1's
// sums followed by the epilogue squares (which must not overlap it).
template <int FM, int FN, int KH>
constexpr size_t gt_lds_bytes() {
    const size_t tiles = (size_t)KH * (64 * FM + 64 * FN) * kGtStride * 2;
    const size_t tail = KH > 1 ? (size_t)FM * FN * 16 * 256 * 4 + 4 * 32 * kGtSqStride * 4 : 0;
    return tiles > tail ? tiles : tail;
}

template <int TYPE, int FM, int FN, int KH = 1>
static hipError_t launch_gt(const GgufTileArgs &args, hipStream_t stream) {
    constexpr int BM = 64 * FM, BN = 64 * FN;
    constexpr size_t lds = gt_lds_bytes<FM, FN, KH>();
    static_assert(lds <= 160 * 1024, "LDS of one workgroup");
    const dim3 grid((unsigned)((args.n + BN - 1) / BN), (unsigned)((args.rows + BM - 1) / BM), (unsigned)args.splits);
    // The split variant is a kernel of its own: its summing code needs registers that would
    // otherwise cost the unsplit kernel occupancy.
    if (args.splits > 1) {
        hipLaunchKernelGGL((gguf_tile_kernel<TYPE, FM, FN, true, KH>), grid, dim3(256 * KH), lds, stream, args);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        hipLaunchKernelGGL((gguf_tile_finish<FM, FN>), dim3(grid.x * grid.y, FM * FN * 4), dim3(256), 0, stream, args);
    } else {
        hipLaunchKernelGGL((gguf_tile_kernel<TYPE, FM, FN, false, KH>), grid, dim3(256 * KH), lds, stream, args);
    }
    return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_gt_rows(const GgufTileArgs &args, hipStream_t stream) {
    switch (gt_fm(args.rows)) {
        case 1: return gt_kh() > 1 ? launch_gt<TYPE, 1, 2, 2>(args, stream) : launch_gt<TYPE, 1, 2>(args, stream);
        default: return launch_gt<TYPE, 2, 2>(args, stream);
    }
}

bool gguf_tile_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda) {
    const int64_t limit = ((int64_t)1 << 31);
    return rows >= 1 && rows <= 65535LL * 64 && columns > 0 && inner % 64 == 0 && lda % 8 == 0 &&
           rows * lda < limit;
}

hipError_t launch_gguf_tile(int type, const uint8_t *w, const uint8_t *plane1, const uint8_t *meta, int64_t rows_w,
                            int64_t inner, const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                            const void *residual, int64_t m, void *workspace, size_t workspace_bytes,
                            hipStream_t stream) {
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
    args.vector_out = ((uintptr_t)out % 16 == 0) && ((uintptr_t)residual % 16 == 0) && ldc % 8 == 0;
    args.splits = workspace ? gt_splits(m, rows_w, inner, workspace_bytes) : 1;
    if (args.splits > 1) {
        args.partial = (char *)workspace + kGtCounterBytes;
        const size_t room = workspace_bytes - kGtCounterBytes;
        args.partial_bytes = (uint32_t)(room < ((size_t)1 << 31) ? room : ((size_t)1 << 31));
    }
    args.rows32 = gguf_layout(type);
    if (type != 13 && type != 12) {
        int elems = 0, bytes = 0;
        gguf_native_block(type, &elems, &bytes);
        args.row_bytes = (uint32_t)(inner / elems * bytes);
        args.w_bytes = (uint32_t)((args.rows32 ? (rows_w + 31) / 32 * 32 : rows_w) * (int64_t)args.row_bytes);
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
