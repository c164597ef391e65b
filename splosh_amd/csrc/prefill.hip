// prefill.hip -- q4 GEMM for prefill (hundreds to thousands of activation rows) on
// v_mfma_f32_32x32x16_bf16, one wave per SIMD.
//
// A workgroup of four waves computes a 256 x 256 output tile; wave w owns all 256 rows of columns
// 64 w .. 64 w + 63 (8 x 2 MFMA tiles of 32 x 32: 256 fp32 accumulators a lane, held in AGPRs,
// which is why the kernel runs one wave per SIMD). Per 64-group of K, one "chunk":
//  * The chunk's activations A[256][64] (32 KB), codes (256 columns x 32 bytes) and sidecars are
//    staged global -> registers -> LDS by all threads, one group ahead, into one of three buffers
//    (row strides 144 and 48 bytes: the operand and code reads do not conflict), with one barrier
//    per group, in its middle.
//  * Lane (r, h) of wave w reads the 16 bytes of the record of column 64 w + 32 j + r (j = 0, 1)
//    that hold words 4 h .. 4 h + 3 -- the B operands of the group's four 16-deep MFMA steps -- and
//    turns each word into eight bf16 weights in 17 VALU (dequant_word_mix) one MFMA step ahead.
//    Every weight is dequantized exactly once, in registers.
//  * MFMA step i uses k = 32 h + 8 i .. + 7 for both operands (the order of the code words), so the
//    A operand of row r is the 16-byte LDS piece 4 h + i of that row.
// Per group a wave issues 64 MFMAs (2048 cycles of the matrix core) against about 160 VALU, 32 LDS
// operand reads and 41 KB of L2 and HBM traffic per workgroup: the kernel is MFMA-bound. Within one
// wave every VALU instruction placed between MFMAs delays the matrix core by about three cycles
// (measured), so the VALU count per group matters.
//
// Work split. Tiles are numbered row block first (tile t: row block t mod MB, column block t / MB),
// so that with eight row blocks every XCD (workgroup id mod 8) works on one row block and keeps
// its activations in its L2. As in mma.hip, whole tiles go round-robin over the grid and the
// remaining tiles' (tile, group) pairs are split evenly over all workgroups (stream-K); a tile
// covered in part is summed by q4_prefill_finish from fp32 partials in the caller's workspace.
//
// Numerics as mma.hip: fp32 dequantized weight rounded to bf16, exact products, fp32 sums.
#include "common.hpp"
#include "launch.hpp"
#include "mix.hpp"

#include <cstdlib>

namespace splosh {

struct PrefillArgs {
    const uint32_t *packed;
    const uint16_t *scales;
    const uint16_t *biases;
    int64_t n;          // weight rows = output columns
    int64_t groups;
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
    uint32_t code_bytes, sidecar_bytes, a_bytes;
};

constexpr int kPB = 256;                       // tile rows and columns
constexpr int kPRow = 144;                     // LDS bytes per activation row (128 + 16)
constexpr int kPABuf = kPB * kPRow;            // one activation buffer
constexpr int kPEpiRow = 68;                   // floats per row of a wave's epilogue staging
constexpr int kPEpi = 32 * kPEpiRow * 4;       // bytes of a wave's epilogue staging (32 rows)
constexpr int kPCodeRow = 48;                  // LDS bytes per column of a code chunk (32 + 16)
constexpr int kPCodeBytes = kPB * kPCodeRow;   // the codes of a chunk
constexpr int kPBuf = kPABuf + kPCodeBytes + 2 * kPB * 2;  // activations, codes, scales and biases
constexpr size_t kPLds = 3 * kPBuf;            // the epilogue staging reuses the buffers
static_assert(8 * kPEpi <= (int)kPLds, "eight waves' epilogue staging fits the activation buffers");
constexpr int kPFinishMax = 1024;              // contributors q4_prefill_finish can list

// WM waves per SIMD: 4 WM waves, wave (wm, wn) = (wave / 4, wave % 4) owns rows
// 256 / WM * wm .. of columns 64 wn ..; the WM waves sharing a SIMD (equal wn) dequantize the same
// weights, each for its own rows. Only WM = 1 is launched: with two waves per SIMD (128
// accumulators each) the doubled dequantization costs more than the second wave hides.
template <int WM>
__global__ void __launch_bounds__(256 * WM) __attribute__((amdgpu_waves_per_eu(WM, WM)))
q4_prefill_kernel(PrefillArgs args) {
    constexpr int kPThreads = 256 * WM;
    constexpr int FM = 8 / WM;     // 32-row blocks per wave
    constexpr int kAPer = 8 / WM;  // activation pieces per thread and chunk
    constexpr int kCPer = 2 / WM;  // code pieces per thread and chunk
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / 4, wn = wave % 4;
    const int r = lane & 31, h = lane >> 5;
    const int G = (int)args.groups;
    const uint32_t G32 = (uint32_t)G;
    const rsrc_t a_rsrc = make_rsrc(args.a, args.a_bytes);
    const rsrc_t q_rsrc = make_rsrc(args.packed, args.code_bytes);
    const rsrc_t s_rsrc = make_rsrc(args.scales, args.sidecar_bytes);
    const rsrc_t b_rsrc = make_rsrc(args.biases, args.sidecar_bytes);
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    {
        // An AGPR operand makes the compiler select the AGPR form of the MFMAs even where a wave's
        // register budget is 256 (two waves per SIMD): the accumulators then live in AGPRs.
        float agpr_use;
        asm volatile("v_accvgpr_write_b32 %0, 0" : "=a"(agpr_use));
        (void)agpr_use;
    }
    char *epi = lds + wave * kPEpi;  // after the main loop, over the activation buffers

    // Tile `tile`, groups [ga, gb); slot < 0 writes the output, else a partial.
    auto run_job = [&](int tile, int ga, int gb, int slot) {
        const int mb = tile % args.mblocks, nb = tile / args.mblocks;
        const int64_t m0 = (int64_t)mb * kPB, n0 = (int64_t)nb * kPB;
        const int T = gb - ga;
        // Chunk staging (group g of the tile, global -> registers -> LDS buffer):
        //  * activation piece p of this thread: c = p * threads + tid, row c / 8, 16-byte piece
        //    c % 8 of the row's 128 bytes (rows past the last clamped);
        //  * code piece p: c = p * threads + tid, half c % 2 of column c / 2's 32-byte record
        //    (columns past the last clamped);
        //  * sidecars: lanes 0..31 of wave 0 (scales) and wave 1 (biases), 8 columns a lane.
        uint32_t a_src[kAPer], c_src[kCPer];
#pragma unroll
        for (int p = 0; p < kAPer; ++p) {
            const int c = p * kPThreads + tid;
            const int64_t m = m0 + (c >> 3);
            a_src[p] = (uint32_t)(((m < args.rows ? m : args.rows - 1) * args.lda + (c & 7) * 8) * 2);
        }
#pragma unroll
        for (int p = 0; p < kCPer; ++p) {
            const int c = p * kPThreads + tid;
            const int64_t nc = n0 + (c >> 1);
            const uint32_t col = (uint32_t)(nc < args.n ? nc : args.n - 1);
            c_src[p] = ((col >> 7) * G32 * 128u + (col & 127u)) * 32u + 16u * (c & 1);
        }
        const bool side_loader = wave < 2 && lane < 32;
        uint32_t side_src;
        {
            const int64_t nc = n0 + 8 * (lane & 31);
            const uint32_t col = (uint32_t)(nc < args.n ? nc : args.n - 8);
            side_src = ((col >> 7) * G32 * 128u + (col & 127u)) * 2u;
        }
        const rsrc_t side_rsrc = wave == 1 ? b_rsrc : s_rsrc;
        auto a_lds = [&](int p) { return (uint32_t)(((p * kPThreads + tid) >> 3) * kPRow + (tid & 7) * 16); };
        auto c_lds = [&](int p) {
            const int c = p * kPThreads + tid;
            return (uint32_t)(kPABuf + (c >> 1) * kPCodeRow + 16 * (c & 1));
        };
        auto clampg = [&](int t) {
            const int g = ga + t < gb ? ga + t : gb - 1;
            return (uint32_t)__builtin_amdgcn_readfirstlane(g);
        };

        u32x4 ar[kAPer], cr[kCPer], sr = {0u, 0u, 0u, 0u};
        // Half 0: the first activation pieces and the codes; half 1: the others and the sidecars.
        constexpr int kHalf = kAPer / 2;
        auto load_half = [&](int t, int half) {
            const uint32_t g = clampg(t);
#pragma unroll
            for (int p = kHalf * half; p < kHalf * (half + 1); ++p) ar[p] = buffer_load16(a_rsrc, a_src[p] + g * 128u, 0);
            if (half == 0) {
#pragma unroll
                for (int p = 0; p < kCPer; ++p) cr[p] = buffer_load16_cp<2>(q_rsrc, c_src[p] + g * (128u * 32u), 0);
            } else if (side_loader) {
                sr = buffer_load16(side_rsrc, side_src + g * 256u, 0);
            }
        };
        auto store_half = [&](int buf, int half) {
            char *b = lds + buf * kPBuf;
#pragma unroll
            for (int p = kHalf * half; p < kHalf * (half + 1); ++p) *(u32x4 *)(b + a_lds(p)) = ar[p];
            if (half == 0) {
#pragma unroll
                for (int p = 0; p < kCPer; ++p) *(u32x4 *)(b + c_lds(p)) = cr[p];
            } else if (side_loader) {
                *(u32x4 *)(b + kPABuf + kPCodeBytes + wave * 512 + lane * 16) = sr;
            }
        };
        // A wave's codes of a chunk (16 bytes of column 64 wn + 32 j + r: words 4 h .. 4 h + 3) and
        // their coefficients (zero for the padding steps).
        auto read_codes = [&](u32x4 *dst, int buf) {
            const char *b = lds + buf * kPBuf + kPABuf + (64 * wn + r) * kPCodeRow + 16 * h;
#pragma unroll
            for (int j = 0; j < 2; ++j) dst[j] = *(const u32x4 *)(b + 32 * j * kPCodeRow);
        };
        MixCoef cf[2];
        auto read_coef = [&](int buf, bool on) {
            const char *b = lds + buf * kPBuf + kPABuf + kPCodeBytes + (64 * wn + r) * 2;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float sc = bf16_bits_to_f32(*(const uint16_t *)(b + 64 * j));
                const float bi = bf16_bits_to_f32(*(const uint16_t *)(b + 512 + 64 * j));
                cf[j] = mix_coef(on ? sc : 0.0f, on ? bi : 0.0f);
            }
        };
        // Operand reads: MFMA step i of row block f takes row 32 (FM wm + f) + r, piece 4 h + i.
        auto read_af = [&](bf16x8 *dst, int buf, int i) {
            const char *p = lds + buf * kPBuf + (FM * wm * 32 + r) * kPRow + (4 * h + i) * 16;
#pragma unroll
            for (int f = 0; f < FM; ++f) dst[f] = as_bf16x8(*(const u32x4 *)(p + f * 32 * kPRow));
        };

        f32x16 acc[FM][2];
#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[f][j][e] = 0.0f;

        // Prologue, loads in the loop's order (so that the wait counts the compiler derives at the
        // loop head leave the younger loads in flight).
        load_half(0, 0);
        load_half(0, 1);
        store_half(0, 0);
        store_half(0, 1);
        __builtin_amdgcn_sched_barrier(0);
        load_half(1, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_half(1, 1);
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();
        u32x4 cq[2];  // codes of the current group
        read_codes(cq, 0);
        read_coef(0, T > 0);
        bf16x8 bw[2];  // B operands of the current MFMA step
#pragma unroll
        for (int j = 0; j < 2; ++j) bw[j] = dequant_word_mix(cq[j][0], cf[j], magic);
        bf16x8 af[FM];
        if (WM == 1) read_af(af, 0, 0);

        // Step t (group ga + t), d = t mod 3 = its LDS buffer. Every MFMA step interleaves its
        // MFMAs with the dequantization of the next MFMA step's operands (with one wave per SIMD
        // the VALU work only hides under the matrix core when its instructions sit between the
        // MFMAs), its fragment reads and a share of the chunk traffic, spread so that no step
        // queues at the texture unit:
        //  * steps 0 and 1 store chunk t + 1 (loaded in step t - 1) into buffer t + 1 mod 3, half
        //    each, and steps 1 and 2 load chunk t + 2 into the registers just stored;
        //  * the barrier before step 2 makes chunk t + 1 readable: step 2 reads its codes and
        //    coefficients, step 3 dequantizes its first operands (and, with one wave per SIMD,
        //    prefetches its first fragments). Every wave has then finished step t - 1, so buffer
        //    t + 2 mod 3 (last read in step t - 1) may be written in step t + 1.
        // Loads past the job re-read its last group.
        auto step = [&](int t, int d) {
            const int next = d == 2 ? 0 : d + 1;
            u32x4 cn[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i == 2) {
                    lds_barrier();
                    __builtin_amdgcn_sched_barrier(0);
                }
                // One wave per SIMD prefetches the next MFMA step's fragments; with two, the other
                // wave covers the read latency and the registers are short.
                constexpr bool kPrefetch = WM == 1;
                bf16x8 an[FM];
                if (kPrefetch)
                    read_af(an, i < 3 ? d : next, i < 3 ? i + 1 : 0);
                else
                    read_af(af, d, i);
                if (i == 2) read_codes(cn, next);
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int f = 0; f < FM; ++f)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[f], bw[j], acc[f][j], 0, 0, 0);
                // The next MFMA step's operands: word i + 1 of this group, or word 0 of the next.
                if (i < 3) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) bw[j] = dequant_word_mix(cq[j][i + 1], cf[j], magic);
                } else {
                    read_coef(next, t + 1 < T);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        cq[j] = cn[j];
                        bw[j] = dequant_word_mix(cq[j][0], cf[j], magic);
                    }
                }
                if (i < 2) store_half(next, i);
                if (i == 1 || i == 2) load_half(t + 2, i - 1);
                constexpr int kMfma = 2 * FM, kValu = (36 + kMfma - 1) / kMfma;
#pragma unroll
                for (int m = 0; m < kMfma; ++m) {
                    if (m < FM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // one LDS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);             // VALU
                    if (m < 8 / WM && (WM == 2 || m % 2 == 1)) {
                        if (i < 2) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
                        if (i == 1 || i == 2) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (kPrefetch) {
#pragma unroll
                    for (int f = 0; f < FM; ++f) af[f] = an[f];
                }
            }
        };
        // The step count is padded to a multiple of three (no early exit, whose extra paths cost
        // the accumulators register copies); steps past T multiply zero weights.
        const int Tp = (T + 2) / 3 * 3;
        for (int t0 = 0; t0 < Tp; t0 += 3) {
            step(t0, 0);
            step(t0 + 1, 1);
            step(t0 + 2, 2);
        }

        // Epilogue, one 32-row block at a time through the wave's own LDS area (over the
        // activation buffers, once every wave is done with them): lane (r, h) holds row
        // 8 (e / 4) + 4 h + e % 4, column 32 j + r; the rows are then written 16 bytes (4 columns)
        // a lane.
        lds_barrier();
        const int64_t nw0 = n0 + 64 * wn;
#pragma unroll
        for (int f = 0; f < FM; ++f) {
            const int tr0 = 32 * (FM * wm + f);  // the block's first row in the tile
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
                const int64_t m = m0 + tr0 + row, n = nw0 + c4;
                if (m >= args.rows || n >= args.n) continue;
                if (slot >= 0) {
                    float *dst = args.partial + ((int64_t)(blockIdx.x * 2 + slot) * kPB + tr0 + row) * kPB +
                                 64 * wn + c4;
                    *(f32x4 *)dst = v;
                    continue;
                }
                const int64_t index = m * args.ldc + n;
                if (args.out_dtype == SPLOSH_F32) {
                    f32x4 o = v;
                    if (args.residual) o += *(const f32x4 *)((const float *)args.residual + index);
                    *(f32x4 *)((float *)args.out + index) = o;
                } else {
                    float o[4] = {v[0], v[1], v[2], v[3]};
                    if (args.residual) {
                        const u32x2 rb = *(const u32x2 *)((const uint16_t *)args.residual + index);
                        o[0] += bf16_bits_to_f32(rb[0] & 0xffffu);
                        o[1] += bf16_bits_to_f32(rb[0] >> 16);
                        o[2] += bf16_bits_to_f32(rb[1] & 0xffffu);
                        o[3] += bf16_bits_to_f32(rb[1] >> 16);
                    }
                    const u32x2 pk = {f32x2_to_bf16x2(o[0], o[1]), f32x2_to_bf16x2(o[2], o[3])};
                    *(u32x2 *)((uint16_t *)args.out + index) = pk;
                }
            }
        }
    };

    // The jobs: whole tiles blockIdx.x, blockIdx.x + P, ... below dp_tiles, then this workgroup's
    // range of the remaining (tile, group) pairs, cut at tile boundaries. One call site, so that
    // run_job is inlined.
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
q4_prefill_finish(const float *__restrict__ partial, int dp_tiles, int64_t sk_units, int P, int64_t groups,
                  int mblocks, int64_t rows, int64_t n, void *out, int64_t ldc, int out_dtype, const void *residual) {
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
    const int64_t m0 = (int64_t)(tile % mblocks) * kPB, n0 = (int64_t)(tile / mblocks) * kPB;
    const int e0 = (blockIdx.y * 256 + threadIdx.x) * 4;  // element of the tile
    const int tr = e0 / kPB, tc = e0 % kPB;
    const int64_t m = m0 + tr, col = n0 + tc;
    if (m >= rows || col >= n) return;
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 < contributors; j0 += 8) {
        f32x4 x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int jj = j0 + j < contributors ? j0 + j : contributors - 1;
            x[j] = *(const f32x4 *)(partial + ((int64_t)(wg[jj] * 2 + slot_of[jj]) * kPB + tr) * kPB + tc);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j0 + j < contributors) v += x[j];
    }
    const int64_t index = m * ldc + col;
    if (out_dtype == SPLOSH_F32) {
        if (residual) v += *(const f32x4 *)((const float *)residual + index);
        *(f32x4 *)((float *)out + index) = v;
    } else {
        float o[4] = {v[0], v[1], v[2], v[3]};
        if (residual) {
            const u32x2 rb = *(const u32x2 *)((const uint16_t *)residual + index);
            o[0] += bf16_bits_to_f32(rb[0] & 0xffffu);
            o[1] += bf16_bits_to_f32(rb[0] >> 16);
            o[2] += bf16_bits_to_f32(rb[1] & 0xffffu);
            o[3] += bf16_bits_to_f32(rb[1] >> 16);
        }
        const u32x2 pk = {f32x2_to_bf16x2(o[0], o[1]), f32x2_to_bf16x2(o[2], o[3])};
        *(u32x2 *)((uint16_t *)out + index) = pk;
    }
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

static size_t prefill_sk_bytes(int grid) { return (size_t)grid * 2 * kPB * kPB * sizeof(float); }

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

template <int WM>
static void launch_prefill_wm(const PrefillPlan &plan, const PrefillArgs &args, hipStream_t stream) {
    static bool once = [] {
        (void)hipFuncSetAttribute((const void *)q4_prefill_kernel<WM>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)kPLds);
        return true;
    }();
    (void)once;
    hipLaunchKernelGGL(q4_prefill_kernel<WM>, dim3((unsigned)plan.grid), dim3(256 * WM), kPLds, stream, args);
}

hipError_t launch_q4_prefill(const PrefillPlan &plan, const splosh_q4_weight &w, const uint16_t *a, int64_t lda,
                             void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                             void *workspace, hipStream_t stream) {
    PrefillArgs args = {};
    args.packed = w.packed;
    args.scales = w.scales;
    args.biases = w.biases;
    args.n = w.rows;
    args.groups = w.inner / kGroup;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = rows;
    args.out_dtype = out_dtype;
    args.mblocks = plan.mblocks;
    args.partial = plan.sk_units > 0 ? (float *)workspace : nullptr;
    args.dp_tiles = plan.dp_tiles;
    args.sk_units = plan.sk_units;
    args.code_bytes = (uint32_t)(w.rows * args.groups * 32);
    args.sidecar_bytes = (uint32_t)(w.rows * args.groups * 2);
    args.a_bytes = (uint32_t)(((rows - 1) * lda + w.inner) * 2);
    launch_prefill_wm<1>(plan, args, stream);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || plan.sk_units == 0) return err;
    const int remainder = plan.tiles - plan.dp_tiles;
    hipLaunchKernelGGL(q4_prefill_finish, dim3((unsigned)remainder, kPB * kPB / 1024), dim3(256), 0, stream,
                       (const float *)workspace, plan.dp_tiles, plan.sk_units, plan.grid, args.groups, plan.mblocks,
                       rows, w.rows, out, ldc, out_dtype, residual);
    return hipGetLastError();
}

}  // namespace splosh
