// prefill.hip -- q4 GEMM for prefill (hundreds to thousands of activation rows) on
// v_mfma_f32_32x32x16_bf16, one wave per SIMD.
//
// A workgroup of four waves computes a 256 x 256 output tile; wave w owns all 256 rows of columns
// 64 w .. 64 w + 63 (8 x 2 MFMA tiles of 32 x 32: 256 fp32 accumulators a lane, held in AGPRs,
// which is why the kernel runs one wave per SIMD). Per 64-group of K:
//  * The activation tile A[256][64] (32 KB) is staged global -> registers -> LDS by all threads,
//    one group ahead, into one of three buffers (row stride 144 bytes: the operand reads do not
//    conflict), with one barrier per group, in its middle.
//  * The weights never pass through LDS: lane (r, h) of wave w loads 16 bytes of the 32-byte tiled
//    record of column n0 + 64 w + 32 j + r (j = 0, 1) -- words 4 h .. 4 h + 3, the B operands of
//    the group's four 16-deep MFMA steps -- three groups ahead, with its scale and bias, and turns
//    each word into eight bf16 weights in 17 VALU (dequant_word_mix) while the previous group's
//    MFMAs run. Every weight is dequantized exactly once.
//  * MFMA step i uses k = 32 h + 8 i .. + 7 for both operands (the order of the code words), so the
//    A operand of row r is the 16-byte LDS piece 4 h + i of that row.
// Per group a wave issues 64 MFMAs (2048 cycles of the matrix core) against 136 VALU, 32 LDS
// operand reads and 16 KB of L2 and HBM traffic per workgroup: the kernel is MFMA-bound.
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
constexpr int kPThreads = 256;                 // four waves
constexpr int kPRow = 144;                     // LDS bytes per activation row (128 + 16)
constexpr int kPABuf = kPB * kPRow;            // one activation buffer
constexpr int kPEpiRow = 68;                   // floats per row of a wave's epilogue staging
constexpr int kPEpi = 32 * kPEpiRow * 4;       // bytes of a wave's epilogue staging (32 rows)
constexpr size_t kPLds = 3 * kPABuf + 4 * kPEpi;
constexpr int kPFinishMax = 1024;              // contributors q4_prefill_finish can list

__global__ void __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
q4_prefill_kernel(PrefillArgs args) {
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, h = lane >> 5;
    const int G = (int)args.groups;
    const uint32_t G32 = (uint32_t)G;
    const rsrc_t a_rsrc = make_rsrc(args.a, args.a_bytes);
    const rsrc_t q_rsrc = make_rsrc(args.packed, args.code_bytes);
    const rsrc_t s_rsrc = make_rsrc(args.scales, args.sidecar_bytes);
    const rsrc_t b_rsrc = make_rsrc(args.biases, args.sidecar_bytes);
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    char *epi = lds + 3 * kPABuf + wave * kPEpi;

    // Tile `tile`, groups [ga, gb); slot < 0 writes the output, else a partial.
    auto run_job = [&](int tile, int ga, int gb, int slot) {
        const int mb = tile % args.mblocks, nb = tile / args.mblocks;
        const int64_t m0 = (int64_t)mb * kPB, n0 = (int64_t)nb * kPB;
        const int T = gb - ga;
        // Activation staging: piece p of this thread is chunk c = p * 256 + tid of the tile, row
        // c / 8, 16-byte chunk c % 8 of the group's 128 bytes; rows past the last are clamped.
        uint32_t a_src[8];
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int c = p * kPThreads + tid;
            const int64_t m = m0 + (c >> 3);
            a_src[p] = (uint32_t)(((m < args.rows ? m : args.rows - 1) * args.lda + (c & 7) * 8) * 2);
        }
        auto a_lds = [&](int p) { return (uint32_t)(((p * kPThreads + tid) >> 3) * kPRow + (tid & 7) * 16); };
        uint32_t q_lane[2], s_lane[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t nc = n0 + 64 * wave + 32 * j + r;
            const uint32_t col = (uint32_t)(nc < args.n ? nc : args.n - 1);
            const uint32_t rec0 = (col >> 7) * G32 * 128u + (col & 127u);
            q_lane[j] = rec0 * 32u + 16u * h;
            s_lane[j] = rec0 * 2u;
        }
        auto clampg = [&](int t) {
            const int g = ga + t < gb ? ga + t : gb - 1;
            return (uint32_t)__builtin_amdgcn_readfirstlane(g);
        };

        u32x4 ar[8];
        auto load_a = [&](int t) {
            const uint32_t off = clampg(t) * 128u;
#pragma unroll
            for (int p = 0; p < 8; ++p) ar[p] = buffer_load16(a_rsrc, a_src[p] + off, 0);
        };
        auto store_a = [&](int buf) {
#pragma unroll
            for (int p = 0; p < 8; ++p) *(u32x4 *)(lds + buf * kPABuf + a_lds(p)) = ar[p];
        };
        u32x4 wq[3][2];
        uint32_t ws[3][2], wb[3][2];
        auto load_w = [&](int slot, int t) {
            const uint32_t g = clampg(t);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                wq[slot][j] = buffer_load16_cp<2>(q_rsrc, q_lane[j], g * (128u * 32u));
                ws[slot][j] = buffer_load_u16(s_rsrc, s_lane[j], g * 256u);
                wb[slot][j] = buffer_load_u16(b_rsrc, s_lane[j], g * 256u);
            }
        };
        MixCoef cf[2];
        auto prepare = [&](int slot, bool on) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
                cf[j] = mix_coef(on ? bf16_bits_to_f32(ws[slot][j]) : 0.0f, on ? bf16_bits_to_f32(wb[slot][j]) : 0.0f);
        };
        bf16x8 bw[2][4];
        // Operand reads: MFMA step i of row block f takes row 32 f + r, piece 4 h + i.
        auto read_af = [&](bf16x8 *dst, int buf, int i) {
            const char *p = lds + buf * kPABuf + r * kPRow + (4 * h + i) * 16;
#pragma unroll
            for (int f = 0; f < 8; ++f) dst[f] = as_bf16x8(*(const u32x4 *)(p + f * 32 * kPRow));
        };

        f32x16 acc[8][2];
#pragma unroll
        for (int f = 0; f < 8; ++f)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[f][j][e] = 0.0f;

        // Prologue, in the loop's load order (chunk, then codes), so that the wait counts the
        // compiler derives at the loop head leave the codes in flight.
        load_a(0);
        load_w(0, 0);
        load_w(1, 1);
        store_a(0);
        __builtin_amdgcn_sched_barrier(0);
        load_a(1);
        __builtin_amdgcn_sched_barrier(0);
        load_w(2, 2);
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();
        prepare(0, T > 0);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) bw[j][i] = dequant_word_mix(wq[0][j][i], cf[j], magic);
        bf16x8 af[8];
        read_af(af, 0, 0);

        // Step t (group ga + t), d = t mod 3 = its activation buffer and code ring slot. Every
        // MFMA step interleaves its 16 MFMAs with the dequantization of the next group's operand
        // i (with one wave per SIMD the VALU work only hides under the matrix core when its
        // instructions sit between the MFMAs), the next MFMA step's fragment reads and a share of
        // the memory traffic, spread so that no step queues at the texture unit:
        //  * steps 0 and 1 store chunk t + 1 (loaded in step t - 1) into buffer t + 1 mod 3, half
        //    each, and steps 1 and 2 load chunk t + 2 into the registers just stored;
        //  * the barrier before step 2 makes chunk t + 1 readable (step 3 prefetches its first
        //    fragments); since every wave has then finished step t - 1, buffer t + 2 mod 3 (read
        //    last in step t - 1) may be written in step t + 1;
        //  * steps 2 and 3 load the codes of step t + 3 into the ring slot of step t, whose
        //    weights were dequantized in step t - 1.
        // Loads past the job re-read its last group.
        auto step = [&](int t, int d) {
            const int next = d == 2 ? 0 : d + 1;
            prepare(next, t + 1 < T);  // zero coefficients for the padding steps
            const uint32_t ga_next = clampg(t + 2) * 128u, gw = clampg(t + 3);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i == 2) {
                    lds_barrier();
                    __builtin_amdgcn_sched_barrier(0);
                }
                bf16x8 an[8];
                read_af(an, i < 3 ? d : next, i < 3 ? i + 1 : 0);
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int f = 0; f < 8; ++f)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[f], bw[j][i], acc[f][j], 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 2; ++j) bw[j][i] = dequant_word_mix(wq[next][j][i], cf[j], magic);
                // Chunk t + 1: pieces 4 i .. 4 i + 3 stored in steps 0 and 1 and reloaded (for
                // chunk t + 2) in steps 1 and 2, half the LDS writes in each of the first steps.
                if (i < 2) {
#pragma unroll
                    for (int p = 4 * i; p < 4 * i + 4; ++p) *(u32x4 *)(lds + next * kPABuf + a_lds(p)) = ar[p];
                }
                if (i == 1 || i == 2) {
#pragma unroll
                    for (int p = 4 * (i - 1); p < 4 * i; ++p) ar[p] = buffer_load16(a_rsrc, a_src[p] + ga_next, 0);
                }
                if (i >= 2) {
                    const int j = i - 2;
                    wq[d][j] = buffer_load16_cp<2>(q_rsrc, q_lane[j], gw * (128u * 32u));
                    ws[d][j] = buffer_load_u16(s_rsrc, s_lane[j], gw * 256u);
                    wb[d][j] = buffer_load_u16(b_rsrc, s_lane[j], gw * 256u);
                }
#pragma unroll
                for (int m = 0; m < 16; ++m) {
                    if (m < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);             // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);             // two VALU
                    if (m % 2 == 1) {
                        if (i < 2 && m < 8) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
                        if (i > 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);         // VMEM read
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int f = 0; f < 8; ++f) af[f] = an[f];
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

        // Epilogue, one 32-row block at a time through the wave's own LDS area: lane (r, h) holds
        // row 8 (e / 4) + 4 h + e % 4, column 32 j + r; the rows are then written 16 bytes (4
        // columns) a lane.
        const int64_t nw0 = n0 + 64 * wave;
#pragma unroll
        for (int f = 0; f < 8; ++f) {
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
                const int64_t m = m0 + 32 * f + row, n = nw0 + c4;
                if (m >= args.rows || n >= args.n) continue;
                if (slot >= 0) {
                    float *dst = args.partial + ((int64_t)(blockIdx.x * 2 + slot) * kPB + 32 * f + row) * kPB +
                                 64 * wave + c4;
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
    for (int j0 = 0; j0 < contributors; j0 += 4) {
        f32x4 x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int jj = j0 + j < contributors ? j0 + j : contributors - 1;
            x[j] = *(const f32x4 *)(partial + ((int64_t)(wg[jj] * 2 + slot_of[jj]) * kPB + tr) * kPB + tc);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
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
    if (const char *env = getenv("SPLOSH_PREFILL_GRID")) cus = atoi(env) > 0 ? atoi(env) : cus;
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
    static bool once = [] {
        (void)hipFuncSetAttribute((const void *)q4_prefill_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)kPLds);
        return true;
    }();
    (void)once;
    hipLaunchKernelGGL(q4_prefill_kernel, dim3((unsigned)plan.grid), dim3(kPThreads), kPLds, stream, args);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || plan.sk_units == 0) return err;
    const int remainder = plan.tiles - plan.dp_tiles;
    hipLaunchKernelGGL(q4_prefill_finish, dim3((unsigned)remainder, kPB * kPB / 1024), dim3(256), 0, stream,
                       (const float *)workspace, plan.dp_tiles, plan.sk_units, plan.grid, args.groups, plan.mblocks,
                       rows, w.rows, out, ldc, out_dtype, residual);
    return hipGetLastError();
}

}  // namespace splosh
