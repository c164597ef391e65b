// verify.hip -- q4 (MLX affine, TILED128) GEMM for 2 < M <= 64 rows: the draft-verify shapes.
//
// At M = 64 the dequantization (about two VALU instructions a weight) and the bf16 MFMAs (M x 2
// flops a weight) take about the same time, and both about as long as streaming the weights from
// HBM. The kernel is built so that the three overlap and nothing is done twice:
//
//  * A workgroup of eight waves (two a SIMD) owns a group of 16-column tiles and a range of K,
//    cut into 128-element chunks (two q4 groups). Its waves take the chunks in turn (KQ = 8 / NW
//    waves a weight; for a fused gate+up pair four waves take the gate, four the up weight), and
//    each wave keeps the accumulators of all of the group's tiles. Every weight byte is loaded and
//    dequantized once, and every activation element once per workgroup and weight.
//  * One 16-byte load gives a lane the 32 codes of its column for one chunk quarter
//    (v_mfma_f32_16x16x32_bf16 reads, in lane (n, j), eight consecutive K of column n): its four
//    code words are the B operands of the chunk's four K-steps, dequantized in registers
//    (dequant_word_mix) right before use. The K positions a lane covers are the same for the
//    activation operand, which each wave streams from L2 into its own LDS ring three steps ahead
//    (direct-to-LDS loads: nothing in flight holds a register). No barrier in the main loop: the
//    two waves on a SIMD co-issue one's VALU with the other's MFMAs.
//  * The waves' accumulators are summed in LDS once per unit, then written (silu(g) * u for the
//    pair, residual added). Tiles beyond a whole number of groups per workgroup are split along K
//    over the workgroups with fewer groups; their fp32 partials go to the workspace, and the last
//    of a tile's contributors sums them in piece order (deterministic) and writes the output.
#include "common.hpp"
#include "launch.hpp"
#include "mix.hpp"

#include <stdlib.h>

#include <type_traits>

namespace splosh {

constexpr int kVThreads = 512;
constexpr uint32_t kVOut = 0xFFFFFFF0u;      // a per-lane offset past every buffer: reads zero
constexpr int kVCodeCpol = 2;                // codes are read once (non-temporal)
constexpr int kVDevCpol = 1 | 16;            // partials cross XCDs: written and read through to memory

struct VerifyArgs {
    const uint32_t *packed[2];
    const uint16_t *scales[2];
    const uint16_t *biases[2];
    int64_t groups;
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int rows;
    int out_dtype;
    // Units: phase 1 = (group of T tiles, piece of K), phase 2 = (one tile, piece of K).
    int n1, s1, n2, s2;
    int units;
    float *partial;
    int *counters;       // one per phase-1 group, then one per phase-2 tile (zero between calls)
    uint32_t partial_bytes;
    uint32_t base2;      // first float of the phase-2 partial slots
    uint32_t code_bytes, sidecar_bytes, a_bytes;
};

template <int NW, int T, int MT>
__global__ void __launch_bounds__(kVThreads, 1) q4_verify_kernel(VerifyArgs args) {
    extern __shared__ float red[];
    __shared__ int fix_last;
    constexpr int KQ = 8 / NW;
    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, ln = lane & 15, j = lane >> 4;
    const int wsel = NW == 2 ? wv / KQ : 0;
    const int kq = wv % KQ;
    const rsrc_t c_rsrc = make_rsrc(args.packed[wsel], args.code_bytes);
    const rsrc_t s_rsrc = make_rsrc(args.scales[wsel], args.sidecar_bytes);
    const rsrc_t b_rsrc = make_rsrc(args.biases[wsel], args.sidecar_bytes);
    const rsrc_t a_rsrc = make_rsrc(args.a, args.a_bytes);
    const int rows = args.rows;
    const int chunks = (int)(args.groups / 2);
    const uint32_t magic = 0x64006400u;
    const uint32_t kOff = (uint32_t)((j >> 1) * 4096 + (j & 1) * 16);   // code offset of the lane's half-record
    // Activation rows of this lane, one a 16-row tile: element (m, 8 j) of the chunk, or no row.
    uint32_t abase[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + ln;
        abase[mt] = m < rows ? (uint32_t)(((int64_t)m * args.lda + 8 * j) * 2) : 0x80000000u;
    }

    // One unit: TT tiles from tile0, chunks [c0, c1), written whole (S == 1) or as piece `piece`
    // of S into the partial slot at float `slot` (tile counter `target`).
    auto run = [&](auto tt_tag, int tile0, int c0, int c1, int S, int piece, int target, uint32_t slot,
                   int slot_stride) {
        constexpr int TT = decltype(tt_tag)::value;
        f32x4 acc[TT][MT];
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // Byte offsets of this lane's records at chunk 0: record (n, 2 c + j / 2), half j % 2.
        uint32_t cbase[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const int64_t n = (int64_t)(tile0 + t) * 16 + ln;
            const int64_t rec = ((n >> 7) * args.groups + (j >> 1)) * kTileRows + (n & (kTileRows - 1));
            cbase[t] = (uint32_t)(rec * 32 + (j & 1) * 16);
        }
        const int steps = (c1 - c0 + KQ - 1) / KQ;   // the same for every wave (empty chunks read zero)
        // Code ring: CD chunks, filled CD - 1 chunks ahead (two at 64 rows, where registers are short).
        constexpr int CD = MT >= 4 ? 2 : 3;
        u32x4 cw[CD][TT];
        uint32_t sc[2][TT], bi[2][TT];   // one chunk's sidecars (its two groups)
        // This wave's activation ring in LDS: four K-steps of MT 1 KB fragments (lane l's 16 bytes at
        // 16 l), filled by direct-to-LDS loads three steps ahead.
        float *ring = red + (size_t)wv * 4 * MT * 256;
        auto load_codes = [&](int i, u32x4 (&w)[TT]) {
            const int c = c0 + kq + i * KQ;
            const uint32_t oob = c < c1 ? 0u : kVOut;   // OR-ed in: no branch around the loads
#pragma unroll
            for (int t = 0; t < TT; ++t)
                w[t] = buffer_load16_cp<kVCodeCpol>(c_rsrc, (cbase[t] + (uint32_t)c * 8192u) | oob, 0);
        };
        auto load_side = [&](int i) {
            const int c = c0 + kq + i * KQ;
            const uint32_t keep = c < c1 ? ~0u : 0u;   // exact out-of-range offset, no branch
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                // Group 2 c + h of the lane's column: the sidecar of record r is at 2 r, the code
                // offset is 32 r + 16 (j % 2) for r = record (n, 2 c + j / 2).
                const uint32_t o0 = (cbase[t] + (uint32_t)c * 8192u - kOff) >> 4;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t o = ((o0 + 256u * h) & keep) | (kVOut & ~keep);
                    sc[h][t] = buffer_load_u16(s_rsrc, o, 0);
                    bi[h][t] = buffer_load_u16(b_rsrc, o, 0);
                }
            }
        };
        auto load_a = [&](int i, int s) {
            const int c = c0 + kq + i * KQ;
            const uint32_t oob = c < c1 ? 0u : kVOut;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                buffer_load_lds16(a_rsrc, ring + (s * MT + mt) * 256, (abase[mt] + (uint32_t)c * 256u + (uint32_t)s * 64u) | oob);
        };
        // One chunk from code ring slot B. Issue order, the same every chunk (the prologue plays
        // the previous chunk's part): step 0: codes of chunk i + CD - 1, activations of step 3; steps
        // 1, 2, 3: activations of steps 0, 1, 2 of chunk i + 1, at step 2 followed by its sidecars
        // (this chunk's second group has just been turned into coefficients). The activations of step s were issued three steps back, so
        // 5 TT + 3 MT loads (4 TT + 3 MT at step 3) may still be in flight when they are read.
        //
        // K order: in step s lane (n, j) covers K 32 s + 8 j .. + 8 of the chunk, so that the four
        // lanes of an activation row read 64 contiguous bytes. Its codes are word 4 s + j of the
        // chunk, while its load brought words 4 j .. 4 j + 3: a 4 x 4 transpose over the lanes
        // n + 16 j (two permlane32 and two permlane16 swaps) puts them in place.
        auto body = [&](auto b_tag, int i) {
            constexpr int B = decltype(b_tag)::value;
            load_codes(i + CD - 1, cw[(B + CD - 1) % CD]);
            __builtin_amdgcn_sched_barrier(0);
            MixCoef coef[TT];
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                u32x4 &w = cw[B][t];
                const auto p = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
                const auto q = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
                const auto r = __builtin_amdgcn_permlane16_swap(p[0], q[0], false, false);
                const auto u = __builtin_amdgcn_permlane16_swap(p[1], q[1], false, false);
                w = u32x4{r[0], r[1], u[0], u[1]};
                coef[t] = mix_coef(bf16_bits_to_f32(sc[0][t]), bf16_bits_to_f32(bi[0][t]));
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (s == 2) {
#pragma unroll
                    for (int t = 0; t < TT; ++t)
                        coef[t] = mix_coef(bf16_bits_to_f32(sc[1][t]), bf16_bits_to_f32(bi[1][t]));
                }
                load_a(s == 0 ? i : i + 1, (s + 3) & 3);
                __builtin_amdgcn_sched_barrier(0);   // the activations go first: the waits count on it
                if (s == 2) {
                    load_side(i + 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (s == 3) wait_vmcnt<4 * TT + 3 * MT>();
                else wait_vmcnt<5 * TT + 3 * MT>();
                u32x4 af[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) af[mt] = *(const u32x4 *)(ring + (s * MT + mt) * 256 + lane * 4);
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const bf16x8 wb = dequant_word_mix(cw[B][t][s], coef[t], magic);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af[mt]), wb, acc[t][mt], 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        __syncthreads();   // the previous unit's reduction has been read: the rings may be refilled
#pragma unroll
        for (int d = 0; d + 1 < CD; ++d) load_codes(d, cw[d]);
        load_a(0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_a(0, 1);
        __builtin_amdgcn_sched_barrier(0);
        load_side(0);
        __builtin_amdgcn_sched_barrier(0);
        load_a(0, 2);
        __builtin_amdgcn_sched_barrier(0);
        int i = 0;
        if constexpr (CD == 3) {
            for (; i + 3 <= steps; i += 3) {
                body(std::integral_constant<int, 0>{}, i);
                body(std::integral_constant<int, 1>{}, i + 1);
                body(std::integral_constant<int, 2>{}, i + 2);
            }
            if (i < steps) body(std::integral_constant<int, 0>{}, i);
            if (i + 1 < steps) body(std::integral_constant<int, 1>{}, i + 1);
        } else {
            for (; i + 2 <= steps; i += 2) {
                body(std::integral_constant<int, 0>{}, i);
                body(std::integral_constant<int, 1>{}, i + 1);
            }
            if (i < steps) body(std::integral_constant<int, 0>{}, i);
        }
        wait_vmcnt<0>();   // prefetches past the end still write the rings

        // Sum the K waves in LDS: kq >= 4 fold into kq - 4 first when a weight has eight.
        constexpr int R = TT * MT * 4;
        __syncthreads();   // every wave is done with its ring
        if constexpr (KQ == 8) {
            if (kq >= 4) {
                float *r = red + (kq - 4) * R * 64;
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) r[((t * MT + mt) * 4 + e) * 64 + lane] = acc[t][mt][e];
            }
            __syncthreads();
            if (kq < 4) {
                const float *r = red + kq * R * 64;
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[t][mt][e] += r[((t * MT + mt) * 4 + e) * 64 + lane];
            }
            __syncthreads();
        }
        if (kq < 4) {
            float *r = red + (wsel * 4 + kq) * R * 64;
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[((t * MT + mt) * 4 + e) * 64 + lane] = acc[t][mt][e];
        }
        __syncthreads();
        constexpr int kCols = TT * 16;
        const int elems = rows * kCols;
        // Element (m, col) of weight w summed over the four K waves, in wave order.
        auto total = [&](int w, int m, int col) {
            const int reg = ((col >> 4) * MT + (m >> 4)) * 4 + (m & 3);
            const int ln2 = ((m & 15) >> 2) * 16 + (col & 15);
            const float *r = red + (w * 4) * R * 64 + reg * 64 + ln2;
            return ((r[0] + r[R * 64]) + r[2 * R * 64]) + r[3 * R * 64];
        };
        auto store_out = [&](int m, int col, const float *v) {
            float value = v[0];
            if constexpr (NW == 2) value = silu(v[0]) * v[1];
            const int64_t index = (int64_t)m * args.ldc + (int64_t)tile0 * 16 + col;
            if (args.out_dtype == SPLOSH_F32) {
                if (args.residual) value += ((const float *)args.residual)[index];
                ((float *)args.out)[index] = value;
            } else {
                if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                ((uint16_t *)args.out)[index] = f32_to_bf16(value);
            }
        };
        if (S == 1) {
            for (int e = tid; e < elems; e += kVThreads) {
                const int m = e / kCols, col = e % kCols;
                float v[NW];
#pragma unroll
                for (int w = 0; w < NW; ++w) v[w] = total(w, m, col);
                store_out(m, col, v);
            }
            return;
        }
        // A piece: the partial goes to its slot; the last contributor of the tile sums them.
        const rsrc_t p_rsrc = make_rsrc(args.partial, args.partial_bytes);
        for (int e = tid; e < elems; e += kVThreads) {
            const int m = e / kCols, col = e % kCols;
#pragma unroll
            for (int w = 0; w < NW; ++w)
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, total(w, m, col)), p_rsrc,
                                                      (slot + (uint32_t)((w * rows + m) * kCols + col)) * 4u, 0, kVDevCpol);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            int *counter = args.counters + target;
            const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            const bool last = old == S - 1;
            if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            fix_last = last ? 1 : 0;
        }
        __syncthreads();
        if (!fix_last) return;
        const uint32_t first = slot - (uint32_t)piece * (uint32_t)slot_stride;
        for (int e = tid; e < elems; e += kVThreads) {
            const int m = e / kCols, col = e % kCols;
            float v[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const uint32_t off = first + (uint32_t)((w * rows + m) * kCols + col);
                float x = 0.0f;
                for (int p = 0; p < S; ++p)
                    x += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                       p_rsrc, (off + (uint32_t)p * (uint32_t)slot_stride) * 4u, 0, kVDevCpol));
                v[w] = x;
            }
            store_out(m, col, v);
        }
    };

    const int u1 = args.n1 * args.s1;
    const int slot1 = NW * rows * T * 16, slot2 = NW * rows * 16;
    for (int u = blockIdx.x; u < args.units; u += gridDim.x) {
        if (u < u1) {
            // Phase 1: group u % n1, piece u / n1; the pieces of a group sit n1 slots apart.
            const int g = u % args.n1, p = u / args.n1;
            const int c0 = (int)((int64_t)chunks * p / args.s1), c1 = (int)((int64_t)chunks * (p + 1) / args.s1);
            run(std::integral_constant<int, T>{}, g * T, c0, c1, args.s1, p, g, (uint32_t)u * (uint32_t)slot1,
                args.n1 * slot1);
        } else {
            const int v = u - u1;
            const int tl = v % args.n2, p = v / args.n2;
            const int c0 = (int)((int64_t)chunks * p / args.s2), c1 = (int)((int64_t)chunks * (p + 1) / args.s2);
            run(std::integral_constant<int, 1>{}, args.n1 * T + tl, c0, c1, args.s2, p, args.n1 + tl,
                args.base2 + (uint32_t)v * (uint32_t)slot2, args.n2 * slot2);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Host side.

static int verify_cus() {
    static int cache[64] = {0};
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

static int verify_tiles(bool) { return 4; }

VerifyPlan plan_verify(int64_t rows, int64_t columns, int64_t groups, bool mlp) {
    VerifyPlan p{};
    const int T = verify_tiles(mlp);
    const int G = verify_cus();
    const int nt = (int)(columns / 16);
    const int chunks = (int)(groups / 2);
    int max_pieces = chunks / 2 > 0 ? chunks / 2 : 1;   // a piece is at least two chunks
    // SPLOSH_VERIFY_SPLIT=n caps the pieces of K a tile is cut into (n = 1: no split).
    if (const char *env = getenv("SPLOSH_VERIFY_SPLIT"))
        if (atoi(env) > 0 && atoi(env) < max_pieces) max_pieces = atoi(env);
    const int q = nt / T;
    if (q >= G) {
        p.n1 = q / G * G;
        p.s1 = 1;
    } else if (q > 0) {
        p.n1 = q;
        p.s1 = G / q < max_pieces ? G / q : max_pieces;
        if (p.s1 < 1) p.s1 = 1;
    }
    p.n2 = nt - p.n1 * T;
    if (p.n2 > 0) {
        // Pieces of about the size of a phase-1 unit's share of a workgroup.
        const int u1 = p.n1 * p.s1;
        const int free = (G - u1 % G) % G;
        int s2 = ((free > 0 ? free : G) + p.n2 - 1) / p.n2;
        p.s2 = s2 < 1 ? 1 : s2 > max_pieces ? max_pieces : s2;
    }
    p.units = p.n1 * p.s1 + p.n2 * p.s2;
    p.grid = p.units < G ? p.units : G;
    const int nw = mlp ? 2 : 1;
    p.partial_floats1 = p.s1 > 1 ? (size_t)p.n1 * p.s1 * nw * rows * T * 16 : 0;
    p.partial_floats2 = p.s2 > 1 ? (size_t)p.n2 * p.s2 * nw * rows * 16 : 0;
    return p;
}

static size_t verify_partial_bytes(const VerifyPlan &p) {
    return ((p.partial_floats1 + p.partial_floats2) * sizeof(float) + 255) / 256 * 256;
}

size_t verify_workspace_bytes(const VerifyPlan &p) {
    const bool split = p.s1 > 1 || p.s2 > 1;
    return split ? verify_partial_bytes(p) + (size_t)(p.n1 + p.n2) * sizeof(int) : 0;
}

bool verify_fits(int64_t rows, int64_t columns, int64_t inner, int order, int64_t lda) {
    if (order != SPLOSH_Q4_TILED128 || rows <= 2 || rows > 64) return false;
    if (columns % 128 != 0 || inner % 128 != 0 || lda % 8 != 0) return false;
    const int64_t groups = inner / 64;
    // 32-bit buffer offsets: codes, sidecars, activations and partials.
    if (columns * groups * 32 >= ((int64_t)1 << 31) || rows * lda * 2 >= ((int64_t)1 << 31)) return false;
    return true;
}

template <int NW, int T, int MT>
static hipError_t launch_verify_v(const VerifyPlan &p, const VerifyArgs &args, hipStream_t stream) {
    auto kernel = q4_verify_kernel<NW, T, MT>;
    const int red_bytes = NW * 4 * T * MT * 4 * 64 * (int)sizeof(float);
    const int ring_bytes = 8 * 4 * MT * 1024;
    const int lds = red_bytes > ring_bytes ? red_bytes : ring_bytes;
    static bool once = [&] {
        (void)hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        return true;
    }();
    (void)once;
    hipLaunchKernelGGL(kernel, dim3((unsigned)p.grid), dim3(kVThreads), lds, stream, args);
    return hipGetLastError();
}

template <int NW, int T>
static hipError_t launch_verify_mt(const VerifyPlan &p, const VerifyArgs &args, int rows, hipStream_t stream) {
    switch ((rows + 15) / 16) {
        case 1: return launch_verify_v<NW, T, 1>(p, args, stream);
        case 2: return launch_verify_v<NW, T, 2>(p, args, stream);
        case 3: return launch_verify_v<NW, T, 3>(p, args, stream);
        default: return launch_verify_v<NW, T, 4>(p, args, stream);
    }
}

hipError_t launch_q4_verify(const VerifyPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                            const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype,
                            const void *residual, int64_t rows, void *workspace, hipStream_t stream) {
    VerifyArgs args = {};
    args.packed[0] = w.packed;
    args.scales[0] = w.scales;
    args.biases[0] = w.biases;
    args.packed[1] = up ? up->packed : w.packed;
    args.scales[1] = up ? up->scales : w.scales;
    args.biases[1] = up ? up->biases : w.biases;
    args.groups = w.inner / kGroup;
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = (int)rows;
    args.out_dtype = out_dtype;
    args.n1 = plan.n1;
    args.s1 = plan.s1;
    args.n2 = plan.n2;
    args.s2 = plan.s2;
    args.units = plan.units;
    const bool split = plan.s1 > 1 || plan.s2 > 1;
    args.partial = split ? (float *)workspace : nullptr;
    args.partial_bytes = split ? (uint32_t)verify_partial_bytes(plan) : 0;
    args.counters = split ? (int *)((char *)workspace + args.partial_bytes) : nullptr;
    args.base2 = (uint32_t)plan.partial_floats1;
    args.code_bytes = (uint32_t)(w.rows * args.groups * 32);
    args.sidecar_bytes = (uint32_t)(w.rows * args.groups * 2);
    args.a_bytes = (uint32_t)(((rows - 1) * lda + w.inner) * 2);
    if (up) return launch_verify_mt<2, 4>(plan, args, (int)rows, stream);
    return launch_verify_mt<1, 4>(plan, args, (int)rows, stream);
}

}  // namespace splosh
