// mma.hip -- quantized GEMM for batched draft-verify (up to 64 activation rows) on
// v_mfma_f32_32x32x16_bf16, for q4 (MLX affine, group 64) and GGUF Q5_K weights.
//
// At 64 rows a K=5120 -> N=17408 pair (gate and up, 95 MB of codes and sidecars) needs 22.8 GFLOP:
// about 9 us of MFMA at the dense bf16 peak and 12 us of VALU to dequantize, against 12-17 us of
// HBM. So every unit has to stay busy, and enough loads have to be in flight to cover HBM latency
// (about 16 MB across the chip). The structure:
//
//  * A wave owns 32 output columns of each of NW weights (NW = 2: fused gate+up, silu(g) * u) for
//    all rows (FM blocks of 32). Each weight is therefore dequantized exactly once, in registers,
//    straight into the MFMA B operand: lane (r, h) = (lane & 31, lane >> 5) feeds column r with the
//    eight weights of 16-byte activation piece 4 h + piece(i) of its wave's 64-element K slice in
//    sub-step i. The format class (Q4Format, Q5Format below) loads the codes and turns them into
//    those bf16 operands; everything else is shared.
//  * The A operand of sub-step i is the matching eight activations of row r. The KW waves of a
//    column slice split a step's K by 64-element slices and the CW column slices of a workgroup
//    share one activation chunk of KW slices, staged in LDS once per step: activations are read
//    from L2 once per workgroup.
//  * Weight codes are loaded three steps ahead into a register ring; the activation chunk and the
//    per-band sidecars (or block metadata) go straight from memory into one of four LDS buffers
//    (buffer loads with the LDS modifier), three steps ahead, ordered by counted vmcnt waits. One
//    barrier per step, in its middle.
//  * At the end of a job the KW partial sums meet in LDS and the workgroup writes whole output
//    rows. With a workspace, the (band, unit) pairs of all bands form one stream cut into equal
//    contiguous ranges, one a workgroup (stream-K); a band shared by several workgroups is summed
//    by the last of them to arrive.
//
// Numerics: w is the fp32 dequantized weight (one rounding, as DequantOracle.swift:20-21 for q4 and
// GgufQuant.swift:205-210 for Q5_K) rounded to bf16 (RNE), products exact in fp32, fp32
// accumulation.
#include "common.hpp"
#include "gguf_decode.hpp"
#include "launch.hpp"
#include "mix.hpp"

#include <cstdlib>
#include <type_traits>
// Weight codes are read once: non-temporal loads (gfx94x cache policy nt).
constexpr int kStreamCpol = 2;
// Stream-K partials cross XCDs: written and read through to memory (cache policy sc0 sc1).
constexpr int kDeviceCpol = 1 | 16;

namespace splosh {

constexpr int kMmaMaxGrid = 1024;  // workgroups of a stream-K launch
constexpr int kMmaMaxGroup = SPLOSH_MAX_GROUP;  // weights of a grouped call

// a / b for 0 <= a, 0 < b, in 32 bits when both fit (the stream-K bookkeeping divides wave-uniform
// values; a 64-bit division is a long VALU sequence, a 32-bit one a short one).
__device__ __forceinline__ int64_t div_nn(int64_t a, int64_t b) {
    if ((uint64_t)a <= 0xffffffffull && (uint64_t)b <= 0xffffffffull) return (int64_t)((uint32_t)a / (uint32_t)b);
    return a / b;
}

struct MmaArgs {
    // q4: the weight (gate) and, for the fused pair, up.
    const uint32_t *packed[2];
    const uint16_t *scales[2];
    const uint16_t *biases[2];
    int64_t stride_words;
    // Q5_K planes.
    const uint8_t *plane0, *plane1, *meta;
    int64_t n;
    int64_t units;      // K units of a band: q4 groups of 64, Q5_K blocks of 256
    const uint16_t *a;
    int64_t lda;
    void *out;
    int64_t ldc;
    const void *residual;
    int64_t rows;
    int out_dtype;
    float *partial;     // stream-K partials [gridDim.x][2][NW][rows][band columns]
    int *counters;      // arrivals per stream-K band (zero between calls)
    uint32_t partial_bytes;
    int dp_bands;       // bands computed whole (a multiple of gridDim.x)
    int64_t sk_units;   // (band, unit) pairs of the remaining bands
    // Buffer extents (the fits checks keep them < 4 GiB): q4 codes and sidecars, or Q5_K plane0,
    // plane1 and meta; activations.
    uint32_t code_bytes, sidecar_bytes, meta_bytes, a_bytes;
    uint32_t row_bytes;  // GGUF native blocks: bytes of a weight row
    int rows32;          // GGUF native blocks in the ROWS32 order (gguf_row)
    // The next RMSNorm's operand, emitted from the epilogue (single weight, fp32 output, N a multiple
    // of 64; null norm_weight: no emit): values = bf16(h norm_weight[col]), and per row and band of
    // 64 columns the sums of the rounded values and of h * h, h being the value written to `out`.
    const uint16_t *norm_weight;
    uint16_t *values;
    int64_t ldv;
    float *sums, *squares;   // [rows][n / 64]
    // A grouped call (several tiled weights on one activation, one launch): weight i owns bands
    // [gband[i], gband[i + 1]) of the band space and writes its own output; n, out, ldc and the
    // weight pointers above are unused.
    int ngroup;
    int gband[kMmaMaxGroup + 1];
    const uint32_t *gpacked[kMmaMaxGroup];
    const uint16_t *gscales[kMmaMaxGroup], *gbiases[kMmaMaxGroup];
    void *gout[kMmaMaxGroup];
    int64_t gn[kMmaMaxGroup], gldc[kMmaMaxGroup];
    // The weight of a grouped call that owns `band` (wave-uniform; a short scalar loop).
    __device__ int group_of(int band) const {
        int gi = 0;
        for (int i = 1; i < ngroup; ++i) gi = band >= gband[i] ? i : gi;
        return gi;
    }
};

// q4 (MLX affine): a step is KW groups of 64; wave kw takes group ga + t KW + kw and lane (r, h)
// feeds column r from words 4 h .. 4 h + 3 of the group's 32-byte record (one 16-byte load; a
// wave reads 32 consecutive records, a contiguous kilobyte of the tiled layout). A word becomes
// eight bf16 weights RNE(s q + b) in 19 instructions (dequant_word_fp8).
//
// Tiled weights stage a step's sidecars for the band (NW weights x {scale, bias} x KW groups x
// band columns of bf16) through LDS: waves 0 .. 2 NW - 1 each load one array of one weight, lane
// l < 8 KW bytes 16 (l & 7) .. of group l >> 3's 128-byte run (groups past the job re-read the
// last one). LDS layout per buffer: [weight][array][group][column]. Row-major weights load the
// sidecars per lane with the codes.
//
// GROUPED (one tiled weight a band, of a grouped call): each job takes its band's weight, buffer
// resources and column offset from the group table.
//
// SPLIT (NW = 2): one weight's two column halves as the pair -- rows [0, n) and [n, 2n) of the
// weight, the epilogue storing each half's sums to its own columns (no silu): half the jobs of a
// wide weight, each over twice the columns of one activation chunk.
template <int NW_, bool TILED, int CW, int KW, int D, bool GROUPED = false, bool EMIT = false, bool SPLIT = false>
struct Q4Format {
    static_assert(!GROUPED || (NW_ == 1 && TILED), "grouped calls take single tiled weights");
    static_assert(!SPLIT || NW_ == 2, "a split weight runs as a pair");
    static constexpr bool kGrouped = GROUPED;
    static constexpr bool kEmit = EMIT && !GROUPED;  // the epilogue emits the next norm's operand
    static constexpr bool kSplit = SPLIT;
    static constexpr int kTblBytes = 0;
    __device__ void build_table(char *, int) {}
    static constexpr int NW = NW_;
    static constexpr bool kStageSide = TILED;
    static constexpr int kWLoads = kStageSide ? NW : NW * 3;  // weight loads per wave and step
    static constexpr int kUnitK = kGroup;
    static constexpr int kBandCols = CW * 32;
    // The staged sidecars of a step: NW x 2 arrays x KW groups x the band's 64 columns (bf16), in
    // that order; wave v stages bytes [256 v, 256 v + 256), 4 a lane, with every lane's load
    // issued (waves past the NW * 4 that hold data read out of range into the rest of the buffer):
    // a branch there would split the step's schedule region and keep the compiler from
    // interleaving the MFMAs with the dequantization.
    static constexpr int kSBuf = kStageSide ? CW * KW * 256 : 0;
    static constexpr int kSideLoads = kStageSide ? 1 : 0;  // staging loads per wave and step
    static_assert(!kStageSide || (KW == 4 && kBandCols == 64 && CW * KW >= NW * 4),
                  "a wave's 256 bytes are two groups of one array");
    static constexpr int piece(int i) { return i; }

    rsrc_t q_rsrc[NW], s_rsrc[NW], b_rsrc[NW], side_rsrc;
    int wave, lane, kw, cw, r, h, ga, gb;
    uint32_t G32, q_lane, side_lane, q_group, side_group, side_src;
    int side_g;      // group (within a step) of this lane's staged sidecar dword
    bool side_bias;  // the array this wave stages: biases (else scales)
    bool side_on;    // this wave stages data (else it reads out of range)
    u32x4 wq[D][NW];
    uint32_t wsc[D][NW], wbi[D][NW];
    float cs[NW], cb[NW];  // scale and bias of the step being dequantized

    __device__ Q4Format(const MmaArgs &args, int wave_, int lane_) : wave(wave_), lane(lane_) {
        kw = wave / CW;
        cw = wave % CW;
        r = lane & 31;
        h = lane >> 5;
        G32 = (uint32_t)args.units;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            q_rsrc[w] = make_rsrc(args.packed[w], args.code_bytes);
            s_rsrc[w] = make_rsrc(args.scales[w], args.sidecar_bytes);
            b_rsrc[w] = make_rsrc(args.biases[w], args.sidecar_bytes);
        }
        // Wave v stages array a = v / 2 (weight a / 2, biases if a is odd), groups 2 (v % 2) and
        // 2 (v % 2) + 1 of the step: lane l the column pair l % 32 of group 2 (v % 2) + l / 32.
        const int arr = wave >> 1;
        side_on = (arr >> 1) < NW;
        const int side_w = side_on ? (arr >> 1) : 0;
        side_bias = (arr & 1) != 0;
        side_rsrc = make_rsrc(side_bias ? (const void *)args.biases[side_w] : (const void *)args.scales[side_w],
                              args.sidecar_bytes);
        side_g = 2 * (wave & 1) + (lane >> 5);
    }
    __device__ int steps(int ga_, int gb_) const { return (gb_ - ga_ + KW - 1) / KW; }
    __device__ bool active(int t) const { return ga + t * KW + kw < gb; }
    __device__ void begin(const MmaArgs &args, int band, int ga_, int gb_) {
        ga = ga_;
        gb = gb_;
        int64_t n = args.n;
        if constexpr (GROUPED) {
            const int gi = args.group_of(band);
            band -= args.gband[gi];
            n = args.gn[gi];
            q_rsrc[0] = make_rsrc(args.gpacked[gi], (uint32_t)n * G32 * 32u);
            side_rsrc = make_rsrc(side_bias ? (const void *)args.gbiases[gi] : (const void *)args.gscales[gi],
                                  (uint32_t)n * G32 * 2u);
        }
        const int64_t ncol = (int64_t)band * kBandCols + cw * 32 + r;
        const uint32_t col = (uint32_t)(ncol < n ? ncol : n - 1);
        if (TILED) {
            const uint32_t rec0 = (col >> 7) * G32 * 128u + (col & 127u);  // record of group 0
            q_lane = rec0 * 32u + 16u * h;
            side_lane = rec0 * 2u;
            q_group = 128u * 32u;
            side_group = 128u * 2u;
            const uint32_t n0 = (uint32_t)band * kBandCols;
            side_src = (((n0 >> 7) * G32 * 128u + (n0 & 127u)) * 2u) + 4u * (lane & 31);  // column pair lane % 32
        } else {
            q_lane = col * (uint32_t)args.stride_words * 4u + 16u * h;
            side_lane = col * G32 * 2u;
            q_group = 32u;
            side_group = 2u;
            side_src = 0;
        }
    }
    // Sidecars of step t, straight into LDS (the staging buffer `sbuf`): wave v writes bytes
    // [256 v, 256 v + 256). Groups past the job re-read the last one.
    __device__ void load_s(int t, char *sbuf) {
        if constexpr (kStageSide) {
            int g = ga + t * KW + side_g;
            g = g < gb ? g : gb - 1;
            buffer_load_lds4(side_rsrc, sbuf + wave * 256, side_on ? side_src + (uint32_t)g * 256u : 0xFFFFFFF0u);
        }
    }
    // Codes (and row-major sidecars) of step t into ring slot `slot`; the group is a wave-uniform
    // offset, clamped into the job so it stays in bounds.
    __device__ void load_w(int slot, int t) {
        int g = ga + t * KW + kw;
        g = g < gb ? g : gb - 1;
        const uint32_t ug = (uint32_t)__builtin_amdgcn_readfirstlane(g);
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            wq[slot][w] = buffer_load16_cp<kStreamCpol>(q_rsrc[w], q_lane, ug * q_group);
            if (!kStageSide) {
                wsc[slot][w] = buffer_load_u16(s_rsrc[w], side_lane, ug * side_group);
                wbi[slot][w] = buffer_load_u16(b_rsrc[w], side_lane, ug * side_group);
            }
        }
    }
    // The staged sidecars of the step after next sit in LDS buffer `sbuf` (recorded at the barrier
    // that makes them visible; read by prepare(), which measured faster for q4 than reading them a
    // step early into registers, as Q5Format does: the registers are not to spare here).
    const char *side_buf = nullptr;
    // One weight: the lane's scale and bias are read from LDS here, at the barrier a step before
    // prepare() needs them, so that the LDS latency does not stall the step (as Q5Format does with
    // its meta records; two weights would need more registers than the gate+up kernel has).
    uint32_t sb_pre = 0, bb_pre = 0;
    __device__ void fetch_side(const char *sbuf) {
        side_buf = sbuf;
        if constexpr (NW == 1 && kStageSide) {
            const char *base = sbuf + ((kw * kBandCols + cw * 32 + r) * 2);
            sb_pre = *(const uint16_t *)base;
            bb_pre = *(const uint16_t *)(base + KW * kBandCols * 2);
        }
    }
    // Coefficients of the step whose codes sit in `slot` (zeros when the step has no group for this
    // wave). The sidecars are read whatever `on` says and then scaled by 0 or 1 (exact), so that the
    // reads of both weights are issued together instead of behind a branch each.
    __device__ void prepare(int slot, bool on) {
        uint32_t sb[NW], bb[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            if (NW == 1 && kStageSide) {
                sb[w] = sb_pre;
                bb[w] = bb_pre;
            } else if (kStageSide) {
                const char *base = side_buf + (((w * 2) * KW + kw) * kBandCols + cw * 32 + r) * 2;
                sb[w] = *(const uint16_t *)base;
                bb[w] = *(const uint16_t *)(base + KW * kBandCols * 2);
            } else {
                sb[w] = wsc[slot][w];
                bb[w] = wbi[slot][w];
            }
        }
        const float one = on ? 1.0f : 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            cs[w] = bf16_bits_to_f32(sb[w]) * one;
            cb[w] = bf16_bits_to_f32(bb[w]) * one;
        }
    }
    __device__ bf16x8 operand(int w, int i, int slot) { return dequant_word_fp8(wq[slot][w][i], cs[w], cb[w]); }
};

// GGUF Q5_K in plane form (GgufPlanes.swift:8-20): a step is one 256-element block; wave kw takes
// its 32-element groups 2 kw and 2 kw + 1, lane (r, h) group j = 2 kw + h of column r: a 16-byte
// plane0 record of low nibbles and a 4-byte plane1 record of fifth bits. The block's 16-byte meta
// record (fp16 d and dmin, twelve bytes of packed 6-bit scales and minimums) of each band column
// is staged through LDS by waves 0 .. 3, a step ahead, like the q4 sidecars.
//
// Chunk order (gguf_formats.h:17-21): word c of a plane0 record holds elements 4c..4c+3 in its
// nibbles at bits 0, 16, 4, 20 and 16+4c..16+4c+3 at bits 8, 24, 12, 28; the fifth bit of the
// nibble at bit 4p + 16l sits at plane1 bit 8c + 2p + l. So w & 0x0F0F0F0F has the codes of
// elements (4c, 16+4c, 4c+1, 16+4c+1) in its bytes and (w >> 4) & 0x0F0F0F0F those of
// (4c+2, 16+4c+2, 4c+3, 16+4c+3), and the fifth bits reach bit 4 of those bytes by one multiply:
// byte x = plane1 >> 8c, ((x & 0x33) * 0x880110) & 0x10101010 moves bits 0, 4, 1, 5 to bits 4, 12,
// 20, 28 (the other partial products and their carries stay below or between them), and x >> 2
// does the same for the second set; both patterns come from a 256-entry LDS table built once a
// workgroup. Words 0 and 1 thus give elements 0..7 (bytes 0 and 2) and
// 16..23 (bytes 1 and 3) of the group, words 2 and 3 elements 8..15 and 24..31: sub-step i takes
// activation piece ((i & 1) << 1) | (i >> 1). w = code d sc - dmin mn as one fma (d sc, code d sc
// and dmin mn are exact in fp32), then RNE to bf16.
// FIFTH = false: Q4_K (no plane1; the codes are the nibbles).
template <int CW, int KW, int D, bool FIFTH = true>
struct Q5Format {
    static constexpr bool kGrouped = false;
    static constexpr bool kEmit = false;
    static constexpr bool kSplit = false;
    static constexpr int NW = 1;
    // The fifth bits of a plane1 byte x (four codes' worth for each of the two code words it
    // serves) at bit 4 of each byte: entry x = {((x & 0x33) * 0x880110) & 0x10101010, the same
    // of x >> 2}; one 8-byte LDS read instead of eight VALU a word.
    static constexpr int kTblBytes = FIFTH ? 256 * 8 : 0;
    const u32x2 *tbl = nullptr;
    __device__ void build_table(char *t, int tid) {
        tbl = (const u32x2 *)t;
        if (tid < 256) {
            const uint32_t x = (uint32_t)tid;
            const u32x2 e = {((x & 0x33u) * 0x880110u) & 0x10101010u, (((x >> 2) & 0x33u) * 0x880110u) & 0x10101010u};
            ((u32x2 *)t)[tid] = e;
        }
    }
    static constexpr int kWLoads = FIFTH ? 2 : 1;  // loads per wave and step: the mid-step wait counts them
    static constexpr int kUnitK = 256;
    static constexpr int kBandCols = CW * 32;
    // The band's 64 meta records of a step (1 KB); wave v stages bytes [256 v, 256 v + 256), 4 a
    // lane, every lane's load issued (waves 4 .. 7 read out of range into the rest of the buffer),
    // as the q4 sidecars.
    static constexpr int kSBuf = CW * KW * 256;
    static_assert(kBandCols * 16 <= 4 * 256 && CW * KW >= 4, "four waves stage the meta records");
    static constexpr int kSideLoads = 1;
    static_assert(KW == 4, "four waves cover the eight groups of a block");
    static_assert(kBandCols <= 64, "one wave loads the band's meta records");
    static constexpr int piece(int i) { return ((i & 1) << 1) | (i >> 1); }

    rsrc_t p0_rsrc, p1_rsrc, m_rsrc;
    int wave, lane, kw, cw, r, h, ga, gb;
    uint32_t blocks, p0_lane, p1_lane, m_lane;
    u32x4 wq[D];
    uint32_t wh[D];
    float scaled, offset;  // d sc and -(dmin mn) of the lane's group in the step being dequantized
    uint32_t lo[2], hi[2]; // 5-bit codes of two words, shared by two sub-steps

    __device__ Q5Format(const MmaArgs &args, int wave_, int lane_) : wave(wave_), lane(lane_) {
        kw = wave / CW;
        cw = wave % CW;
        r = lane & 31;
        h = lane >> 5;
        blocks = (uint32_t)args.units;
        p0_rsrc = make_rsrc(args.plane0, args.code_bytes);
        p1_rsrc = make_rsrc(FIFTH ? (const void *)args.plane1 : (const void *)args.plane0, FIFTH ? args.sidecar_bytes : 0u);
        m_rsrc = make_rsrc(args.meta, args.meta_bytes);
    }
    __device__ int steps(int ga_, int gb_) const { return gb_ - ga_; }
    __device__ bool active(int) const { return true; }
    // Records are ((row / 128) units + unit) 128 + row % 128 (GgufPlanes.swift:62-74), 8 groups
    // a block; a block step moves plane0 by 8 x 128 x 16 bytes, plane1 by 8 x 128 x 4, meta by
    // 128 x 16.
    __device__ void begin(const MmaArgs &args, int band, int ga_, int gb_) {
        ga = ga_;
        gb = gb_;
        const int64_t ncol = (int64_t)band * kBandCols + cw * 32 + r;
        const uint32_t col = (uint32_t)(ncol < args.n ? ncol : args.n - 1);
        const uint32_t rec0 = ((col >> 7) * blocks * 8u + 2u * kw + h) * 128u + (col & 127u);
        p0_lane = rec0 * 16u;
        p1_lane = rec0 * 4u;
        // The meta record word this lane stages: word l % 4 of band column 16 v + l / 4.
        const int64_t mcol64 = (int64_t)band * kBandCols + 16 * (wave & 3) + (lane >> 2);
        const uint32_t mcol = (uint32_t)(mcol64 < args.n ? mcol64 : args.n - 1);
        m_lane = ((mcol >> 7) * blocks * 128u + (mcol & 127u)) * 16u + 4u * (lane & 3);
    }
    __device__ uint32_t block(int t) const {
        const int b = ga + t < gb ? ga + t : gb - 1;
        return (uint32_t)__builtin_amdgcn_readfirstlane(b);
    }
    // Meta records of step t's block straight into LDS (`sbuf`, one 16-byte record a column).
    __device__ void load_s(int t, char *sbuf) {
        buffer_load_lds4(m_rsrc, sbuf + wave * 256, wave < 4 ? m_lane + block(t) * (128u * 16u) : 0xFFFFFFF0u);
    }
    __device__ void load_w(int slot, int t) {
        const uint32_t b = block(t);
        wq[slot] = buffer_load16_cp<kStreamCpol>(p0_rsrc, p0_lane, b * (8u * 128u * 16u));
        if constexpr (FIFTH) wh[slot] = buffer_load_u32(p1_rsrc, p1_lane, b * (8u * 128u * 4u));
        else wh[slot] = 0u;
    }
    // Scale and minimum of group j = 2 kw + h (GgufQuant.swift:196-203): packed byte k is meta byte
    // 4 + k, so for j < 4 (kw < 2, wave-uniform) sc and mn are the low six bits of meta bytes 4 + j
    // and 8 + j; for j >= 4 they are the nibbles of byte 12 + (j - 4) joined with the top two bits
    // of bytes 4 + (j - 4) and 8 + (j - 4). Either way the byte within its word is 2 (kw & 1) + h.
    // The meta record of the step after next, read from LDS a step before prepare() needs it, so
    // the LDS latency does not stall the step that uses it.
    u32x4 rm;
    __device__ void fetch_side(const char *sbuf) { rm = *(const u32x4 *)(sbuf + (cw * 32 + r) * 16); }
    __device__ void prepare(int, bool on) {
        const u32x4 m = rm;
        const float d = half_bits_to_f32(m[0]), dmin = half_bits_to_f32(m[0] >> 16);
        const uint32_t sh = 8u * (2u * (kw & 1) + h);
        uint32_t sc, mn;
        if (kw < 2) {
            sc = __builtin_amdgcn_ubfe(m[1], sh, 6);
            mn = __builtin_amdgcn_ubfe(m[2], sh, 6);
        } else {
            sc = __builtin_amdgcn_ubfe(m[3], sh, 4) | (__builtin_amdgcn_ubfe(m[1], sh + 6, 2) << 4);
            mn = __builtin_amdgcn_ubfe(m[3], sh + 4, 4) | (__builtin_amdgcn_ubfe(m[2], sh + 6, 2) << 4);
        }
        scaled = on ? d * (float)sc : 0.0f;
        offset = on ? -(dmin * (float)mn) : 0.0f;
    }
    __device__ float weight(uint32_t codes, int j) const { return __builtin_fmaf(cvt_byte(codes, j), scaled, offset); }
    __device__ bf16x8 operand(int, int i, int slot) {
        if ((i & 1) == 0) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int c = i + e;
                const uint32_t w = wq[slot][c];
                lo[e] = w & 0x0F0F0F0Fu;
                hi[e] = (w >> 4) & 0x0F0F0F0Fu;
                if constexpr (FIFTH) {
                    const u32x2 f = tbl[__builtin_amdgcn_ubfe(wh[slot], 8 * c, 8)];
                    lo[e] |= f[0];
                    hi[e] |= f[1];
                }
            }
        }
        const int b = i & 1;  // byte b and b + 2: the lower (0) or upper (1) four elements of a word
        u32x4 d;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            d[2 * e] = f32x2_to_bf16x2(weight(lo[e], b), weight(lo[e], b + 2));
            d[2 * e + 1] = f32x2_to_bf16x2(weight(hi[e], b), weight(hi[e], b + 2));
        }
        return as_bf16x8(d);
    }
};

// GGUF native blocks (Q8_0, IQ4_NL, Q6_K, Q3_K, IQ3_S, IQ4_XS; GgufQuant.swift:136-300), rows of
// blocks back to back as the file holds them: a step is 256 elements of K (one super-block, or
// eight 32-element blocks); wave kw takes its 32-element groups 2 kw and 2 kw + 1, lane (r, h)
// group j = 2 kw + h of column r, fetched by gguf_fetch (every load per lane, the blocks being
// 2-byte aligned at best) D steps ahead like the q4 codes. prepare() takes the group's scales and
// aligned words from the ring slot; operand(i) decodes elements 8 i .. 8 i + 7 in the reference
// decoder's fp32 operation order (gguf_decode) and rounds them to bf16 (RNE), the MFMA's B operand
// -- the same weights as the tiled and prefill kernels use.
template <int TYPE, int CW, int KW, int D>
struct GgufFormat {
    static constexpr bool kGrouped = false;
    static constexpr bool kEmit = false;
    static constexpr bool kSplit = false;
    static constexpr int NW = 1;
    // IQ3_S: the codebook's four magnitudes of each of its 512 entries as bytes, in LDS.
    static constexpr int kTblBytes = TYPE == 21 ? 512 * 4 : 0;
    const uint32_t *tbl = nullptr;
    __device__ void build_table(char *t, int tid) {
        if constexpr (TYPE == 21) {
            tbl = (const uint32_t *)t;
            if (tid < 512) {
                const uint32_t packed = kIq3sPacked[tid];
                uint32_t m = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q) m |= (2u * ((packed >> (3 * q)) & 7u) + 1u) << (8 * q);
                ((uint32_t *)t)[tid] = m;
            }
        }
    }
    // Buffer loads of gguf_fetch<TYPE> as issued (the mid-step wait counts them; IQ3_S's two
    // dword loads of codebook indices merge into one); the assembly check in the tests fails if
    // the code issues fewer.
    static constexpr int kWLoads = TYPE == 8 ? 4 : TYPE == 20 ? 3 : TYPE == 14 ? 8 : TYPE == 11 ? 9 : TYPE == 21 ? 7 : 4;
    static constexpr int kUnitK = 256;
    static constexpr int kBandCols = CW * 32;
    static constexpr int kSBuf = 0;
    static constexpr int kSideLoads = 0;
    static_assert(KW == 4, "four waves cover the eight groups of a step");
    static constexpr int piece(int i) { return i; }

    rsrc_t rs;
    int kw, cw, r, h, ga, gb;
    GgufRow row;
    GgufRaw<TYPE> raw[D];
    // The group being dequantized: its scales (zero when the step has no group for this wave) and
    // its code words in place.
    float s0, s1;
    uint32_t wd[8];
    uint32_t extra;  // IQ3_S: the group's ninth bits

    __device__ GgufFormat(const MmaArgs &args, int wave, int lane) {
        kw = wave / CW;
        cw = wave % CW;
        r = lane & 31;
        h = lane >> 5;
        rs = make_rsrc(args.plane0, args.code_bytes);
    }
    __device__ int steps(int ga_, int gb_) const { return gb_ - ga_; }
    __device__ bool active(int) const { return true; }
    __device__ void begin(const MmaArgs &args, int band, int ga_, int gb_) {
        ga = ga_;
        gb = gb_;
        const int64_t ncol = (int64_t)band * kBandCols + cw * 32 + r;
        row = gguf_row<TYPE>((uint32_t)(ncol < args.n ? ncol : args.n - 1), args.row_bytes, args.rows32);
    }
    __device__ void load_s(int, char *) {}
    __device__ void fetch_side(const char *) {}
    __device__ void load_w(int slot, int t) {
        const int b = ga + t < gb ? ga + t : gb - 1;
        const int ub = __builtin_amdgcn_readfirstlane(b);
        raw[slot] = gguf_fetch<TYPE>(rs, row, 8 * ub + 2 * kw + h);
    }
    __device__ void prepare(int slot, bool on) {
        const GgufRaw<TYPE> &w = raw[slot];
        const float one = on ? 1.0f : 0.0f;
        if constexpr (TYPE == 8) {
            s0 = half_bits_to_f32(w.d) * one;
            uint32_t t[8];
            align_span(w.codes, t);
#pragma unroll
            for (int q = 0; q < 8; ++q) wd[q] = t[q];
        } else if constexpr (TYPE == 20) {
            s0 = half_bits_to_f32(w.d) * one;
            uint32_t t[4];
            align_span(w.codes, t);
#pragma unroll
            for (int q = 0; q < 4; ++q) wd[q] = t[q];
        } else if constexpr (TYPE == 23) {
            const int j = w.j;
            const uint32_t low = (w.lowb >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
            const uint32_t scale = low | (((w.high >> (2 * j)) & 3) << 4);
            s0 = half_bits_to_f32(w.d) * ((float)scale - 32.0f) * one;
#pragma unroll
            for (int q = 0; q < 4; ++q) wd[q] = w.q[q];
        } else if constexpr (TYPE == 14) {
            const int quarter = w.j & 3;
            const float d = half_bits_to_f32(w.d);
            s0 = d * (float)(int8_t)(w.sc & 0xFF) * one;
            s1 = d * (float)(int8_t)(w.sc >> 8) * one;
            uint32_t ql[8], qh[8];
            align_span(w.ql, ql);
            align_span(w.qh, qh);
            const int lsh = 4 * (quarter >> 1), hsh = 2 * quarter;
#pragma unroll
            for (int q = 0; q < 8; ++q) wd[q] = ((ql[q] >> lsh) & 0x0F0F0F0Fu) | (((qh[q] >> hsh) & 0x03030303u) << 4);
        } else if constexpr (TYPE == 11) {
            const int j = w.j, shift = 2 * (j & 3), word = j >> 1;
            const float d = half_bits_to_f32(w.d);
            const uint32_t lows = w.lows >> (4 * (word >> 1)), highs = w.highs >> (2 * word);
            s0 = d * ((float)((lows & 0xF) | ((highs & 3) << 4)) - 32.0f) * one;
            s1 = d * ((float)(((lows >> 8) & 0xF) | (((highs >> 8) & 3) << 4)) - 32.0f) * one;
            uint32_t hm[8], qs[8];
            align_span(w.hm, hm);
            align_span(w.qs, qs);
#pragma unroll
            for (int q = 0; q < 8; ++q) wd[q] = ((qs[q] >> shift) & 0x03030303u) | (((hm[q] >> j) & 0x01010101u) << 2);
        } else {
            const int j = w.j;
            const uint32_t scale = (w.scale >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
            s0 = half_bits_to_f32(w.d) * (1.0f + 2.0f * (float)scale) * one;
            extra = (w.ninth >> (8 * (j & 1))) & 0xFF;
            uint32_t cb[2], sg[1];
            align_span(w.cb, cb);
            align_span(w.sg, sg);
            wd[0] = cb[0];
            wd[1] = cb[1];
            wd[2] = sg[0];
        }
    }
    // Elements 8 i .. 8 i + 7 of the group as bf16 (RNE) in k order, each the decoder's value
    // (gguf_decode, same fp32 operations).
    __device__ bf16x8 operand(int, int i, int) {
        float v[8];
        if constexpr (TYPE == 8) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = s0 * (float)(int8_t)((wd[2 * i + (e >> 2)] >> (8 * (e & 3))) & 0xFF);
        } else if constexpr (TYPE == 20 || TYPE == 23) {
            // Element e < 16: the low nibble of byte e; e >= 16: the high nibble of byte e - 16.
            const int hi = i >> 1;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint32_t x = wd[2 * (i & 1) + q];
                const uint32_t vals = iq4_lookup4(hi ? (x >> 4) & 0x0F0F0F0Fu : x & 0x0F0F0F0Fu);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * q + e] = s0 * (float)(int8_t)((vals >> (8 * e)) & 0xFF);
            }
        } else if constexpr (TYPE == 14 || TYPE == 11) {
            // ds (c - o) as fma(c, ds, -o ds): o is a power of two, so -o ds is exact, the fma's
            // sum is ds (c - o) exactly and its one rounding is the product's.
            constexpr float kOff = TYPE == 14 ? 32.0f : 4.0f;
            const float ds = i < 2 ? s0 : s1;
            const float nd = -kOff * ds;
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * q + e] = __builtin_fmaf(cvt_byte(wd[2 * i + q], e), ds, nd);
        } else {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int k = 2 * i + q;
                const uint32_t code = ((wd[k >> 2] >> (8 * (k & 3))) & 0xFF) | (((extra >> k) & 1) << 8);
                const uint32_t m = tbl[code];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x = s0 * cvt_byte(m, e);
                    const uint32_t sign = ((wd[2] >> (4 * k + e)) & 1u) << 31;
                    v[4 * q + e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) ^ sign);
                }
            }
        }
        u32x4 d;
#pragma unroll
        for (int p = 0; p < 4; ++p) d[p] = f32x2_to_bf16x2(v[2 * p], v[2 * p + 1]);
        return as_bf16x8(d);
    }
};

template <int FM, int NW, int CW, int KW, int D, int SBUF, int TBL = 0>
struct MmaShape {
    static constexpr int kThreads = CW * KW * 64;
    static constexpr int kRows = FM * 32;
    static constexpr int kBandCols = CW * 32;
    static constexpr int kKc = KW * 8;                             // 16-byte pieces per chunk row
    static constexpr int kAPieces = kRows * kKc;
    static_assert(kAPieces % kThreads == 0, "whole activation pieces per thread");
    static constexpr int kAPer = kAPieces / kThreads;              // activation loads per wave and step
    static constexpr int kABuf = kAPieces * 16;                    // bytes of one chunk buffer
    static constexpr int kSBuf = SBUF;                             // bytes of one staged-sidecar buffer
    static constexpr int kNB = 4;                                  // stage buffers (chunk + sidecars)
    static constexpr int kAcc = FM * NW * 16;                      // accumulator floats per lane
    static constexpr size_t kRedBytes = (size_t)KW * CW * kAcc * 64 * sizeof(float);
    static constexpr size_t kABytes = (size_t)kNB * (kABuf + kSBuf);
    static constexpr size_t kEmitBytes = (size_t)kRows * 2 * 2 * sizeof(float);  // emit band sums
    // The format's lookup table (TBL bytes, kept for the whole kernel) after the rest.
    static constexpr size_t kTblAt = kRedBytes + kEmitBytes > kABytes ? kRedBytes + kEmitBytes : kABytes;
    static constexpr size_t kLds = kTblAt + TBL;
    static_assert(D >= 3, "the pipeline below keeps weights at least three steps ahead");
    static_assert(kLds <= 160 * 1024, "the workgroup's LDS fits a CU");
};

// Work split. The N columns form `bands` bands of CW * 32. Bands [0, dp_bands) are computed whole
// by workgroup (band mod gridDim.x), written straight to the output. The (band, unit) pairs of the
// other bands, sk_units of them, are cut into gridDim.x equal contiguous ranges (stream-K), one a
// workgroup. Only a range's first and last band can be partial: their fp32 partials go to slot 0
// and 1 of the workgroup's workspace. The workgroups sharing a band count their arrivals on the
// band's counter, and the last one sums the partials and writes the band.
//
// Pipeline of a job (units [ga, gb) of one band), in steps of KW x 64 elements of K, D steps deep:
// weight codes go to a D-slot register ring, the activation chunk of a step (rows x KW x 64) and
// its sidecars via registers to LDS buffer t mod 3, the chunk XOR-swizzled (16-byte piece kc of
// row m at position kc ^ (m & 15)) so the MFMA operand reads do not conflict. Barriers wait for LDS
// traffic only, never for global stores.
template <class F, int FM, int CW, int KW, int D>
__global__ void __launch_bounds__(CW * KW * 64)
mma_kernel(MmaArgs args) {
    constexpr int NW = F::NW;
    using S = MmaShape<FM, NW, CW, KW, D, F::kSBuf, F::kTblBytes>;
    static_assert(F::kBandCols == S::kBandCols, "one band geometry");
    constexpr int kWLoads = F::kWLoads;
    extern __shared__ __align__(16) uint16_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cw = wave % CW, kw = wave / CW;
    const int r = lane & 31, h = lane >> 5;
    const int U = (int)args.units;

    const rsrc_t a_rsrc = make_rsrc(args.a, args.a_bytes);
    const int P = gridDim.x;
    const rsrc_t p_rsrc = make_rsrc(args.partial, args.partial_bytes);
    // Workgroup i takes stream-K units [sk_start(i), sk_start(i + 1)).
    auto sk_start = [&](int i) { return div_nn(args.sk_units * i, P); };
    __shared__ int fix_count;
    __shared__ uint16_t fix_list[kMmaMaxGrid];  // contributors of a shared band: 2 wg + slot
    F fmt(args, wave, lane);
    // The format's lookup table, written here and first read after the job prologue's barrier.
    if constexpr (F::kTblBytes > 0) fmt.build_table((char *)lds + S::kTblAt, tid);
    // Activation staging: this thread's piece j of a chunk sits at buffer position
    // (wave * kAPer + j) * 64 + lane, i.e. row m = pos / kKc, holding piece kc = (pos % kKc) ^ (m & 15)
    // of the row (an XOR swizzle, so the MFMA operand reads do not conflict), read from byte
    // (m lda + k0 + 8 kc) * 2. Rows past the last are clamped (their outputs are not stored);
    // K past the job belongs to inactive waves; reads past the buffer return zero.
    uint32_t a_src[S::kAPer];
#pragma unroll
    for (int j = 0; j < S::kAPer; ++j) {
        const int pos = (wave * S::kAPer + j) * 64 + lane;
        const int row = pos / S::kKc, kc = (pos % S::kKc) ^ (row & 15);
        const int64_t rc = row < args.rows ? row : args.rows - 1;
        a_src[j] = (uint32_t)((rc * args.lda + kc * 8) * 2);
    }
    // MFMA operand reads: sub-step i of block f takes row 32 f + r, piece kw * 8 + 4 h + piece(i).
    uint32_t a_rd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        a_rd[i] = (uint32_t)((r * S::kKc + ((kw * 8 + 4 * h + F::piece(i)) ^ (r & 15))) * 16);
    char *lds_bytes = (char *)lds;
    char *side_lds = lds_bytes + S::kNB * S::kABuf;

    // The K-summed results of a job, in the MFMA output layout: wave (kw, cw) owns rows
    // 32 f + 8 kw + 4 h + i (i < 4) of band column cw 32 + r, for each weight.
    f32x4 fin[NW][FM];

    // One job: column band `band`, units [ga, gb); leaves its sums in `fin`. `after_prologue`
    // runs once every wave has passed the prologue's barrier (all of the workgroup's earlier
    // stores are complete by then).
    // The emit's norm weight of the lane's column of the job's band, loaded when the job starts
    // (its latency hides behind the job instead of stalling the epilogue).
    int wn_band = -1;
    uint32_t wn_bits = 0;
    auto run_job = [&](int band, int ga, int gb, auto &&after_prologue) {
        const int T = fmt.steps(ga, gb);
        fmt.begin(args, band, ga, gb);
        if constexpr (NW == 1 && F::kEmit) {
            if (args.norm_weight) {
                const int64_t c = (int64_t)band * S::kBandCols + cw * 32 + r;
                wn_band = band;
                wn_bits = args.norm_weight[c < args.n ? c : args.n - 1];
            }
        }

        // Pieces [j0, j1) of chunk t, straight from memory into LDS buffer `buf` (buffer loads with
        // the LDS modifier: lane l of the wave's piece j lands at ((wave kAPer + j) 64 + l) 16).
        // They count in vmcnt like any load and are complete in LDS when it says so.
        auto load_a_part = [&](int t, int buf, int j0, int j1) {
            const uint32_t gbyte = (uint32_t)(ga * F::kUnitK + t * KW * 64) * 2u;
#pragma unroll
            for (int j = j0; j < j1; ++j)
                buffer_load_lds16(a_rsrc, lds_bytes + buf * S::kABuf + (wave * S::kAPer + j) * 1024, a_src[j] + gbyte);
        };
        auto load_a = [&](int t, int buf) { load_a_part(t, buf, 0, S::kAPer); };
        constexpr int kAHalf = (S::kAPer + 1) / 2;
        // Stage j = the activation chunk of step j and the sidecars (or block metadata) of step
        // j + 1, both straight into buffer j mod 4 (chunk area and sidecar area).
        auto load_side = [&](int t, int buf) { fmt.load_s(t, side_lds + buf * S::kSBuf); };
        auto load_w = [&](int slot_, int t) { fmt.load_w(slot_, t); };
        // Loads a wave issues per stage, and the mid-step wait: at the middle of step t the wave
        // needs stage t + 1 (issued in step t - 2); after it it has issued the weights of step
        // t + 2, stage t + 2 and the weights of step t + 3, which may stay in flight.
        constexpr int kStageLoads = S::kAPer + F::kSideLoads;
        constexpr int kMidWait = 2 * kWLoads + kStageLoads;
        static_assert(kMidWait + kWLoads + kStageLoads <= 63, "vmcnt holds 6 bits");
        // Dequantized weights of the current step; operand i is replaced by the next step's as
        // soon as the MFMAs of sub-step i have been issued.
        bf16x8 bw[NW][4];
        auto fetch_side = [&](int sbuf) { fmt.fetch_side(side_lds + sbuf * S::kSBuf); };
        auto dequant = [&](int slot_, int sbuf, bool on) {
            fetch_side(sbuf);
            fmt.prepare(slot_, on);
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int i = 0; i < 4; ++i) bw[w][i] = fmt.operand(w, i, slot_);
        };

        f32x16 acc[NW][FM];
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int f = 0; f < FM; ++f)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[w][f][e] = 0.0f;

        // The step count is padded to a multiple of 3 (the weight ring's depth): steps past T
        // compute nothing but keep the load pattern regular (their loads re-read in-bounds data).
        // Each step has its barrier in the middle, between MFMA sub-steps 1 and 2. There the wave
        // waits for stage t + 1 (loaded two steps earlier), passes the barrier and reads the next
        // step's first activation fragments; after the barrier it issues stage t + 3 into buffer
        // t + 3 mod 4, which last held stage t - 1: chunk t - 1 (read in step t - 1) and the
        // sidecars of step t (read at the start of step t - 1), both finished by every wave before
        // this barrier. Loads complete in issue order (vmcnt counts down in order, and a load
        // into LDS counts like any other and has written LDS when it is counted off), so "stage
        // t + 1 has arrived" is "at most the kMidWait loads issued after it are outstanding":
        // the weights of steps t + 2 and t + 3 stay in flight across the wait. The compiler does
        // not track loads into LDS, so these waits, the barriers and the issue order (kept by the
        // sched_barriers) are the whole of their synchronisation.
        const int Tp = (T + D - 1) / D * D;
        auto nbuf = [&](int b) { return (b + 1) & (S::kNB - 1); };
        static_assert(S::kNB == 4, "buffer arithmetic mod 4");
        load_side(0, 3);  // sidecars of step 0: "stage -1"
        load_w(0, 0);
        load_a(0, 0);
        load_side(1, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_w(1, 1);
        load_a(1, 1);
        load_side(2, 1);
        __builtin_amdgcn_sched_barrier(0);
        load_w(2, 2);
        load_a(2, 2);
        load_side(3, 2);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 3; j < D; ++j) load_w(j, j);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(D - 1) * kWLoads + 2 * kStageLoads>();  // stage -1, stage 0 and the weights of step 0
        lds_barrier_staged<2 * kStageLoads>();         // stages 1 and 2 may be in flight
        after_prologue();
        dequant(0, 3, T > 0 && fmt.active(0));
        auto read_af = [&](bf16x8 *dst, int buf, int i) {
            const char *ap = lds_bytes + buf * S::kABuf;
#pragma unroll
            for (int f = 0; f < FM; ++f) dst[f] = as_bf16x8(*(const u32x4 *)(ap + a_rd[i] + f * 32 * S::kKc * 16));
        };
        bf16x8 af_pre[FM];  // sub-step 0 fragments of the current step
        read_af(af_pre, 0, 0);
        fetch_side(0);  // the sidecars of step 1 came with stage 0

        // Step t: MFMA sub-steps with the dequantization of step t + 1 interleaved, `mid` between
        // sub-steps 1 and 2.
        // Every step issues its MFMAs; a step with no unit for this wave (stream-K tails, padding)
        // gets zero coefficients, so its weights dequantize to exact zeros and add nothing (an
        // infinite activation would turn that into NaN, where its row is not finite anyway). A
        // branch-free body keeps the register allocation of one path.
        auto live = [&](int t) { return t < T && fmt.active(t); };
        auto step = [&](int t, int d, int abuf, auto &&mid, auto &&hook) {
            const int next = (d + 1) % D;
            // The sidecars of step t + 1 came with stage t (buffer t mod 4 = abuf), fetched at the
            // previous step's barrier.
            fmt.prepare(next, live(t + 1));
            // Fragments of sub-step i + 1 are read as soon as sub-step i's MFMAs are issued, so their
            // LDS latency hides behind the dequantization (two alternating register sets; sub-step 0
            // uses af_pre, read at the previous step's barrier).
            bf16x8 af_odd[FM], af_even[FM];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i == 2) mid();
                bf16x8 *af = i == 0 ? af_pre : (i & 1) ? af_odd : af_even;
#pragma unroll
                for (int w = 0; w < NW; ++w)
#pragma unroll
                    for (int f = 0; f < FM; ++f)
                        acc[w][f] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[f], bw[w][i], acc[w][f], 0, 0, 0);
                if (i < 3) read_af(((i + 1) & 1) ? af_odd : af_even, abuf, i + 1);
#pragma unroll
                for (int w = 0; w < NW; ++w) bw[w][i] = fmt.operand(w, i, next);
                hook(i);
                __builtin_amdgcn_sched_barrier(0);  // sub-steps stay in order (register pressure, load order)
            }
        };

        // Loads are spread over the step so that the workgroup's waves do not all queue at the
        // texture unit at once: sub-step 0 issues the weights of step t + 3 (their ring slot was
        // dequantized in step t - 1), sub-steps 2 and 3 the halves of stage t + 3.
        int abuf = 0;  // buffer of step t's chunk
        for (int t0 = 0; t0 < Tp - D; t0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int t = t0 + d;
                const int sbuf = (abuf + 3) & 3;  // stage t + 3
                step(t, d, abuf,
                     [&] {
                         wait_vmcnt<kMidWait>();  // stage t + 1 has arrived
                         lds_barrier_staged<kStageLoads>();  // stage t + 2 may be in flight
                         read_af(af_pre, nbuf(abuf), 0);
                         fetch_side(nbuf(abuf));  // the sidecars of step t + 2 (stage t + 1)
                     },
                     [&](int i) {
                         if (i == 0) load_w(d, t + D);
                         if (i == 2) {
                             load_a_part(t + 3, sbuf, 0, kAHalf);
                             load_side(t + 4, sbuf);
                         }
                         if (i == 3) load_a_part(t + 3, sbuf, kAHalf, S::kAPer);
                     });
                abuf = nbuf(abuf);
            }
        }
        // The last D steps load no weights (every step's were issued already) and, but for D - 3 of
        // them, no stages; they wait for everything. Steps past T (at most D - 1; T is uniform over
        // the workgroup) are skipped.
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int t = Tp - D + d;
            if (t >= T) break;
            const int sbuf = (abuf + 3) & 3;  // stage t + 3
            step(t, d, abuf,
                 [&] {
                     wait_vmcnt<0>();
                     lds_barrier();
                     if (d < D - 1) {
                         read_af(af_pre, nbuf(abuf), 0);
                         fetch_side(nbuf(abuf));
                     }
                 },
                 [&](int i) {
                     if (d + 3 < D) {
                         if (i == 2) {
                             load_a_part(t + 3, sbuf, 0, kAHalf);
                             load_side(t + 4, sbuf);
                         }
                         if (i == 3) load_a_part(t + 3, sbuf, kAHalf, S::kAPer);
                     }
                 });
            abuf = nbuf(abuf);
        }
        wait_vmcnt<0>();  // nothing is in flight any more (the last steps waited); stated for every path
        lds_barrier();    // every wave is past its last fragment read
        // The last barrier also ended every read of the chunk buffers.

        // Sum the KW K-slices: every wave parks its accumulators in LDS as 16-byte quarters
        // ([kw][cw][w][f][quarter][lane], conflict-free), and wave kw collects quarter kw of its
        // column slice from all KW waves, in kw order (the same order whatever the timing).
        {
            char *x = (char *)lds;
            auto xoff = [&](int s, int w, int f, int q) {
                return (((((s * CW + cw) * NW + w) * FM + f) * 4 + q) * 64 + lane) * 16;
            };
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int f = 0; f < FM; ++f)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *(f32x4 *)(x + xoff(kw, w, f, q)) =
                            f32x4{acc[w][f][4 * q], acc[w][f][4 * q + 1], acc[w][f][4 * q + 2], acc[w][f][4 * q + 3]};
            lds_barrier();
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int f = 0; f < FM; ++f) {
                    f32x4 sum = *(const f32x4 *)(x + xoff(0, w, f, kw));
#pragma unroll
                    for (int s2 = 1; s2 < KW; ++s2) sum += *(const f32x4 *)(x + xoff(s2, w, f, kw));
                    fin[w][f] = sum;
                }
        }
    };

    const int rows = (int)args.rows;
    // Row i of this lane's quarter of block f, and the lane's band column.
    auto own_row = [&](int f, int i) { return 32 * f + 8 * kw + 4 * h + i; };
    const int bcol = cw * 32 + r;
    // The epilogue of a finished band: every wave calls it (the emit's band sums meet in LDS).
    auto store_out = [&](int band, const f32x4 (&v)[NW][FM]) {
        void *out = args.out;
        int64_t ldc = args.ldc, n = args.n;
        if constexpr (F::kGrouped) {
            const int gi = args.group_of(band);
            out = args.gout[gi];
            ldc = args.gldc[gi];
            n = args.gn[gi];
            band -= args.gband[gi];
        }
        const int64_t ocol = (int64_t)band * S::kBandCols + bcol;
        if constexpr (F::kSplit) {
            // Half w's columns start at w n.
#pragma unroll
            for (int w = 0; w < 2; ++w)
#pragma unroll
                for (int f = 0; f < FM; ++f)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int m = own_row(f, i);
                        if (m >= rows || ocol >= n) continue;
                        const int64_t index = (int64_t)m * ldc + ocol + w * n;
                        float value = v[w][f][i];
                        if (args.out_dtype == SPLOSH_F32) {
                            if (args.residual) value += ((const float *)args.residual)[index];
                            ((float *)out)[index] = value;
                        } else {
                            if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                            ((uint16_t *)out)[index] = f32_to_bf16(value);
                        }
                    }
            return;
        }
        float hv[FM][4];
#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = own_row(f, i);
                float value = v[0][f][i];
                if constexpr (NW == 2) value = silu(v[0][f][i]) * v[1][f][i];
                hv[f][i] = value;
                if (m >= rows || ocol >= n) continue;
                const int64_t index = (int64_t)m * ldc + ocol;
                if (args.out_dtype == SPLOSH_F32) {
                    if (args.residual) value += ((const float *)args.residual)[index];
                    ((float *)out)[index] = value;
                } else {
                    if (args.residual) value += bf16_bits_to_f32(((const uint16_t *)args.residual)[index]);
                    ((uint16_t *)out)[index] = f32_to_bf16(value);
                }
                hv[f][i] = value;
            }
        if constexpr (NW == 1 && F::kEmit) {
            if (args.norm_weight) {
                // Emit (engine_na.metal:365-411 restated): the rounded operand, then per row the
                // band's sums: over this wave's 32 columns inside the lane half that holds the
                // rows, then the two column waves' halves through LDS. The 32-lane sums of the
                // lane's NQ rows run as a reduce-scatter (exchange half the rows with lane r ^ 16,
                // then a quarter with r ^ 8, ...; plain sums over the lanes left): 31 shuffles a
                // quantity at most instead of 5 a row. Lane r ends with the sum of slot
                // q(r) = sum over level k of bit 4 - k of r times NQ / 2^(k+1).
                const float wn = bf16_bits_to_f32(band == wn_band ? wn_bits : (uint32_t)args.norm_weight[ocol]);
                float *part = (float *)((char *)lds + S::kRedBytes);  // [FM * 32 rows][2 cw][2]
                const int64_t groups = args.n / 64;
                constexpr int NQ = FM * 4;
                constexpr int L = NQ == 16 ? 4 : NQ == 8 ? 3 : 2;  // reduce-scatter levels
                auto lane_sum = [&](float (&x)[NQ]) {
#pragma unroll
                    for (int k = 0; k < L; ++k) {
                        // Keep slots [0, half) (the upper lane of the pair r, r ^ 2 half: slots
                        // [half, 2 half), moved down) and add the partner's copy of them.
                        const int half = NQ >> (k + 1), xm = 16 >> k;
                        const bool upper = (r & xm) != 0;
#pragma unroll
                        for (int j = 0; j < half; ++j) {
                            const float keep = upper ? x[half + j] : x[j], give = upper ? x[j] : x[half + j];
                            x[j] = keep + __shfl_xor(give, xm, 64);
                        }
                    }
#pragma unroll
                    for (int xm = 16 >> L; xm >= 1; xm >>= 1) x[0] += __shfl_xor(x[0], xm, 64);
                    return x[0];
                };
                int q = 0;
#pragma unroll
                for (int k = 0; k < L; ++k) q += ((r >> (4 - k)) & 1) * (NQ >> (k + 1));
                const bool lead = (r & ((32 >> L) - 1)) == 0;
                const int qm = own_row(q >> 2, q & 3);
                float x[NQ];
#pragma unroll
                for (int f = 0; f < FM; ++f)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int m = own_row(f, i);
                        const uint16_t vb = f32_to_bf16(hv[f][i] * wn);
                        if (m < rows) args.values[(int64_t)m * args.ldv + ocol] = vb;
                        x[f * 4 + i] = bf16_bits_to_f32(vb);
                    }
                const float sv = lane_sum(x);
                if (lead) part[(qm * 2 + cw) * 2] = sv;
#pragma unroll
                for (int f = 0; f < FM; ++f)
#pragma unroll
                    for (int i = 0; i < 4; ++i) x[f * 4 + i] = hv[f][i] * hv[f][i];
                const float sq = lane_sum(x);
                if (lead) part[(qm * 2 + cw) * 2 + 1] = sq;
                __syncthreads();
                if (cw == 0 && r == 0) {
#pragma unroll
                    for (int f = 0; f < FM; ++f)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int m = own_row(f, i);
                            if (m >= rows) continue;
                            args.sums[(int64_t)m * groups + band] = part[m * 4] + part[m * 4 + 2];
                            args.squares[(int64_t)m * groups + band] = part[m * 4 + 1] + part[m * 4 + 3];
                        }
                }
                __syncthreads();  // the band sums are read before the next band writes them
            }
        }
    };
    // Partial of workgroup wg, slot sl, weight w, row m, this lane's band column: a byte offset
    // into the partial area ([grid][2][NW][rows][band columns] fp32).
    auto part_off = [&](int wg, int sl, int w, int m) {
        return (uint32_t)((((wg * 2 + sl) * NW + w) * rows + m) * S::kBandCols + bcol) * 4u;
    };
    // Written through to memory (gfx94x cache policy sc0 sc1): the workgroup that sums the band
    // may run on another XCD, whose L2 is not coherent with this one's.
    auto write_partial = [&](int sl) {
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int f = 0; f < FM; ++f) {
                const u32x4 bits = __builtin_bit_cast(u32x4, fin[w][f]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = own_row(f, i);
                    if (m < rows) __builtin_amdgcn_raw_buffer_store_b32(bits[i], p_rsrc, part_off(blockIdx.x, sl, w, m), 0, kDeviceCpol);
                }
            }
    };
    // The contributors of a shared band (workgroups whose non-empty range meets it), in order,
    // each as 2 wg + the slot it used: 1 if its range began in an earlier band. Thread 0 fills
    // fix_list; the count is returned to every thread.
    auto contributors = [&](int band) {
        const int64_t lo = (int64_t)(band - args.dp_bands) * U, hi = lo + U;  // the band's units
        const int i_lo = (int)div_nn((lo + 1) * P - 1, args.sk_units), i_hi = (int)div_nn(hi * P - 1, args.sk_units);
        if (tid == 0) {
            int count = 0;
            for (int i = i_lo; i <= i_hi; ++i) {
                const int64_t st = sk_start(i);
                if (st == sk_start(i + 1)) continue;
                fix_list[count++] = (uint16_t)(i * 2 + (st < lo ? 1 : 0));
            }
            fix_count = count;
        }
        __syncthreads();
        return fix_count;
    };
    // The sum of a shared band over its contributors in workgroup order (so the result does not
    // depend on who sums it), then the epilogue. `own` >= 0: this workgroup's contribution is the
    // one in `fin` (entry `own` of the list), not yet in memory.
    auto sum_band = [&](int band, int count, int own) {
        f32x4 v[NW][FM];
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int f = 0; f < FM; ++f) v[w][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // Four contributors' partials are loaded before any is added (one memory round trip per
        // four, not per contributor); the sum still runs in contributor order.
        constexpr int kBatch = 4;
        for (int c0 = 0; c0 < count; c0 += kBatch) {
            f32x4 part[kBatch][NW][FM];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                // Past the list or this workgroup's own entry: a harmless read of entry 0's partial.
                int entry = c0 + j < count ? fix_list[c0 + j] : own;
                if (entry == own) entry = fix_list[0] == own ? fix_list[count > 1 ? 1 : 0] : fix_list[0];
#pragma unroll
                for (int w = 0; w < NW; ++w)
#pragma unroll
                    for (int f = 0; f < FM; ++f)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int m = own_row(f, i) < rows ? own_row(f, i) : rows - 1;
                            part[j][w][f][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                            p_rsrc, part_off(entry >> 1, entry & 1, w, m), 0, kDeviceCpol));
                        }
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                if (c0 + j >= count) break;
                const bool mine = fix_list[c0 + j] == own;
#pragma unroll
                for (int w = 0; w < NW; ++w)
#pragma unroll
                    for (int f = 0; f < FM; ++f) v[w][f] += mine ? fin[w][f] : part[j][w][f];
            }
        }
        store_out(band, v);
    };
    // Arrival counters, one per shared band, at the start of the workspace; the workgroup that
    // sums a band returns its counter to zero for the next call.
    auto counter = [&](int band) { return args.counters + (band - args.dp_bands); };

    auto nothing = [] {};
    for (int band = blockIdx.x; band < args.dp_bands; band += P) {
        run_job(band, 0, U, nothing);
        store_out(band, fin);
        lds_barrier();  // the next job's loads overwrite the reduction area; stores need not drain
    }
    if (args.sk_units > 0) {
        // A workgroup's range meets at most two bands partially: its first job (slot 0) and its
        // last (slot 1). The first job's partial is written at once and announced after the next
        // job's prologue (its stores have completed by then, and the wait for them hides behind
        // that prologue's loads); whether that made this workgroup the band's last contributor is
        // looked at when the range is done. The last job's band is summed at once if every other
        // contributor has already announced itself (the usual case: they did so long before),
        // from this workgroup's registers and their partials; otherwise this workgroup writes and
        // announces its partial too, and the last to arrive sums.
        int64_t u = sk_start(blockIdx.x);
        const int64_t u_end = sk_start(blockIdx.x + 1);
        int slot = 0, pending = -1, pending_old = -1, announce = -1;
        __shared__ int arrival;
        while (u < u_end) {
            const int64_t uq = div_nn(u, U);
            const int band = args.dp_bands + (int)uq;
            const int ga = (int)(u - uq * U);
            const int gb = (int)((int64_t)ga + (u_end - u) < U ? ga + (u_end - u) : U);
            const bool whole = ga == 0 && gb == U;
            const bool last_partial = !whole && u + (gb - ga) >= u_end;
            int count = 0, early = -1;
            run_job(band, ga, gb, [&] {
                if (announce >= 0 && tid == 0)
                    pending_old = __hip_atomic_fetch_add(counter(announce), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                announce = -1;  // once: later jobs of the range announce nothing
                // The last job's band: its contributors, and how many have announced so far (read
                // now, so that the round trip hides behind the job; once count - 1 have announced,
                // the count stays there until this workgroup sums).
                if (last_partial) {
                    count = contributors(band);
                    if (tid == 0) early = __hip_atomic_load(counter(band), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
            });
            u += gb - ga;
            if (whole) {
                store_out(band, fin);
            } else if (u < u_end) {
                write_partial(slot);
                pending = announce = band;
            } else {
                if (tid == 0)
                    arrival = early == count - 1 ? early
                                                 : __hip_atomic_load(counter(band), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                __syncthreads();
                if (arrival == count - 1) {
                    if (tid == 0) __hip_atomic_store(counter(band), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    sum_band(band, count, (int)blockIdx.x * 2 + slot);
                } else {
                    write_partial(slot);
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial is in memory
                    __syncthreads();
                    if (tid == 0) {
                        const int old = __hip_atomic_fetch_add(counter(band), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        if (old == count - 1) __hip_atomic_store(counter(band), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        arrival = old;
                    }
                    __syncthreads();
                    if (arrival == count - 1) sum_band(band, count, -1);
                }
            }
            lds_barrier();
            slot = 1;
        }
        if (pending >= 0) {
            if (tid == 0) arrival = pending_old;
            __syncthreads();
            const int count = contributors(pending);
            if (arrival == count - 1) {
                if (tid == 0) __hip_atomic_store(counter(pending), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                sum_band(pending, count, -1);
            }
        }
    }
}

constexpr int kMmaCW = 2, kMmaKW = 4;

constexpr int kMmaDepth = 3;  // weight ring depth (steps the weight loads run ahead)

// Activation and code offsets are 32-bit; 64 rows at most.
bool mma_fits(int64_t rows, int64_t columns, int64_t inner, int64_t stride_words, int64_t lda) {
    const int64_t limit = ((int64_t)1 << 32) - 256;  // byte extents of the buffer resources
    const int64_t groups = inner / kGroup;
    return rows >= 1 && rows <= 64 && columns > 0 && groups > 0 && (rows * lda + inner) * 2 < limit &&
           columns * stride_words * 4 < limit && columns * groups * 32 < limit;
}

// Q5_K: plane0 holds 16 bytes per 32 elements of a row, plane1 4, meta 16 per 256.
bool q5k_mma_fits(int64_t rows, int64_t columns, int64_t inner, int64_t lda) {
    const int64_t limit = ((int64_t)1 << 32) - 256;
    return rows >= 1 && rows <= 64 && columns > 0 && inner >= 256 && (rows * lda + inner) * 2 < limit &&
           columns * (inner / 32) * 16 < limit;
}

// Compute units of the current device (the stream-K grid), cached per device.
static int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cache[dev] = cus;
    }
    return cache[dev];
}

// Workspace: a fixed region of arrival counters (one per shared band, zero between calls) at the
// start, then the partials [grid][2][nw][rows][band columns] fp32. The counters sit at the same
// place for every shape, kernel variant and row count, so calls of different shapes can share one
// workspace: a call never writes partials where another call keeps counters.
constexpr size_t kCounterBytes = 16384;
constexpr int kMaxSkBands = (int)(kCounterBytes / sizeof(int));
static size_t sk_partial_bytes(int grid, int64_t rows, bool mlp) {
    return ((size_t)grid * 2 * (mlp ? 2 : 1) * rows * (kMmaCW * 32) * sizeof(float) + 255) / 256 * 256;
}
static size_t sk_bytes(int grid, int64_t rows, int, bool mlp) { return kCounterBytes + sk_partial_bytes(grid, rows, mlp); }

MmaPlan plan_mma(int64_t rows, int64_t columns, int64_t groups, bool mlp, size_t workspace_bytes, int64_t unit_elems) {
    MmaPlan p;
    p.fm = rows <= 32 ? 1 : 2;
    p.bands = (int)((columns + kMmaCW * 32 - 1) / (kMmaCW * 32));
    int grid = device_cus();
    // At least 1280 elements of K (five q4 steps) a workgroup: below that the fixed cost of a job
    // (pipeline fill, reduction, the shared band's fix-up) outweighs the extra CUs (measured on the
    // 5120 -> 1024 projection at M=64: 19 us on 256 workgroups, 12.4 us on 64).
    const int64_t min_units = (1280 + unit_elems - 1) / unit_elems;
    const int64_t want = ((int64_t)p.bands * groups + min_units - 1) / min_units;
    if (want < grid) grid = (int)(want > 0 ? want : 1);
    // A development override of the grid, read from the environment once per process.
    static const int grid_override = [] { const char *e = getenv("SPLOSH_MMA_GRID"); return e ? atoi(e) : 0; }();
    if (grid_override > 0) grid = grid_override;
    // At least two workgroups a band: the same number on every band, so that every workgroup's
    // range lies in one band -- one job, one pipeline fill, one reduction -- at the price of up
    // to bands - 1 idle CUs (K=17408 -> N=5120 at M=64: 240 workgroups, 31.5 -> 30.2 us; the
    // 5120 -> 5120 projections 23.4 -> 19.1 us).
    else if (p.bands < grid && grid / p.bands >= 2) grid = p.bands * (grid / p.bands);
    // Between three quarters of the CUs and all of them: one band a workgroup beats two jobs a
    // workgroup (5120 -> 12288 at M=64, 192 bands: 23.1 -> 19.9 us with 64 CUs idle).
    else if (p.bands < grid && 4 * p.bands >= 3 * grid) grid = p.bands;
    grid = grid < kMmaMaxGrid ? grid : kMmaMaxGrid;  // the fix-up's contributor list
    p.grid = grid;
    // Every band's units go into one stream, cut into `grid` equal contiguous ranges: a band is
    // shared by at most a few workgroups and no step is wasted on a partial round of bands.
    p.dp_bands = 0;
    p.sk_units = (int64_t)p.bands * groups;
    if (p.bands % grid == 0) {
        // Whole bands per workgroup already balance: no partials.
        p.dp_bands = p.bands;
        p.sk_units = 0;
    } else if (sk_bytes(grid, rows, p.bands, mlp) > workspace_bytes || p.bands > kMaxSkBands) {
        // No room for partials: every band whole, one workgroup each.
        p.grid = p.bands;
        p.dp_bands = p.bands;
        p.sk_units = 0;
    }
    return p;
}

size_t mma_workspace_bytes(int64_t rows, int64_t columns, int64_t groups, bool mlp) {
    const MmaPlan p = plan_mma(rows, columns, groups, mlp, (size_t)-1);
    return p.sk_units > 0 ? sk_bytes(p.grid, rows, p.bands, mlp) : 0;
}

template <class F, int FM>
static hipError_t launch_mma_v(const MmaPlan &p, const MmaArgs &args, hipStream_t stream) {
    using S = MmaShape<FM, F::NW, kMmaCW, kMmaKW, kMmaDepth, F::kSBuf, F::kTblBytes>;
    auto kernel = mma_kernel<F, FM, kMmaCW, kMmaKW, kMmaDepth>;
    static bool once = [&] {
        (void)hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLds);
        return true;
    }();
    (void)once;
    hipLaunchKernelGGL(kernel, dim3((unsigned)p.grid), dim3(S::kThreads), S::kLds, stream, args);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_mma_fm(const MmaPlan &p, const MmaArgs &args, hipStream_t stream) {
    return p.fm == 1 ? launch_mma_v<F, 1>(p, args, stream) : launch_mma_v<F, 2>(p, args, stream);
}

// EMIT: a build with the emit epilogue, kept apart so that its registers do not weigh on the
// kernel without it.
template <int NW, bool TILED, bool GROUPED = false, bool EMIT = false, bool SPLIT = false>
using Q4F = Q4Format<NW, TILED, kMmaCW, kMmaKW, kMmaDepth, GROUPED, EMIT, SPLIT>;

static void set_io(MmaArgs &args, const MmaPlan &plan, const uint16_t *a, int64_t lda, void *out, int64_t ldc,
                   int out_dtype, const void *residual, int64_t rows, int64_t inner, void *workspace, bool mlp) {
    args.a = a;
    args.lda = lda;
    args.out = out;
    args.ldc = ldc;
    args.residual = residual;
    args.rows = rows;
    args.out_dtype = out_dtype;
    args.counters = plan.sk_units > 0 ? (int *)workspace : nullptr;
    args.partial = plan.sk_units > 0 ? (float *)((char *)workspace + kCounterBytes) : nullptr;
    args.partial_bytes = plan.sk_units > 0 ? (uint32_t)sk_partial_bytes(plan.grid, rows, mlp) : 0;
    args.dp_bands = plan.dp_bands;
    args.sk_units = plan.sk_units;
    args.a_bytes = (uint32_t)(((rows - 1) * lda + inner) * 2);
}

hipError_t launch_q4_mma(const MmaPlan &plan, const splosh_q4_weight &w, const splosh_q4_weight *up,
                         const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                         int64_t rows, void *workspace, hipStream_t stream, const EmitOperand *emit) {
    MmaArgs args = {};
    if (emit) {
        args.norm_weight = emit->norm_weight;
        args.values = emit->values;
        args.ldv = emit->ldv;
        args.sums = emit->sums;
        args.squares = emit->squares;
    }
    args.packed[0] = w.packed;
    args.scales[0] = w.scales;
    args.biases[0] = w.biases;
    args.packed[1] = up ? up->packed : w.packed;
    args.scales[1] = up ? up->scales : w.scales;
    args.biases[1] = up ? up->biases : w.biases;
    args.stride_words = w.row_stride_words;
    args.n = w.rows;
    const int64_t groups = w.inner / kGroup;
    args.units = groups;
    set_io(args, plan, a, lda, out, ldc, out_dtype, residual, rows, w.inner, workspace, up != nullptr);
    const bool tiled = w.order == SPLOSH_Q4_TILED128;
    args.code_bytes = (uint32_t)(tiled ? w.rows * groups * 32 : w.rows * w.row_stride_words * 4);
    args.sidecar_bytes = (uint32_t)(w.rows * groups * 2);
    hipError_t err;
    if (up)
        err = tiled ? launch_mma_fm<Q4F<2, true>>(plan, args, stream) : launch_mma_fm<Q4F<2, false>>(plan, args, stream);
    else if (emit)
        err = tiled ? launch_mma_fm<Q4F<1, true, false, true>>(plan, args, stream)
                    : launch_mma_fm<Q4F<1, false, false, true>>(plan, args, stream);
    else
        err = tiled ? launch_mma_fm<Q4F<1, true>>(plan, args, stream) : launch_mma_fm<Q4F<1, false>>(plan, args, stream);
    return err;
}

// A wide single weight runs as the pair of its column halves (Q4Format SPLIT): from two bands a
// CU, so that every workgroup has at least two jobs and halving them saves their fixed cost.
// Measured at M=64 (M=16): K5120 N=248320 285 -> 242 us (226 -> 196), N=65536 75 -> 67 (61 ->
// 55), N=34816 50 -> 47 (42 -> 40), K17408 N=34816 124 -> 115 (101 -> 90), K2048 N=131072 73 -> 63;
// N=49152 (three jobs a CU) within the spread. Below two bands a CU (N=17408) the pair's longer
// step costs more than the job it saves. The halves start on a 128-row tile (tiled) or a row.
bool mma_split(const splosh_q4_weight &w) {
    const int64_t bands = (w.rows + kMmaCW * 32 - 1) / (kMmaCW * 32);
    const bool halves = w.order == SPLOSH_Q4_TILED128 ? w.rows % 256 == 0 : w.rows % 2 == 0;
    return halves && bands >= 2 * (int64_t)device_cus();
}

hipError_t launch_q4_mma_split(const MmaPlan &plan, const splosh_q4_weight &w, const uint16_t *a, int64_t lda,
                               void *out, int64_t ldc, int out_dtype, const void *residual, int64_t rows,
                               void *workspace, hipStream_t stream) {
    MmaArgs args = {};
    const int64_t half = w.rows / 2, groups = w.inner / kGroup;
    const bool tiled = w.order == SPLOSH_Q4_TILED128;
    // Row `half`'s first record: tiled, (half / 128) G 128 records of 8 words; row-major, half rows.
    const int64_t rec = tiled ? half / 128 * groups * 128 : half * groups;
    const int64_t words = tiled ? rec * 8 : half * w.row_stride_words;
    args.packed[0] = w.packed;
    args.scales[0] = w.scales;
    args.biases[0] = w.biases;
    args.packed[1] = w.packed + words;
    args.scales[1] = w.scales + rec;
    args.biases[1] = w.biases + rec;
    args.stride_words = w.row_stride_words;
    args.n = half;
    args.units = groups;
    set_io(args, plan, a, lda, out, ldc, out_dtype, residual, rows, w.inner, workspace, true);
    args.code_bytes = (uint32_t)(tiled ? half * groups * 32 : half * w.row_stride_words * 4);
    args.sidecar_bytes = (uint32_t)(half * groups * 2);
    return tiled ? launch_mma_fm<Q4F<2, true, false, false, true>>(plan, args, stream)
                 : launch_mma_fm<Q4F<2, false, false, false, true>>(plan, args, stream);
}

// Several tiled weights of one inner size on one activation (the reference's concurrent encoder of
// independent projections, Engine.swift:1402): their bands form one band space, split as one call.
hipError_t launch_q4_mma_group(const MmaPlan &plan, const splosh_q4_weight *w, int count, void *const *outs,
                               const int64_t *ldcs, const uint16_t *a, int64_t lda, int out_dtype, int64_t rows,
                               void *workspace, hipStream_t stream) {
    MmaArgs args = {};
    const int64_t groups = w[0].inner / kGroup;
    args.units = groups;
    args.ngroup = count;
    int band = 0;
    for (int i = 0; i < count; ++i) {
        args.gband[i] = band;
        args.gpacked[i] = w[i].packed;
        args.gscales[i] = w[i].scales;
        args.gbiases[i] = w[i].biases;
        args.gout[i] = outs[i];
        args.gn[i] = w[i].rows;
        args.gldc[i] = ldcs[i];
        band += (int)(w[i].rows / (kMmaCW * 32));
    }
    args.gband[count] = band;
    // The first weight's pointers stand in for the single-weight fields (never read for codes).
    args.packed[0] = args.packed[1] = w[0].packed;
    args.scales[0] = args.scales[1] = w[0].scales;
    args.biases[0] = args.biases[1] = w[0].biases;
    args.n = w[0].rows;
    args.stride_words = w[0].row_stride_words;
    set_io(args, plan, a, lda, outs[0], ldcs[0], out_dtype, nullptr, rows, w[0].inner, workspace, false);
    args.code_bytes = (uint32_t)(w[0].rows * groups * 32);
    args.sidecar_bytes = (uint32_t)(w[0].rows * groups * 2);
    return launch_mma_fm<Q4F<1, true, true>>(plan, args, stream);
}

hipError_t launch_q5k_mma(const MmaPlan &plan, const splosh_q5k_weight &w, const uint16_t *a, int64_t lda, void *out,
                          int64_t ldc, int out_dtype, const void *residual, int64_t rows, void *workspace,
                          hipStream_t stream) {
    MmaArgs args = {};
    args.plane0 = w.plane0;
    args.plane1 = w.plane1;
    args.meta = w.meta;
    args.n = w.rows;
    const int64_t blocks = w.inner / 256;
    args.units = blocks;
    set_io(args, plan, a, lda, out, ldc, out_dtype, residual, rows, w.inner, workspace, false);
    args.code_bytes = (uint32_t)(w.rows * blocks * 8 * 16);
    args.sidecar_bytes = (uint32_t)(w.rows * blocks * 8 * 4);
    args.meta_bytes = (uint32_t)(w.rows * blocks * 16);
    if (!w.plane1) return launch_mma_fm<Q5Format<kMmaCW, kMmaKW, kMmaDepth, false>>(plan, args, stream);  // Q4_K
    return launch_mma_fm<Q5Format<kMmaCW, kMmaKW, kMmaDepth>>(plan, args, stream);
}

bool gguf_mma_fits(int type, int64_t rows, int64_t columns, int64_t inner, int64_t lda) {
    int elems = 0, bytes = 0;
    if (!gguf_native_block(type, &elems, &bytes)) return false;
    const int64_t limit = ((int64_t)1 << 32) - 256;
    return rows >= 1 && rows <= 64 && columns > 0 && inner >= 256 && inner % 256 == 0 &&
           (rows * lda + inner) * 2 < limit && (columns + 31) * (inner / elems) * bytes < limit;
}

hipError_t launch_gguf_mma(const MmaPlan &plan, int type, const uint8_t *native, int64_t columns, int64_t inner,
                           const uint16_t *a, int64_t lda, void *out, int64_t ldc, int out_dtype, const void *residual,
                           int64_t rows, void *workspace, hipStream_t stream) {
    int elems = 0, bytes = 0;
    gguf_native_block(type, &elems, &bytes);
    MmaArgs args = {};
    args.rows32 = gguf_layout(type);
    args.plane0 = native;
    args.n = columns;
    args.units = inner / 256;
    set_io(args, plan, a, lda, out, ldc, out_dtype, residual, rows, inner, workspace, false);
    args.row_bytes = (uint32_t)(inner / elems * bytes);
    args.code_bytes = (uint32_t)((args.rows32 ? (columns + 31) / 32 * 32 : columns) * args.row_bytes);
    switch (type) {
        case 8: return launch_mma_fm<GgufFormat<8, kMmaCW, kMmaKW, kMmaDepth>>(plan, args, stream);
        case 20: return launch_mma_fm<GgufFormat<20, kMmaCW, kMmaKW, kMmaDepth>>(plan, args, stream);
        case 14: return launch_mma_fm<GgufFormat<14, kMmaCW, kMmaKW, kMmaDepth>>(plan, args, stream);
        case 11: return launch_mma_fm<GgufFormat<11, kMmaCW, kMmaKW, kMmaDepth>>(plan, args, stream);
        case 21: return launch_mma_fm<GgufFormat<21, kMmaCW, kMmaKW, kMmaDepth>>(plan, args, stream);
        default: return launch_mma_fm<GgufFormat<23, kMmaCW, kMmaKW, kMmaDepth>>(plan, args, stream);
    }
}

}  // namespace splosh
