// gguf_decode.hpp -- device decoders of the GGUF formats kept in native blocks (Q8_0, Q3_K, Q6_K,
// IQ4_NL, IQ3_S, IQ4_XS) and of Q5_K / Q4_K groups in plane form: one 32-element group at a
// time, in the reference decoder's fp32 operation order (GgufQuant.swift), so every value is
// bit-identical to GgufTensorType.decode. Shared by the dequant, GEMV, embedding and tile kernels.
#pragma once

#include "common.hpp"

namespace splosh {

// IQ4_NL / IQ4_XS code values (llama.cpp's kvalues_iq4nl, the format's table: -127, -104, -83,
// -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113) as int8 bytes, four to a dword.
constexpr uint32_t kIq4Tab0 = 0xBFAD9881u, kIq4Tab1 = 0xF6EADDCFu, kIq4Tab2 = 0x26190D01u, kIq4Tab3 = 0x71594535u;

// Table values (int8) of the four 4-bit codes in the bytes of `idx`: entries 0..7 and 8..15 by two
// byte permutes, then per byte the half that bit 3 of the code picks.
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t idx) {
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = perm_bytes(kIq4Tab1, kIq4Tab0, sel), hi = perm_bytes(kIq4Tab3, kIq4Tab2, sel);
    const uint32_t mask = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (hi & mask) | (lo & ~mask);
}

template <int TYPE>
struct GgufGeom;
template <> struct GgufGeom<8> { static constexpr int kElems = 32, kBytes = 34; };    // Q8_0
template <> struct GgufGeom<20> { static constexpr int kElems = 32, kBytes = 18; };   // IQ4_NL
template <> struct GgufGeom<14> { static constexpr int kElems = 256, kBytes = 210; }; // Q6_K
template <> struct GgufGeom<23> { static constexpr int kElems = 256, kBytes = 136; }; // IQ4_XS
template <> struct GgufGeom<11> { static constexpr int kElems = 256, kBytes = 110; }; // Q3_K
template <> struct GgufGeom<21> { static constexpr int kElems = 256, kBytes = 110; }; // IQ3_S

// Bytes of 256 elements of a row (one super-block, or eight 32-element blocks): the unit of the
// ROWS32 layout.
template <int TYPE>
constexpr uint32_t gguf_unit_bytes() { return 256 / GgufGeom<TYPE>::kElems * GgufGeom<TYPE>::kBytes; }

// Where row n's 256-element units lie: unit u at base + u ustride.
//  * NATIVE (the file's order, rows back to back): base n row_bytes, ustride one unit.
//  * ROWS32 (inner % 256 == 0, rows padded to a multiple of 32): the units of 32 consecutive rows
//    interleaved -- unit u of row n at ((n / 32) units 32 + u 32 + n % 32) unit bytes -- so the 32
//    lanes that read one unit of 32 rows each read one contiguous run.
struct GgufRow {
    uint32_t base, ustride;
};
template <int TYPE>
__device__ __forceinline__ GgufRow gguf_row(uint32_t n, uint32_t row_bytes, bool rows32) {
    constexpr uint32_t UB = gguf_unit_bytes<TYPE>();
    if (rows32) return GgufRow{((n >> 5) * (row_bytes / UB) * 32u + (n & 31u)) * UB, 32u * UB};
    return GgufRow{n * row_bytes, UB};
}

// The IQ3_S codebook (the format's table, llama.cpp's iq3s_grid, kept by the reference as
// GgufTensorType.iq3sGrid, GgufQuant.swift:60): entry i holds four magnitudes, each 1..15 and odd,
// stored as twelve bits: magnitude t = 2 ((code >> 3t) & 7) + 1.
__constant__ uint16_t kIq3sPacked[512] = {
    0x000, 0x001, 0x002, 0x005, 0x007, 0x008, 0x009, 0x00a, 0x00c, 0x00e, 0x010, 0x011, 0x015, 0x01b, 0x020, 0x022,
    0x025, 0x027, 0x029, 0x02b, 0x030, 0x032, 0x039, 0x03c, 0x03f, 0x040, 0x041, 0x042, 0x044, 0x048, 0x049, 0x04d,
    0x050, 0x053, 0x057, 0x059, 0x05d, 0x064, 0x071, 0x075, 0x07a, 0x080, 0x081, 0x085, 0x087, 0x088, 0x08b, 0x08e,
    0x091, 0x095, 0x098, 0x09c, 0x0a2, 0x0a5, 0x0a7, 0x0a9, 0x0ab, 0x0b8, 0x0bb, 0x0c3, 0x0c9, 0x0cd, 0x0d0, 0x0d2,
    0x0d9, 0x0db, 0x0de, 0x0e4, 0x0e8, 0x0ea, 0x0f7, 0x0f9, 0x0fd, 0x100, 0x10b, 0x10f, 0x111, 0x114, 0x11a, 0x120,
    0x123, 0x129, 0x138, 0x142, 0x144, 0x150, 0x152, 0x156, 0x15b, 0x161, 0x165, 0x167, 0x176, 0x17b, 0x186, 0x189,
    0x18b, 0x199, 0x1aa, 0x1b9, 0x1c0, 0x1c2, 0x1c4, 0x1d0, 0x1d2, 0x1d6, 0x1db, 0x1e8, 0x1ec, 0x200, 0x201, 0x202,
    0x204, 0x208, 0x209, 0x20b, 0x20d, 0x20f, 0x210, 0x212, 0x219, 0x21c, 0x21e, 0x22c, 0x22e, 0x231, 0x23a, 0x240,
    0x241, 0x243, 0x246, 0x248, 0x24c, 0x251, 0x258, 0x25b, 0x261, 0x268, 0x26a, 0x278, 0x27e, 0x280, 0x28a, 0x28d,
    0x28f, 0x290, 0x294, 0x29a, 0x2a0, 0x2a3, 0x2ad, 0x2b0, 0x2ba, 0x2c1, 0x2c4, 0x2c7, 0x2c8, 0x2cb, 0x2d1, 0x2d7,
    0x2d8, 0x2dc, 0x2e1, 0x2f2, 0x2f8, 0x303, 0x305, 0x30a, 0x30c, 0x319, 0x31b, 0x322, 0x326, 0x328, 0x32c, 0x341,
    0x348, 0x34b, 0x351, 0x358, 0x35a, 0x369, 0x390, 0x394, 0x397, 0x3a4, 0x3a6, 0x3c1, 0x3c3, 0x3c8, 0x3ca, 0x3d1,
    0x3dd, 0x3e1, 0x3f2, 0x3f8, 0x400, 0x401, 0x403, 0x405, 0x407, 0x408, 0x40a, 0x40c, 0x40e, 0x411, 0x413, 0x417,
    0x418, 0x41a, 0x421, 0x423, 0x425, 0x428, 0x42a, 0x437, 0x438, 0x43b, 0x43d, 0x440, 0x442, 0x448, 0x44b, 0x44f,
    0x452, 0x455, 0x459, 0x45c, 0x462, 0x469, 0x481, 0x484, 0x487, 0x491, 0x493, 0x498, 0x49f, 0x4a1, 0x4ab, 0x4af,
    0x4b9, 0x4bc, 0x4c0, 0x4c2, 0x4c5, 0x4c9, 0x4d2, 0x4d4, 0x4d9, 0x4db, 0x4e2, 0x4e8, 0x4f6, 0x501, 0x507, 0x510,
    0x513, 0x51a, 0x51d, 0x521, 0x53a, 0x53d, 0x544, 0x549, 0x552, 0x55f, 0x560, 0x56b, 0x578, 0x580, 0x582, 0x587,
    0x591, 0x5ad, 0x5b1, 0x5c5, 0x5c9, 0x5d6, 0x5d8, 0x5e3, 0x5e8, 0x602, 0x609, 0x60b, 0x60d, 0x60f, 0x612, 0x619,
    0x61b, 0x61d, 0x622, 0x624, 0x627, 0x629, 0x633, 0x639, 0x641, 0x643, 0x645, 0x64c, 0x651, 0x653, 0x660, 0x670,
    0x67a, 0x67e, 0x680, 0x68a, 0x690, 0x69a, 0x69c, 0x6a8, 0x6c1, 0x6c8, 0x6cc, 0x6d1, 0x6d3, 0x6d7, 0x6d8, 0x6e1,
    0x6e3, 0x6e7, 0x6ed, 0x6fb, 0x703, 0x709, 0x70e, 0x712, 0x719, 0x72a, 0x730, 0x734, 0x741, 0x748, 0x74a, 0x755,
    0x75a, 0x764, 0x76e, 0x77b, 0x78e, 0x7a1, 0x7c1, 0x7c3, 0x7d0, 0x7d2, 0x7dd, 0x800, 0x804, 0x80a, 0x810, 0x814,
    0x817, 0x81a, 0x821, 0x828, 0x838, 0x842, 0x847, 0x849, 0x84b, 0x852, 0x858, 0x85d, 0x863, 0x869, 0x86d, 0x881,
    0x883, 0x888, 0x88d, 0x891, 0x89b, 0x8a0, 0x8af, 0x8b2, 0x8b8, 0x8c4, 0x8c9, 0x8cb, 0x8d0, 0x8d2, 0x8d9, 0x8dd,
    0x900, 0x902, 0x914, 0x91f, 0x920, 0x939, 0x945, 0x947, 0x951, 0x972, 0x98b, 0x99c, 0x9b0, 0x9c8, 0x9cd, 0x9d8,
    0x9e3, 0x9e9, 0xa02, 0xa08, 0xa0c, 0xa12, 0xa20, 0xa24, 0xa27, 0xa2a, 0xa36, 0xa3c, 0xa41, 0xa43, 0xa45, 0xa4a,
    0xa51, 0xa5a, 0xa7a, 0xa80, 0xa89, 0xa93, 0xa98, 0xa9e, 0xaab, 0xac2, 0xac7, 0xac8, 0xad7, 0xae4, 0xae9, 0xaf5,
    0xafb, 0xb01, 0xb04, 0xb10, 0xb1a, 0xb26, 0xb4a, 0xb56, 0xb69, 0xb6b, 0xba2, 0xbc2, 0xbc4, 0xbd2, 0xc09, 0xc0b,
    0xc0d, 0xc19, 0xc1b, 0xc30, 0xc40, 0xc50, 0xc57, 0xc74, 0xc8a, 0xc9c, 0xca2, 0xcad, 0xcb2, 0xcb8, 0xcc0, 0xccc,
    0xcd1, 0xce0, 0xd15, 0xd23, 0xd32, 0xd40, 0xd43, 0xd5c, 0xd70, 0xd85, 0xda0, 0xdc9, 0xdcb, 0xe00, 0xe04, 0xe07,
    0xe10, 0xe12, 0xe1e, 0xe20, 0xe2c, 0xe32, 0xe42, 0xe49, 0xe54, 0xe63, 0xe65, 0xe81, 0xe84, 0xe88, 0xe8e, 0xe91,
    0xe98, 0xea9, 0xec2, 0xeda, 0xedd, 0xeeb, 0xf01, 0xf05, 0xf0b, 0xf10, 0xf28, 0xf52, 0xf62, 0xf82, 0xf99, 0xfc0,
};

__device__ __forceinline__ uint32_t ld16(rsrc_t r, uint32_t off) { return buffer_load_u16(r, off, 0); }

// W dwords of bytes starting at a 2-aligned `off` (all 4 W of them inside the weight), fetched as
// the dword-aligned window that covers them (W + 1 dwords, the first in 16-byte pieces; buffer
// loads need only dword alignment) and, at decode, shifted into place by the 0- or 2-byte
// misalignment (v_alignbyte_b32). Every byte read lies in the weight.
template <int W>
struct Span {
    uint32_t win[W + 1];
    uint32_t sh;
};
template <int W>
__device__ __forceinline__ Span<W> fetch_span(rsrc_t r, uint32_t off) {
    Span<W> s;
    const uint32_t a0 = off & ~3u;
    s.sh = off & 3u;
#pragma unroll
    for (int q = 0; q < (W + 1) / 4; ++q) {
        const u32x4 x = buffer_load16(r, a0 + 16u * q, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) s.win[4 * q + e] = x[e];
    }
#pragma unroll
    for (int e = (W + 1) / 4 * 4; e < W; ++e) s.win[e] = buffer_load_u32(r, a0 + 4u * e, 0);
    // Only the low half of the last window dword is ever used (when off is 2 mod 4), and its high
    // half may lie past the weight, where a dword load would read zero for the whole dword.
    s.win[W] = buffer_load_u16(r, a0 + 4u * W, 0);
    return s;
}
template <int W>
__device__ __forceinline__ void align_span(const Span<W> &s, uint32_t (&out)[W]) {
#pragma unroll
    for (int i = 0; i < W; ++i) out[i] = __builtin_amdgcn_alignbyte(s.win[i + 1], s.win[i], s.sh);
}
template <int W>
__device__ __forceinline__ uint32_t byte_of(const uint32_t (&w)[W], int e) { return (w[e >> 2] >> (8 * (e & 3))) & 0xFF; }

// Each native format's group decoder in two halves: gguf_fetch issues every load of group g of a
// row (where its units lie: gguf_row) and returns the raw bytes (GgufRaw<TYPE>); gguf_decode turns
// them into the 32 values with no memory access, so that a kernel can fetch one step ahead.
// Values follow GgufQuant.swift's decode in its fp32 operation order.
template <int TYPE>
struct GgufRaw;

template <>
struct GgufRaw<8> {  // Q8_0 (GgufQuant.swift:172-175): d, 32 int8 codes
    uint32_t d;
    Span<8> codes;
};
template <>
struct GgufRaw<20> {  // IQ4_NL (:179-185): d, 16 bytes of two 4-bit codes
    uint32_t d;
    Span<4> codes;
};
template <>
struct GgufRaw<14> {  // Q6_K (:218-230): ql[128], qh[64], scales[16], d
    uint32_t d, sc;
    Span<8> ql, qh;
    int j;
};
template <>
struct GgufRaw<11> {  // Q3_K (:238-256): hmask[32], qs[64], scales[12], d
    uint32_t d, lows, highs;
    Span<8> hm, qs;
    int j;
};
template <>
struct GgufRaw<21> {  // IQ3_S (:283-300): d, qs[64], qh[8], signs[32], scales[4]
    uint32_t d, scale, ninth;
    Span<2> cb;
    Span<1> sg;
    int j;
};
template <>
struct GgufRaw<23> {  // IQ4_XS (:261-275): d, scales_h, scales_l[4], qs[128]
    uint32_t d, high, lowb;
    u32x4 q;
    int j;
};

template <int TYPE>
__device__ __forceinline__ GgufRaw<TYPE> gguf_fetch(rsrc_t r, GgufRow row_, int g) {
    GgufRaw<TYPE> w;
    // The group's unit (8 groups of 32), then its block within the unit for 32-element blocks.
    const uint32_t row = row_.base + (uint32_t)(g >> 3) * row_.ustride;
    if constexpr (TYPE == 8) {
        const uint32_t b = row + (uint32_t)(g & 7) * 34u;
        w.d = ld16(r, b);
        w.codes = fetch_span<8>(r, b + 2);
    } else if constexpr (TYPE == 20) {
        const uint32_t b = row + (uint32_t)(g & 7) * 18u;
        w.d = ld16(r, b);
        w.codes = fetch_span<4>(r, b + 2);
    } else if constexpr (TYPE == 14) {
        const int j = g & 7, half = j >> 2, quarter = j & 3;
        const uint32_t b = row;
        w.j = j;
        w.d = ld16(r, b + 208);
        w.sc = ld16(r, b + 192 + 2 * j);
        w.ql = fetch_span<8>(r, b + 64 * half + 32 * (quarter & 1));
        w.qh = fetch_span<8>(r, b + 128 + 32 * half);
    } else if constexpr (TYPE == 11) {
        const int j = g & 7, half = j >> 2, word = j >> 1;
        const uint32_t b = row;
        w.j = j;
        w.d = ld16(r, b + 108);
        // Scales 2 j and 2 j + 1: bytes 2 (j % 2), 2 (j % 2) + 1 of word j / 2 % 2 (their low or
        // high nibbles) and of the third word (bits 2 (j / 2)).
        w.lows = ld16(r, b + 96 + 4 * (word & 1) + 2 * (j & 1));
        w.highs = ld16(r, b + 104 + 2 * (j & 1));
        w.hm = fetch_span<8>(r, b);
        w.qs = fetch_span<8>(r, b + 32 + 32 * half);
    } else if constexpr (TYPE == 21) {
        const int j = g & 7;
        const uint32_t b = row;
        w.j = j;
        w.d = ld16(r, b);
        w.scale = ld16(r, b + 106 + 2 * (j >> 2));
        w.ninth = ld16(r, b + 66 + (j & ~1));
        w.cb = fetch_span<2>(r, b + 2 + 8 * j);
        w.sg = fetch_span<1>(r, b + 74 + 4 * j);
    } else {
        const int j = g & 7;
        const uint32_t b = row;
        w.j = j;
        w.d = ld16(r, b);
        w.high = ld16(r, b + 2);
        w.lowb = ld16(r, b + 4 + 2 * (j >> 2));  // bytes 4 + 2 (j / 4) .. + 1
        w.q = buffer_load16(r, b + 8 + 16 * j, 0);  // blocks of 136 bytes: 8-aligned runs
    }
    return w;
}

template <int TYPE>
__device__ __forceinline__ void gguf_decode(const GgufRaw<TYPE> &w, float (&v)[32]) {
    if constexpr (TYPE == 8) {
        const float d = half_bits_to_f32(w.d);
        uint32_t h[8];
        align_span(w.codes, h);
#pragma unroll
        for (int e = 0; e < 32; ++e) v[e] = d * (float)(int8_t)byte_of(h, e);
    } else if constexpr (TYPE == 20) {
        const float d = half_bits_to_f32(w.d);
        uint32_t h[4];
        align_span(w.codes, h);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t lo = iq4_lookup4(h[q] & 0x0F0F0F0Fu), hi = iq4_lookup4((h[q] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[4 * q + e] = d * (float)(int8_t)((lo >> (8 * e)) & 0xFF);
                v[16 + 4 * q + e] = d * (float)(int8_t)((hi >> (8 * e)) & 0xFF);
            }
        }
    } else if constexpr (TYPE == 14) {
        const int quarter = w.j & 3;
        const float d = half_bits_to_f32(w.d);
        const float ds0 = d * (float)(int8_t)(w.sc & 0xFF), ds1 = d * (float)(int8_t)(w.sc >> 8);
        uint32_t ql[8], qh[8];
        align_span(w.ql, ql);
        align_span(w.qh, qh);
        const int lsh = 4 * (quarter >> 1), hsh = 2 * quarter;
        // Four codes a word: the 6-bit (low | high << 4) of each byte, then ds (code - 32) in the
        // reference's order (the subtraction is exact).
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t codes = ((ql[q] >> lsh) & 0x0F0F0F0Fu) | (((qh[q] >> hsh) & 0x03030303u) << 4);
            const float ds = q < 4 ? ds0 : ds1;
#pragma unroll
            for (int t = 0; t < 4; ++t) v[4 * q + t] = ds * (cvt_byte(codes, t) - 32.0f);
        }
    } else if constexpr (TYPE == 11) {
        const int j = w.j, shift = 2 * (j & 3), word = j >> 1;
        const float d = half_bits_to_f32(w.d);
        const uint32_t lows = w.lows >> (4 * (word >> 1)), highs = w.highs >> (2 * word);
        const float s0 = (float)((lows & 0xF) | ((highs & 3) << 4)) - 32.0f;
        const float s1 = (float)(((lows >> 8) & 0xF) | (((highs >> 8) & 3) << 4)) - 32.0f;
        const float ds0 = d * s0, ds1 = d * s1;
        uint32_t hm[8], qs[8];
        align_span(w.hm, hm);
        align_span(w.qs, qs);
        // Four codes a word, then ds (code - 4) in the reference's order.
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t codes = ((qs[q] >> shift) & 0x03030303u) | (((hm[q] >> j) & 0x01010101u) << 2);
            const float ds = q < 4 ? ds0 : ds1;
#pragma unroll
            for (int t = 0; t < 4; ++t) v[4 * q + t] = ds * (cvt_byte(codes, t) - 4.0f);
        }
    } else if constexpr (TYPE == 21) {
        const int j = w.j;
        const float d = half_bits_to_f32(w.d);
        const uint32_t scale = (w.scale >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
        const float weight = d * (1.0f + 2.0f * (float)scale);
        const uint32_t ninth = (w.ninth >> (8 * (j & 1))) & 0xFF;
        uint32_t cb[2], sg[1];
        align_span(w.cb, cb);
        align_span(w.sg, sg);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t code = ((cb[k >> 2] >> (8 * (k & 3))) & 0xFF) | (((ninth >> k) & 1) << 8);
            const uint32_t packed = kIq3sPacked[code];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int e = 4 * k + t;
                const float magnitude = (float)(2u * ((packed >> (3 * t)) & 7u) + 1u);
                const float sign = 1.0f - 2.0f * (float)((sg[0] >> e) & 1u);
                v[e] = (weight * magnitude) * sign;
            }
        }
    } else {
        const int j = w.j;
        const float d = half_bits_to_f32(w.d);
        const uint32_t low = (w.lowb >> (8 * ((j >> 1) & 1) + 4 * (j & 1))) & 15;
        const uint32_t scale = low | (((w.high >> (2 * j)) & 3) << 4);
        const float scaled = d * ((float)scale - 32.0f);
        const uint32_t qs[4] = {w.q[0], w.q[1], w.q[2], w.q[3]};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = iq4_lookup4(qs[k] & 0x0F0F0F0Fu), hi = iq4_lookup4((qs[k] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[4 * k + e] = scaled * (float)(int8_t)((lo >> (8 * e)) & 0xFF);
                v[16 + 4 * k + e] = scaled * (float)(int8_t)((hi >> (8 * e)) & 0xFF);
            }
        }
    }
}

// Group g of a row (gguf_row): fetch and decode at once.
template <int TYPE>
__device__ __forceinline__ void decode_group(rsrc_t r, GgufRow row, int g, float (&v)[32]) {
    gguf_decode<TYPE>(gguf_fetch<TYPE>(r, row, g), v);
}


// Group g of row `row` of a Q5_K / Q4_K weight in plane form (GgufPlanes.swift:62-74; plane1 null:
// Q4_K), as decodeQ45K computes it (GgufQuant.swift:191-212): code (low nibble, fifth bit) times
// d sc, less dmin mn.
__device__ __forceinline__ int plane_slot(int e) { return 8 * ((e >> 2) & 3) + 4 * (e >> 4) + (e & 3); }
struct PlaneRaw {
    u32x4 words, m;  // the group's 16 bytes of low nibbles; its block's 16 bytes of meta
    uint32_t bits;   // the group's 32 fifth bits (0 for Q4_K)
    int j;           // the group within its block
};
__device__ __forceinline__ PlaneRaw fetch_plane_group(const uint8_t *plane0, const uint8_t *plane1,
                                                      const uint8_t *meta, int64_t inner, int64_t row, int64_t g) {
    PlaneRaw w;
    const int64_t groups = inner / 32, blocks = inner / 256;
    const int64_t rec = ((row >> 7) * groups + g) * 128 + (row & 127);
    w.words = *(const u32x4 *)(plane0 + rec * 16);
    w.bits = plane1 ? *(const uint32_t *)(plane1 + rec * 4) : 0u;
    const int64_t mrec = ((row >> 7) * blocks + g / 8) * 128 + (row & 127);
    w.m = *(const u32x4 *)(meta + mrec * 16);
    w.j = (int)(g % 8);
    return w;
}
__device__ __forceinline__ void decode_plane(const PlaneRaw &w, float (&v)[32]) {
    const int j = w.j;
    const float d = half_bits_to_f32(w.m[0]), dmin = half_bits_to_f32(w.m[0] >> 16);
    // Packed 6-bit scale and minimum of group j (bytes 4..15 of the block = m[1..3]).
    auto pk = [&](int k) { return (w.m[1 + (k >> 2)] >> (8 * (k & 3))) & 0xFFu; };
    uint32_t sc, mn;
    if (j < 4) {
        sc = pk(j) & 63u;
        mn = pk(j + 4) & 63u;
    } else {
        sc = (pk(j + 4) & 0xFu) | ((pk(j - 4) >> 6) << 4);
        mn = (pk(j + 4) >> 4) | ((pk(j) >> 6) << 4);
    }
    const float scaled = d * (float)sc, offset = dmin * (float)mn;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const int slot = plane_slot(e), i = slot & 7;
        const uint32_t code =
            ((w.words[slot >> 3] >> ((i & 1) * 16 + 4 * (i >> 1))) & 15u) | (((w.bits >> slot) & 1u) << 4);
        const float p = (float)code * scaled;
        v[e] = p - offset;
    }
}
__device__ __forceinline__ void decode_plane_group(const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta,
                                                   int64_t inner, int64_t row, int64_t g, float (&v)[32]) {
    decode_plane(fetch_plane_group(plane0, plane1, meta, inner, row, g), v);
}

}  // namespace splosh
