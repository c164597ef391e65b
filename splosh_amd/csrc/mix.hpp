// mix.hpp -- q4 dequantization to bf16 MFMA operands with binary16 magic numbers and
// v_fma_mix_f32 (shared by the M <= 64 and the prefill kernels).
#pragma once

#include "common.hpp"

namespace splosh {

// fma(x, s, b) with x the binary16 number in the low (HI = false) or high half of `h`, widened
// exactly: v_fma_mix_f32, one instruction and one rounding.
template <bool HI>
__device__ __forceinline__ float fma_mix(uint32_t h, float s, float b) {
    float r;
    if (HI)
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(s), "v"(b));
    else
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(s), "v"(b));
    return r;
}

// Coefficients for dequant_word_mix from a group's scale s and bias b: nibbles become the
// binary16 numbers 1024 + q (bits 0..3 of a half) or 1024 + 16 q (bits 4..7), so
// s q + b = fma(1024 + q, s, b - 1024 s) = fma(1024 + 16 q, s / 16, b - 64 s). s / 16 is exact and
// so is b - 1024 s whenever the exponents of b and 1024 s are less than 16 apart (any practical
// affine group); then the result is the one-rounding fp32 s q + b exactly.
struct MixCoef {
    float s, b0, s16, b1;
};
__device__ __forceinline__ MixCoef mix_coef(float s, float b) {
    return MixCoef{s, __builtin_fmaf(-1024.0f, s, b), s * 0.0625f, __builtin_fmaf(-64.0f, s, b)};
}

// (x & mask) | magic in one v_and_or_b32 (the compiler splits it into two VOP2s, since a VOP3 takes no
// literal here): the mask comes from an SGPR, the magic from a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(magic));
    return r;
}

// Eight weights of one q4 code word (nibble k at bits 4k) as bf16 RNE(s q + b) in k order, 17 VALU:
// four AND-ORs and a shift build the binary16 pairs (q0, q4), (16 q1, 16 q5), (q2, q6),
// (16 q3, 16 q7) with exponent bits 0x6400 (`magic`, 0x64006400), eight v_fma_mix_f32 scale them,
// four v_cvt_pk_bf16_f32 pack.
__device__ __forceinline__ bf16x8 dequant_word_mix(uint32_t w, const MixCoef &c, uint32_t magic) {
    const uint32_t w8 = w >> 8;
    const uint32_t t0 = and_or(w, 0x000F000Fu, magic), t1 = and_or(w, 0x00F000F0u, magic);
    const uint32_t t2 = and_or(w8, 0x000F000Fu, magic), t3 = and_or(w8, 0x00F000F0u, magic);
    u32x4 d;
    d[0] = f32x2_to_bf16x2(fma_mix<false>(t0, c.s, c.b0), fma_mix<false>(t1, c.s16, c.b1));
    d[1] = f32x2_to_bf16x2(fma_mix<false>(t2, c.s, c.b0), fma_mix<false>(t3, c.s16, c.b1));
    d[2] = f32x2_to_bf16x2(fma_mix<true>(t0, c.s, c.b0), fma_mix<true>(t1, c.s16, c.b1));
    d[3] = f32x2_to_bf16x2(fma_mix<true>(t2, c.s, c.b0), fma_mix<true>(t3, c.s16, c.b1));
    return as_bf16x8(d);
}

}  // namespace splosh
