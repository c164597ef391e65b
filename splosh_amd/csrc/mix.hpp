// mix.hpp -- q4 dequantization to bf16 MFMA operands (shared by the M <= 64 and the prefill
// kernels).
#pragma once

#include "common.hpp"

namespace splosh {

// Eight weights of one code word (nibble j at bits 4 j = element k0 + j) as bf16 RNE(s q + b) in k
// order, 19 instructions, 11 of them simple VOP2-class ones: an AND and a shift-AND make the nibbles
// bytes; bytes 0..15 read as fp8 e4m3 are q 2^-9 exactly, so v_cvt_scalef32_pk_f32_fp8 with scale
// 2^9 (the scale only moves the exponent) gives two exact fp32 codes; fma(q, s, b) is DequantOracle's
// one-rounding weight (DequantOracle.swift:20-21) for any s and b; v_cvt_pk_bf16_f32 packs two.
__device__ __forceinline__ bf16x8 dequant_word_fp8(uint32_t w, float s, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const uint32_t lo = w & 0x0F0F0F0Fu;          // bytes: nibbles 0, 2, 4, 6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes: nibbles 1, 3, 5, 7
    const f32x2 q02 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, false);
    const f32x2 q46 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.0f, true);
    const f32x2 q13 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, false);
    const f32x2 q57 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.0f, true);
    u32x4 d;
    d[0] = f32x2_to_bf16x2(__builtin_fmaf(q02.x, s, b), __builtin_fmaf(q13.x, s, b));
    d[1] = f32x2_to_bf16x2(__builtin_fmaf(q02.y, s, b), __builtin_fmaf(q13.y, s, b));
    d[2] = f32x2_to_bf16x2(__builtin_fmaf(q46.x, s, b), __builtin_fmaf(q57.x, s, b));
    d[3] = f32x2_to_bf16x2(__builtin_fmaf(q46.y, s, b), __builtin_fmaf(q57.y, s, b));
    return as_bf16x8(d);
}

}  // namespace splosh
