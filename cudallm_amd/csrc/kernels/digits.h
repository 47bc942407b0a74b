// Fixed-point digits of a normalised input for the integer dot products of the quantised weights, shared by the
// persistent decode kernel and the standalone matvec.  The input x^ is written as a 22-bit fixed-point integer with
// one power-of-two scale, xi = rint(x^ 2^e) (|xi| <= 2^22), offset by C so that every base-256 (int8) or base-16
// (int4) digit is non-negative, and packed in the weights' own layout; xor C then makes each digit signed, so that
// v_dot4_i32_i8 / v_dot8_i32_i4 multiply raw weight words by digits.  The integer sums are exact; the only new
// rounding is that of xi (at most 2^-23 of max |x^|), against fp32's 2^-24 of each |x^|.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cllm {

// Exponent e of the fixed-point scale from a bound m >= max |x^|: m 2^e < 2^22.  At most 126, so that 2^e and 2^-e
// are normal floats (inputs below 2^-104 then keep fewer bits, which changes nothing measurable).
__device__ __forceinline__ int dig_exponent(float m) {
    if (!(m > 0.f) || !(m < INFINITY)) return 0;
    return min(21 - ilogbf(m), 126);
}

// The offset fixed-point word (xi + C) mod 2^32 of xi = rint(v 2^e), from one FMA: v 2^e + 1.5 2^23 lands in
// [2^23, 2^24), where the float's bit pattern is 0x4B400000 + xi, rounded to nearest even like rintf.  The xor
// with C that makes the digits signed is applied to the packed digit words instead (every digit's top bit).
__device__ __forceinline__ uint32_t fixed_word(float v, float scale, uint32_t C) {
    return __builtin_bit_cast(uint32_t, fmaf(v, scale, 12582912.f)) + (C - 0x4B400000u);
}

// Byte planes of four 24-bit words: P[j] byte i = byte j of a_i (v_perm_b32 picks bytes of {s0, s1}; selector
// 0-3 = s1's bytes, 4-7 = s0's, 12 = zero).  Seven permutes instead of a shift, mask and insert per byte.
__device__ __forceinline__ void byte_planes(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t (&P)[3]) {
    const uint32_t t01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u), t23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
    P[0] = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
    P[1] = __builtin_amdgcn_perm(t23, t01, 0x07060302u);
    const uint32_t s01 = __builtin_amdgcn_perm(a1, a0, 0x0c0c0602u), s23 = __builtin_amdgcn_perm(a3, a2, 0x0c0c0602u);
    P[2] = __builtin_amdgcn_perm(s23, s01, 0x05040100u);
}

// The six base-16 digit words of eight 24-bit offset values u[b] (column b at nibble b): byte planes of the
// even and the odd columns, whose low and high nibbles interleave into digits 2j and 2j + 1.
__device__ __forceinline__ void nibble_words(const uint32_t (&u)[8], uint32_t (&w)[6]) {
    uint32_t E[3], O[3];
    byte_planes(u[0], u[2], u[4], u[6], E);
    byte_planes(u[1], u[3], u[5], u[7], O);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        w[2 * j] = ((O[j] << 4) & 0xF0F0F0F0u) | (E[j] & 0x0F0F0F0Fu);
        w[2 * j + 1] = (O[j] & 0xF0F0F0F0u) | ((E[j] >> 4) & 0x0F0F0F0Fu);
    }
}

}  // namespace cllm
