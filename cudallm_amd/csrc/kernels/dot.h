// Weight formats and the dot product of one 16-byte weight chunk, shared by the standalone matvec
// and the persistent decode kernel.  A chunk holds 8 bf16, 16 int8 or 32 int4 columns of one row.
#pragma once

#include "../common.h"
#include "device.h"

namespace cllm {
namespace mv {

template <WType WT>
struct Fmt;
template <>
struct Fmt<WType::BF16> {
    static constexpr int CPC = 8;  // columns per 16-byte chunk
    static constexpr int CPL = 4;  // chunks per lane per 2048-column slice
};
template <>
struct Fmt<WType::INT8> {
    static constexpr int CPC = 16;
    static constexpr int CPL = 2;
};
template <>
struct Fmt<WType::INT4> {
    static constexpr int CPC = 32;
    static constexpr int CPL = 1;
};

template <WType WT>
__host__ __device__ constexpr size_t row_bytes(int cols) {
    return static_cast<size_t>(cols) * 16 / Fmt<WT>::CPC;
}

// Quantised chunks are dotted as unsigned codes: int8 q is read as q + 128 (sign bit flipped,
// then v_cvt_f32_ubyteN takes each byte straight from the register), int4 as its stored nibble
// q + 8.  The caller removes the bias once per lane: sum(q x) = sum(u x) - kBias * sum(x).
template <WType WT>
constexpr float kBias = WT == WType::INT8 ? 128.f : WT == WType::INT4 ? 8.f : 0.f;

// Dot of one 16-byte weight chunk with its CPC inputs (biased for quantised weights, see kBias).
template <WType WT>
__device__ __forceinline__ float chunk_dot(const u32x4 v, const float* x) {
    float acc = 0.f;
    if constexpr (WT == WType::BF16) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            acc = fmaf(bf16_lo(v[t]), x[2 * t], acc);
            acc = fmaf(bf16_hi(v[t]), x[2 * t + 1], acc);
        }
    } else if constexpr (WT == WType::INT8) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t u = v[t] ^ 0x80808080u;
#pragma unroll
            for (int b = 0; b < 4; ++b) acc = fmaf(static_cast<float>((u >> (8 * b)) & 0xffu), x[4 * t + b], acc);
        }
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t lo = v[t] & 0x0F0F0F0Fu;
            uint32_t hi = (v[t] >> 4) & 0x0F0F0F0Fu;
            // Opaque to the optimiser: with the masked words kept whole, each nibble converts straight
            // from its byte (v_cvt_f32_ubyteN) instead of a bit-field extract plus a conversion.
            asm("" : "+v"(lo), "+v"(hi));
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                acc = fmaf(static_cast<float>((lo >> (8 * b)) & 0xffu), x[8 * t + 2 * b], acc);
                acc = fmaf(static_cast<float>((hi >> (8 * b)) & 0xffu), x[8 * t + 2 * b + 1], acc);
            }
        }
    }
    return acc;
}

}  // namespace mv
}  // namespace cllm
