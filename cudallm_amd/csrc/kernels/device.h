// Device helpers shared by the gfx950 kernels: wave64 reductions built from DPP row operations,
// streaming 128-bit loads, bf16/fp16 conversions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cllm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// 128-bit load marked non-temporal: weights are read exactly once per decode step, so they
// should not displace the activations and the KV cache from the caches.
// The pointer is cast to the global address space so the load is a global_load even when the
// pointer itself was read from memory (a generic pointer would become a slower flat_load).
typedef const __attribute__((address_space(1))) u32x4 global_u32x4;
__device__ __forceinline__ u32x4 load_stream(const void* p) {
    return __builtin_nontemporal_load((global_u32x4*)p);
}

// Plain load through the global address space (for pointers that were read from memory).
template <typename T>
__device__ __forceinline__ T gload(const T* p) {
    return *((const __attribute__((address_space(1))) T*)p);
}

// DPP move of a float within 16-lane rows (control words of the gfx9 DPP encoding).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i inside each 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i inside each 16

// Sum over all 64 lanes; every lane gets the same result.  Fixed association order, so the
// result is deterministic: (((row0 + row1) + row2) + row3) of the 16-lane butterfly sums.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return ((a + b) + c) + d;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// x of lane l plus x of lane l ^ M, for M = 16 or 32, by gfx950's permlane swaps (VALU, no LDS).  With x in both
// registers, v_permlane16_swap exchanges the odd 16-lane rows of the first with the even rows of the second (the
// 32-lane form: the upper half of the first with the lower half of the second), so each register ends with one lane
// of every pair (l, l ^ M) and their sum is the pair's sum in both lanes.  Inline asm because the compiler's builtin
// returns the first register for both results; the s_nop covers the wait states after the VALU writes of x.
template <int M>
__device__ __forceinline__ float sum_lanes_xor(float x) {
    static_assert(M == 16 || M == 32, "row swaps");
    unsigned a = __builtin_bit_cast(unsigned, x), b = a;
    if constexpr (M == 16) {
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    } else {
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    }
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// x of lane l ^ M (M a power of two below 64): quad permutes for 1 and 2, a rotation by 8 inside each 16-lane row
// for 8 (the same lanes), the LDS crossbar's swizzle (bit mode, 32-lane groups) for 4 and 16, a permute for 32.
template <int M>
__device__ __forceinline__ float xor_lanes(float x) {
    if constexpr (M == 1) return dpp<kDppXor1>(x);
    if constexpr (M == 2) return dpp<kDppXor2>(x);
    if constexpr (M == 8) return dpp<0x128>(x);  // row_ror:8
    if constexpr (M == 4 || M == 16)
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x1F | (M << 10)));
    if constexpr (M == 32) return __shfl_xor(x, 32);
}

// Sums R per-lane partials (one per row; R = 1, 2, 4 or 8) over the wave: lane l ends with the sum of row l mod R.
// log2 R exchange steps halve the values a lane holds (bit b of the lane picks the half it keeps; the other half goes
// to lane l ^ 2^b, which keeps it), then the remaining lane bits are summed directly.  About 3 instructions per
// row instead of a full reduction (4 row operations, 4 readlanes, 3 adds) per row.  The last two steps are the
// permlane swaps (sum_lanes_xor).
template <int R, int B = 0>
__device__ __forceinline__ void exchange(float (&v)[R], int lane) {
    if constexpr ((1 << B) < R) {
        constexpr int M = 1 << B;
        const bool hi = (lane & M) != 0;
#pragma unroll
        for (int k = 0; k < R / (2 << B); ++k) {
            const float a = v[2 * k], c = v[2 * k + 1];
            v[k] = (hi ? c : a) + xor_lanes<M>(hi ? a : c);
        }
        exchange<R, B + 1>(v, lane);
    }
}
template <int R>
__device__ __forceinline__ float rows_sum(const float (&d)[R], int lane) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8, "rows per pass");
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = d[i];
    exchange<R>(v, lane);
    float x = v[0];
    if constexpr (R < 2) x += xor_lanes<1>(x);
    if constexpr (R < 4) x += xor_lanes<2>(x);
    if constexpr (R < 8) x += xor_lanes<4>(x);
    x += xor_lanes<8>(x);
    x = sum_lanes_xor<16>(x);
    return sum_lanes_xor<32>(x);
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024); `scratch` holds 16 floats.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) scratch[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += scratch[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__device__ __forceinline__ float half_bits_to_float(uint16_t b) { return static_cast<float>(__builtin_bit_cast(_Float16, b)); }
// Round-to-nearest-even fp32 -> fp16 bits.
__device__ __forceinline__ uint16_t float_to_half_bits(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

__device__ __forceinline__ float silu(float g) { return g / (1.f + expf(-g)); }

}  // namespace cllm
