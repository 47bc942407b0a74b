// Weight quantisers on the GPU, bit-identical to reference python/cudallm/quantize.py:5-38.
//
// Both use IEEE single-precision division (HIP's default, correctly rounded) and rintf
// (round half to even), exactly the operations numpy performs in float32; the int4 scale is
// rounded to fp16 with round-to-nearest-even before it divides the weights.
#include "../kernels.h"
#include "device.h"

namespace cllm {

namespace {

// One workgroup of 256 threads per row.
__global__ void __launch_bounds__(256) quant_int8_kernel(const float* w, int cols, int8_t* q, float* scales) {
    __shared__ float scratch[4];
    const size_t r = blockIdx.x;
    const float* wr = w + r * cols;
    float m = 0.f;
    for (int j = threadIdx.x; j < cols; j += 256) m = fmaxf(m, fabsf(wr[j]));
    m = wave_max(m);
    if (threadIdx.x % kWave == 0) scratch[threadIdx.x / kWave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
    float s = m / 127.f;
    if (s == 0.f) s = 1.f;
    for (int j = threadIdx.x; j < cols; j += 256)
        q[r * cols + j] = static_cast<int8_t>(fmaxf(fminf(rintf(wr[j] / s), 127.f), -127.f));
    if (threadIdx.x == 0) scales[r] = s;
}

// One wave per 128-column group; lane l owns columns 2l and 2l+1 and writes packed byte l.
__global__ void __launch_bounds__(256) quant_int4_kernel(const float* w, int rows, int cols, uint8_t* packed,
                                                         uint16_t* scales) {
    const int groups = cols / 128;
    const long g = static_cast<long>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (g >= static_cast<long>(rows) * groups) return;  // wave-uniform
    const int lane = threadIdx.x % kWave;
    const long r = g / groups, gi = g % groups;
    const float* src = w + r * cols + gi * 128 + 2 * lane;
    const float a0 = src[0], a1 = src[1];
    const float m = wave_max(fmaxf(fabsf(a0), fabsf(a1)));
    float s = m / 7.f;
    if (s == 0.f) s = 1.f;
    const _Float16 s16 = static_cast<_Float16>(s);
    const float sf = static_cast<float>(s16);
    const int q0 = static_cast<int>(fmaxf(fminf(rintf(a0 / sf), 7.f), -8.f));
    const int q1 = static_cast<int>(fmaxf(fminf(rintf(a1 / sf), 7.f), -8.f));
    packed[r * (cols / 2) + gi * 64 + lane] = static_cast<uint8_t>((q0 + 8) | ((q1 + 8) << 4));
    if (lane == 0) scales[r * groups + gi] = __builtin_bit_cast(uint16_t, s16);
}

__global__ void __launch_bounds__(256) unpack_int4_kernel(const uint8_t* packed, long n_bytes, int8_t* q) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n_bytes) return;
    const uint8_t b = packed[i];
    q[2 * i] = static_cast<int8_t>((b & 0x0F) - 8);
    q[2 * i + 1] = static_cast<int8_t>((b >> 4) - 8);
}

}  // namespace

void launch_quantize_int8_rows(const float* w, int rows, int cols, int8_t* q, float* scales, hipStream_t s) {
    CLLM_REQUIRE(w && q && scales && rows > 0 && cols > 0, "quantize_int8_rows: bad arguments");
    hipLaunchKernelGGL(quant_int8_kernel, dim3(rows), dim3(256), 0, s, w, cols, q, scales);
    CLLM_HIP(hipGetLastError());
}

void launch_quantize_int4_groups(const float* w, int rows, int cols, uint8_t* packed, uint16_t* scales, hipStream_t s) {
    CLLM_REQUIRE(w && packed && scales && rows > 0 && cols > 0 && cols % 128 == 0,
                 "quantize_int4_groups: bad arguments (cols must be a multiple of 128)");
    const long groups = static_cast<long>(rows) * (cols / 128);
    CLLM_REQUIRE((groups + 3) / 4 <= 0x7fffffffL, "quantize_int4_groups: too many groups");
    hipLaunchKernelGGL(quant_int4_kernel, dim3(static_cast<unsigned>((groups + 3) / 4)), dim3(256), 0, s, w, rows, cols,
                       packed, scales);
    CLLM_HIP(hipGetLastError());
}

void launch_unpack_int4(const uint8_t* packed, int rows, int cols, int8_t* q, hipStream_t s) {
    CLLM_REQUIRE(packed && q && rows > 0 && cols > 0 && cols % 2 == 0, "unpack_int4: bad arguments");
    const long n = static_cast<long>(rows) * (cols / 2);
    hipLaunchKernelGGL(unpack_int4_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, packed, n, q);
    CLLM_HIP(hipGetLastError());
}

}  // namespace cllm
