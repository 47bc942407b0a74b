// Small kernels of the decode step and the matvec dispatcher.
//
//  * launch_matvec: argument checks of reference src/kernels/matvec_opt.cu:223-233, then the per
//    weight-type translation units.
//  * matvec_naive: reference src/kernels/matvec_naive.cu:13-32 (one thread per row, bf16, STORE).
//  * rmsnorm / add_inplace / silu_mul / set_token: reference src/kernels/rmsnorm.cu:12-28 and
//    src/kernels/elementwise.cu:10-44.
//  * embedding: reference src/kernels/embedding.cu:14-51 (token read on the device).
//  * argmax: reference src/kernels/argmax.cu:12-85 (ties to the lowest index; the final pass
//    writes the token and advances the device position).
#include <climits>
#include <vector>

#include "../kernels.h"
#include "device.h"

namespace cllm {

int device_cu_count() {
    static std::vector<int> cache;
    int dev = 0;
    CLLM_HIP(hipGetDevice(&dev));
    if (static_cast<int>(cache.size()) <= dev) cache.resize(dev + 1, 0);
    if (!cache[dev]) CLLM_HIP(hipDeviceGetAttribute(&cache[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cache[dev];
}

// The standalone matvec's launch per weight type and shape class, from a joint sweep of rpb and grid size on
// MI355X (each class's fastest mean kernel time).  Classes: 0 other (qkv, wo), 1 SwiGLU (gate_up), 2 8192 columns
// (down), 3 vocabulary-sized (>= 65536 rows: lm_head).
//
// kDefaultRpb is the rpb used when the caller passes 0.  kGridPerCu caps the grid at that many workgroups per CU
// (0: as many as can be resident at once).  Smaller grids mean fewer workgroups, each with more passes, so fewer
// repeats of the input and norm prologue; for bf16 lm_head a grid of 16 workgroups per CU, more than can be resident
// at once, spreads the last passes more evenly.  Measured effects: bf16 qkv 4.69 -> 4.40 us, gate_up 12.50 -> 12.00,
// down 7.65 -> 7.50, lm_head 79.8 -> 78.0 (8 per CU) -> 77.0 (16); int8 gate_up 8.53 -> 7.25; int4 gate_up
// 7.72 -> 6.68, lm_head 26.50 -> 25.28.
constexpr int kDefaultRpb[3][4] = {
    {1, 1, 2, 2},  // bf16
    {4, 2, 4, 4},  // int8
    {4, 4, 8, 4},  // int4
};
constexpr int kGridPerCu[3][4] = {
    {1, 1, 2, 16},  // bf16
    {0, 1, 0, 0},   // int8
    {0, 1, 0, 2},   // int4
};

namespace {
int shape_class(Epilogue ep, int rows, int cols) { return ep == Epilogue::SWIGLU ? 1 : cols >= 8192 ? 2 : rows >= 65536 ? 3 : 0; }

int type_index(WType wt) {
    switch (wt) {
        case WType::BF16: return 0;
        case WType::INT8: return 1;
        case WType::INT4: return 2;
    }
    throw ArgError("unknown weight type");
}
}  // namespace

int default_rpb(WType wt, Epilogue ep, int rows, int cols) { return kDefaultRpb[type_index(wt)][shape_class(ep, rows, cols)]; }

int grid_per_cu(WType wt, Epilogue ep, int rows, int cols) { return kGridPerCu[type_index(wt)][shape_class(ep, rows, cols)]; }

namespace {
thread_local KernelEvents t_kernel_events;
}

void arm_kernel_events(hipEvent_t start, hipEvent_t stop) { t_kernel_events = {start, stop}; }

KernelEvents take_kernel_events() {
    const KernelEvents e = t_kernel_events;
    t_kernel_events = {};
    return e;
}

template <WType WT>
void launch_matvec_wt(Epilogue ep, const MatvecArgs& a, int rpb, hipStream_t s);

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

void launch_matvec(WType wt, Epilogue ep, const MatvecArgs& a, int rpb, hipStream_t s) {
    CLLM_REQUIRE(a.w && a.x && a.y, "matvec: null pointer");
    CLLM_REQUIRE(a.rows > 0 && a.cols > 0, "matvec: bad shape");
    CLLM_REQUIRE(a.cols % 1024 == 0, "matvec: cols must be a multiple of 1024");
    CLLM_REQUIRE(a.cols <= 12288, "matvec: cols must be at most 12288");
    CLLM_REQUIRE(ep != Epilogue::SWIGLU || a.rows % 2 == 0, "matvec: SWIGLU needs an even row count");
    CLLM_REQUIRE(rpb == 1 || rpb == 2 || rpb == 4 || rpb == 8, "matvec: rpb must be 1, 2, 4 or 8");
    CLLM_REQUIRE(aligned16(a.w) && aligned16(a.x) && aligned16(a.y) && (!a.norm_w || aligned16(a.norm_w)),
                 "matvec: pointers must be 16-byte aligned");
    CLLM_REQUIRE(wt == WType::BF16 || a.scales, "matvec: quantized weights need scales");
    CLLM_REQUIRE(static_cast<const void*>(a.x) != static_cast<const void*>(a.y), "matvec: x and y alias");
    switch (wt) {
        case WType::BF16: return launch_matvec_wt<WType::BF16>(ep, a, rpb, s);
        case WType::INT8: return launch_matvec_wt<WType::INT8>(ep, a, rpb, s);
        case WType::INT4: return launch_matvec_wt<WType::INT4>(ep, a, rpb, s);
    }
    throw ArgError("matvec: unknown weight type");
}

namespace {

__global__ void __launch_bounds__(256) matvec_naive_kernel(const uint16_t* w, const float* x, float* y, int rows,
                                                           int cols) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint16_t* wr = w + static_cast<size_t>(r) * cols;
    float acc = 0.f;
    for (int j = 0; j < cols; ++j) acc += __builtin_bit_cast(float, static_cast<uint32_t>(wr[j]) << 16) * x[j];
    y[r] = acc;
}

__global__ void __launch_bounds__(256) rmsnorm_kernel(const float* x, const float* w, float eps, float* y, int n) {
    __shared__ float scratch[16];
    float ss = 0.f;
    for (int j = threadIdx.x; j < n; j += blockDim.x) ss += x[j] * x[j];
    ss = block_sum(ss, scratch);
    const float inv = rsqrtf(ss / static_cast<float>(n) + eps);
    for (int j = threadIdx.x; j < n; j += blockDim.x) y[j] = x[j] * inv * w[j];
}

__global__ void add_inplace_kernel(float* x, const float* y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

__global__ void silu_mul_kernel(const float* gu, float* act, int inter) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < inter) act[i] = silu(gu[i]) * gu[i + inter];
}

__global__ void set_token_kernel(int* d_token, int token) { *d_token = token; }

template <WType WT>
__global__ void __launch_bounds__(256) embedding_kernel(const void* w, const void* scales, const int* d_token, float* x,
                                                        int cols, int group) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= cols) return;
    const size_t tok = static_cast<size_t>(*d_token);
    if constexpr (WT == WType::BF16) {
        x[j] = __builtin_bit_cast(float, static_cast<uint32_t>(static_cast<const uint16_t*>(w)[tok * cols + j]) << 16);
    } else if constexpr (WT == WType::INT8) {
        x[j] = static_cast<float>(static_cast<const int8_t*>(w)[tok * cols + j]) * static_cast<const float*>(scales)[tok];
    } else {
        const uint8_t b = static_cast<const uint8_t*>(w)[tok * (cols / 2) + j / 2];
        const int q = static_cast<int>((j & 1) ? (b >> 4) : (b & 0x0F)) - 8;
        const uint16_t sb = static_cast<const uint16_t*>(scales)[tok * (cols / group) + j / group];
        x[j] = static_cast<float>(q) * half_bits_to_float(sb);
    }
}

// (value, index) order of the argmax: larger value first, then lower index.  NaN never wins.
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}

template <int CTRL>
__device__ __forceinline__ void arg_dpp_step(float& v, int& i) {
    const float ov = dpp<CTRL>(v);
    const int oi = dpp_i<CTRL>(i);
    if (arg_better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}

// Block of 256 threads: reduce (v, i) into (*out_v, *out_i) in a fixed order.
__device__ __forceinline__ void block_argmax(float v, int i, float* sv, int* si, float* out_v, int* out_i) {
    arg_dpp_step<kDppXor1>(v, i);
    arg_dpp_step<kDppXor2>(v, i);
    arg_dpp_step<kDppHalfMirror>(v, i);
    arg_dpp_step<kDppMirror>(v, i);
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    if ((lane & 15) == 0) {
        sv[w * 4 + lane / 16] = v;
        si[w * 4 + lane / 16] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = sv[0];
        int bi = si[0];
        for (int k = 1; k < 16; ++k)
            if (arg_better(sv[k], si[k], bv, bi)) {
                bv = sv[k];
                bi = si[k];
            }
        *out_v = bv;
        *out_i = bi;
    }
}

__global__ void __launch_bounds__(256) argmax_partial_kernel(const float* logits, int n, float* part_v, int* part_i) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x) {
        const float v = logits[j];
        if (arg_better(v, j, bv, bi)) {
            bv = v;
            bi = j;
        }
    }
    block_argmax(bv, bi, sv, si, part_v + blockIdx.x, part_i + blockIdx.x);
}

__global__ void __launch_bounds__(256) argmax_final_kernel(const float* part_v, const int* part_i, int* d_token,
                                                           int* d_pos) {
    __shared__ float sv[16];
    __shared__ int si[16];
    __shared__ float rv;
    __shared__ int ri;
    block_argmax(part_v[threadIdx.x], part_i[threadIdx.x], sv, si, &rv, &ri);
    if (threadIdx.x == 0) {
        *d_token = ri;
        *d_pos = *d_pos + 1;
    }
}

}  // namespace

void launch_matvec_naive(const MatvecArgs& a, hipStream_t s) {
    CLLM_REQUIRE(a.w && a.x && a.y && a.rows > 0 && a.cols > 0, "matvec_naive: bad arguments");
    CLLM_REQUIRE(a.norm_w == nullptr, "matvec_naive: no fused norm");
    CLLM_REQUIRE(static_cast<const void*>(a.x) != static_cast<const void*>(a.y), "matvec_naive: x and y alias");
    hipLaunchKernelGGL(matvec_naive_kernel, dim3((a.rows + 255) / 256), dim3(256), 0, s,
                       static_cast<const uint16_t*>(a.w), a.x, a.y, a.rows, a.cols);
    CLLM_HIP(hipGetLastError());
}

void launch_rmsnorm(const float* x, const float* w, float eps, float* y, int n, hipStream_t s) {
    CLLM_REQUIRE(x && w && y, "rmsnorm: null pointer");
    CLLM_REQUIRE(n > 0 && n % 256 == 0, "rmsnorm: n must be a positive multiple of 256");
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, s, x, w, eps, y, n);
    CLLM_HIP(hipGetLastError());
}

void launch_add_inplace(float* x, const float* y, int n, hipStream_t s) {
    CLLM_REQUIRE(x && y && n > 0, "add_inplace: bad arguments");
    hipLaunchKernelGGL(add_inplace_kernel, dim3((n + 255) / 256), dim3(256), 0, s, x, y, n);
    CLLM_HIP(hipGetLastError());
}

void launch_silu_mul(const float* gu, float* act, int inter, hipStream_t s) {
    CLLM_REQUIRE(gu && act && inter > 0, "silu_mul: bad arguments");
    hipLaunchKernelGGL(silu_mul_kernel, dim3((inter + 255) / 256), dim3(256), 0, s, gu, act, inter);
    CLLM_HIP(hipGetLastError());
}

void launch_set_token(int* d_token, int token, hipStream_t s) {
    CLLM_REQUIRE(d_token && token >= 0, "set_token: bad arguments");
    hipLaunchKernelGGL(set_token_kernel, dim3(1), dim3(1), 0, s, d_token, token);
    CLLM_HIP(hipGetLastError());
}

void launch_embedding(WType wt, const void* w, const void* scales, const int* d_token, float* x, int hidden, int vocab,
                      int group, hipStream_t s) {
    CLLM_REQUIRE(w && d_token && x && hidden > 0 && vocab > 0, "embedding: bad arguments");
    const dim3 grid((hidden + 255) / 256), block(256);
    switch (wt) {
        case WType::BF16:
            hipLaunchKernelGGL(embedding_kernel<WType::BF16>, grid, block, 0, s, w, scales, d_token, x, hidden, group);
            break;
        case WType::INT8:
            CLLM_REQUIRE(scales, "embedding: int8 needs scales");
            hipLaunchKernelGGL(embedding_kernel<WType::INT8>, grid, block, 0, s, w, scales, d_token, x, hidden, group);
            break;
        case WType::INT4:
            CLLM_REQUIRE(scales && group > 0 && hidden % group == 0 && hidden % 2 == 0, "embedding: int4 needs scales");
            hipLaunchKernelGGL(embedding_kernel<WType::INT4>, grid, block, 0, s, w, scales, d_token, x, hidden, group);
            break;
    }
    CLLM_HIP(hipGetLastError());
}

void launch_argmax(const float* logits, int n, float* part_v, int* part_i, int* d_token, int* d_pos, hipStream_t s) {
    CLLM_REQUIRE(logits && part_v && part_i && d_token && d_pos && n > 0, "argmax: bad arguments");
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxParts), dim3(256), 0, s, logits, n, part_v, part_i);
    CLLM_HIP(hipGetLastError());
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxParts), 0, s, part_v, part_i, d_token, d_pos);
    CLLM_HIP(hipGetLastError());
}

}  // namespace cllm
