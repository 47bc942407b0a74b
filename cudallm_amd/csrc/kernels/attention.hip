// RoPE + fp16 KV-cache write, split-K GQA decode attention and the naive attention baseline.
//
// Semantics (what is computed, which buffers change) follow the reference:
//   rope_kv fused / unfused      src/kernels/rope_kv.cu:10-79  (pairs (i, i+hd/2), angle fp32(pos)*inv_freq[i],
//                                fused leaves the k slice of qkv unrotated)
//   split-K partial + LSE merge  src/kernels/attention_opt.cu:17-134 (scale 0.125, 128-token splits, splits at or
//                                past ctx exit at once so the grid is fixed and graph-capturable, merge in split order)
//   naive                        src/kernels/attention_naive.cu:18-81 (one workgroup per query head)
// The gfx950 layout is this file's: a 256-thread workgroup = 4 waves = the 4 query heads of one
// kv head, each lane scores two tokens (lane, lane+64) with the query held in VGPRs, and each lane
// owns one of the 64 output dimensions for the p.V accumulation.
#include <array>
#include <mutex>

#include "../kernels.h"
#include "device.h"

namespace cllm {

namespace {

constexpr int kHd = 64;
constexpr int kGroup = 4;

// Rotation of pair (x0, x1) = (v[i], v[i+half]) by angle pos*inv_freq[i].
__device__ __forceinline__ void rotate(float x0, float x1, float ang, float& r0, float& r1) {
    float s, c;
    sincosf(ang, &s, &c);
    r0 = x0 * c - x1 * s;
    r1 = x1 * c + x0 * s;
}

// Work items: [0, (nh+nkv)*half) rotate one pair of a q or k head; then nkv*hd copies of v.
__global__ void __launch_bounds__(256) rope_kv_fused_kernel(float* qkv, const float* inv_freq, uint16_t* kc, uint16_t* vc,
                                                            const int* d_pos, int nh, int nkv, int hd, int max_seq) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2;
    const int pos = *d_pos;
    const int n_rot = (nh + nkv) * half;
    if (t < n_rot) {
        const int head = t / half, i = t % half;
        float* v = qkv + head * hd;
        float r0, r1;
        rotate(v[i], v[i + half], static_cast<float>(pos) * inv_freq[i], r0, r1);
        if (head < nh) {
            v[i] = r0;
            v[i + half] = r1;
        } else {
            uint16_t* dst = kc + (static_cast<size_t>(head - nh) * max_seq + pos) * hd;
            dst[i] = float_to_half_bits(r0);
            dst[i + half] = float_to_half_bits(r1);
        }
    } else if (t < n_rot + nkv * hd) {
        const int e = t - n_rot;
        const int head = e / hd, d = e % hd;
        vc[(static_cast<size_t>(head) * max_seq + pos) * hd + d] = float_to_half_bits(qkv[(nh + nkv) * hd + e]);
    }
}

__global__ void __launch_bounds__(256) rope_inplace_kernel(float* qkv, const float* inv_freq, const int* d_pos, int nh,
                                                           int nkv, int hd) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2;
    if (t >= (nh + nkv) * half) return;
    const int head = t / half, i = t % half;
    float* v = qkv + head * hd;
    float r0, r1;
    rotate(v[i], v[i + half], static_cast<float>(*d_pos) * inv_freq[i], r0, r1);
    v[i] = r0;
    v[i + half] = r1;
}

__global__ void __launch_bounds__(256) kv_write_kernel(const float* qkv, uint16_t* kc, uint16_t* vc, const int* d_pos,
                                                       int nh, int nkv, int hd, int max_seq) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= 2 * nkv * hd) return;
    const bool is_k = t < nkv * hd;
    const int e = is_k ? t : t - nkv * hd;
    const int head = e / hd, d = e % hd;
    uint16_t* cache = is_k ? kc : vc;
    cache[(static_cast<size_t>(head) * max_seq + *d_pos) * hd + d] = float_to_half_bits(qkv[nh * hd + t]);
}

// grid (nkv, max_seq/128), block 256.  LDS: K tile with one padding dword per row so lane j's row
// reads hit distinct banks, V tile unpadded (lanes read consecutive halves), p per head.
__global__ void __launch_bounds__(256) attn_partial_kernel(const float* q, const uint16_t* kc, const uint16_t* vc,
                                                           const int* d_pos, float* part_o, float* part_ml, int max_seq) {
    __shared__ uint32_t Ks[kAttnChunk][kHd / 2 + 1];
    __shared__ u32x4 Vs[kAttnChunk][kHd / 8];
    __shared__ float ps[kGroup][kAttnChunk];

    const int ctx = *d_pos + 1;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int t0 = split * kAttnChunk;
    if (t0 >= ctx) return;
    const int n = min(kAttnChunk, ctx - t0);
    const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;

    const uint16_t* Kg = kc + (static_cast<size_t>(kvh) * max_seq + t0) * kHd;
    const uint16_t* Vg = vc + (static_cast<size_t>(kvh) * max_seq + t0) * kHd;
    for (int idx = tid; idx < n * 8; idx += 256) {
        const int t = idx / 8, c = idx % 8;
        const u32x4 kv = *reinterpret_cast<const u32x4*>(Kg + t * kHd + c * 8);
        Ks[t][c * 4 + 0] = kv[0];
        Ks[t][c * 4 + 1] = kv[1];
        Ks[t][c * 4 + 2] = kv[2];
        Ks[t][c * 4 + 3] = kv[3];
        Vs[t][c] = *reinterpret_cast<const u32x4*>(Vg + t * kHd + c * 8);
    }
    const int h = kvh * kGroup + w;
    float qr[kHd];
#pragma unroll
    for (int d = 0; d < kHd; d += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(q + h * kHd + d);
        qr[d] = v[0];
        qr[d + 1] = v[1];
        qr[d + 2] = v[2];
        qr[d + 3] = v[3];
    }
    __syncthreads();

    float s[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int j = lane + kWave * k;
        if (j < n) {
            float dot = 0.f;
#pragma unroll
            for (int d2 = 0; d2 < kHd / 2; ++d2) {
                const uint32_t kk = Ks[j][d2];
                dot = fmaf(half_bits_to_float(static_cast<uint16_t>(kk)), qr[2 * d2], dot);
                dot = fmaf(half_bits_to_float(static_cast<uint16_t>(kk >> 16)), qr[2 * d2 + 1], dot);
            }
            s[k] = 0.125f * dot;
        } else {
            s[k] = -INFINITY;
        }
    }
    const float m = wave_max(fmaxf(s[0], s[1]));
    const float p0 = lane < n ? expf(s[0] - m) : 0.f;
    const float p1 = lane + kWave < n ? expf(s[1] - m) : 0.f;
    const float l = wave_sum(p0 + p1);
    ps[w][lane] = p0;
    ps[w][lane + kWave] = p1;
    __syncthreads();

    // Lane = output dimension d: o_d = sum_j p_j V[j][d].
    const uint16_t* vrow = reinterpret_cast<const uint16_t*>(&Vs[0][0]);
    float o = 0.f;
    for (int j = 0; j < n; ++j) o = fmaf(ps[w][j], half_bits_to_float(vrow[j * kHd + lane]), o);
    const int n_split = max_seq / kAttnChunk;
    const size_t slot = static_cast<size_t>(h) * n_split + split;
    part_o[slot * kHd + lane] = o;
    if (lane == 0) {
        part_ml[slot * 2] = m;
        part_ml[slot * 2 + 1] = l;
    }
}

// grid nh, block 64: merge the active splits of head h in split order.
__global__ void __launch_bounds__(64) attn_combine_kernel(const float* part_o, const float* part_ml, const int* d_pos,
                                                          float* out, int max_seq) {
    const int h = blockIdx.x, d = threadIdx.x;
    const int ctx = *d_pos + 1;
    const int used = (ctx + kAttnChunk - 1) / kAttnChunk;
    const int n_split = max_seq / kAttnChunk;
    const float* ml = part_ml + static_cast<size_t>(h) * n_split * 2;
    const float* po = part_o + static_cast<size_t>(h) * n_split * kHd;
    float M = -INFINITY;
    for (int s = 0; s < used; ++s) M = fmaxf(M, ml[2 * s]);
    float L = 0.f, acc = 0.f;
    for (int s = 0; s < used; ++s) {
        const float e = expf(ml[2 * s] - M);
        L = fmaf(ml[2 * s + 1], e, L);
        acc = fmaf(po[static_cast<size_t>(s) * kHd + d], e, acc);
    }
    out[h * kHd + d] = acc / L;
}

// grid nh, block 256, dynamic LDS max_seq floats of scores + 16 scratch.
__global__ void __launch_bounds__(256) attn_naive_kernel(const float* q, const uint16_t* kc, const uint16_t* vc,
                                                         const int* d_pos, float* out, int nh, int nkv, int hd,
                                                         int max_seq) {
    extern __shared__ float sm[];
    float* sc = sm;
    float* scratch = sm + max_seq;
    const int h = blockIdx.x, kvh = h / (nh / nkv);
    const int ctx = *d_pos + 1;
    const float* qh = q + h * hd;
    const uint16_t* K = kc + static_cast<size_t>(kvh) * max_seq * hd;
    const uint16_t* V = vc + static_cast<size_t>(kvh) * max_seq * hd;
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < ctx; t += blockDim.x) {
        float dot = 0.f;
        for (int d = 0; d < hd; ++d) dot += qh[d] * half_bits_to_float(K[static_cast<size_t>(t) * hd + d]);
        sc[t] = 0.125f * dot;
        mx = fmaxf(mx, sc[t]);
    }
    mx = wave_max(mx);
    if (threadIdx.x % kWave == 0) scratch[threadIdx.x / kWave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
    __syncthreads();
    float sum = 0.f;
    for (int t = threadIdx.x; t < ctx; t += blockDim.x) {
        sc[t] = expf(sc[t] - mx);
        sum += sc[t];
    }
    sum = block_sum(sum, scratch);
    if (threadIdx.x < hd) {
        float acc = 0.f;
        for (int t = 0; t < ctx; ++t) acc += sc[t] * half_bits_to_float(V[static_cast<size_t>(t) * hd + threadIdx.x]);
        out[h * hd + threadIdx.x] = acc / sum;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

void launch_rope_kv_fused(float* qkv, const float* inv_freq, uint16_t* k_cache, uint16_t* v_cache, const int* d_pos,
                          int nh, int nkv, int hd, int max_seq, hipStream_t s) {
    CLLM_REQUIRE(qkv && inv_freq && k_cache && v_cache && d_pos, "rope_kv: null pointer");
    CLLM_REQUIRE(nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && max_seq > 0, "rope_kv: bad dimensions");
    const int items = (nh + nkv) * (hd / 2) + nkv * hd;
    hipLaunchKernelGGL(rope_kv_fused_kernel, dim3((items + 255) / 256), dim3(256), 0, s, qkv, inv_freq, k_cache,
                       v_cache, d_pos, nh, nkv, hd, max_seq);
    CLLM_HIP(hipGetLastError());
}

void launch_rope_inplace(float* qkv, const float* inv_freq, const int* d_pos, int nh, int nkv, int hd, hipStream_t s) {
    CLLM_REQUIRE(qkv && inv_freq && d_pos, "rope: null pointer");
    CLLM_REQUIRE(nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0, "rope: bad dimensions");
    const int items = (nh + nkv) * (hd / 2);
    hipLaunchKernelGGL(rope_inplace_kernel, dim3((items + 255) / 256), dim3(256), 0, s, qkv, inv_freq, d_pos, nh, nkv,
                       hd);
    CLLM_HIP(hipGetLastError());
}

void launch_kv_write(const float* qkv, uint16_t* k_cache, uint16_t* v_cache, const int* d_pos, int nh, int nkv, int hd,
                     int max_seq, hipStream_t s) {
    CLLM_REQUIRE(qkv && k_cache && v_cache && d_pos, "kv_write: null pointer");
    CLLM_REQUIRE(nh > 0 && nkv > 0 && hd > 0 && max_seq > 0, "kv_write: bad dimensions");
    const int items = 2 * nkv * hd;
    hipLaunchKernelGGL(kv_write_kernel, dim3((items + 255) / 256), dim3(256), 0, s, qkv, k_cache, v_cache, d_pos, nh,
                       nkv, hd, max_seq);
    CLLM_HIP(hipGetLastError());
}

void launch_attention_splitk(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* d_pos,
                             float* part_o, float* part_ml, float* out, int nh, int nkv, int hd, int max_seq,
                             hipStream_t s) {
    CLLM_REQUIRE(q && k_cache && v_cache && d_pos && part_o && part_ml && out, "attention: null pointer");
    CLLM_REQUIRE(nkv > 0 && nh == kGroup * nkv, "attention (split-K): needs nh == 4 * nkv");
    CLLM_REQUIRE(hd == kHd, "attention (split-K): needs head_dim 64");
    CLLM_REQUIRE(max_seq > 0 && max_seq % kAttnChunk == 0, "attention (split-K): max_seq must be a multiple of 128");
    CLLM_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache), "attention: pointers must be 16-byte aligned");
    hipLaunchKernelGGL(attn_partial_kernel, dim3(nkv, max_seq / kAttnChunk), dim3(256), 0, s, q, k_cache, v_cache,
                       d_pos, part_o, part_ml, max_seq);
    CLLM_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_combine_kernel, dim3(nh), dim3(kHd), 0, s, part_o, part_ml, d_pos, out, max_seq);
    CLLM_HIP(hipGetLastError());
}

void launch_attention_naive(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* d_pos,
                            float* out, int nh, int nkv, int hd, int max_seq, hipStream_t s) {
    CLLM_REQUIRE(q && k_cache && v_cache && d_pos && out, "attention: null pointer");
    CLLM_REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0, "attention (naive): nh must be a multiple of nkv");
    CLLM_REQUIRE(hd > 0 && hd <= 256 && max_seq > 0, "attention (naive): bad dimensions");
    const size_t smem = (static_cast<size_t>(max_seq) + 16) * sizeof(float);
    CLLM_REQUIRE(smem <= 48 * 1024, "attention (naive): max_seq too large for the LDS score buffer");
    hipLaunchKernelGGL(attn_naive_kernel, dim3(nh), dim3(256), smem, s, q, k_cache, v_cache, d_pos, out, nh, nkv, hd,
                       max_seq);
    CLLM_HIP(hipGetLastError());
}

// ---- split-K attention with the partials in static device memory (no allocation on any call) ----------

namespace {

// The split partials of launch_attention_splitk_static: o [slot][64] then (m, l) [slot][2], slot = head * splits +
// split, for at most kStaticAttnSlots slots.  Each device holds its own copy of this array until the process ends.
// Its name is a host-side stand-in: host code uses only the address hipGetSymbolAddress reports, per device.
__device__ __align__(256) float scratch[kStaticAttnSlots * (kHd + 2)];

std::mutex g_scratch_mu;
std::array<float*, 64> g_scratch{};  // device address of `scratch`, indexed by device (no allocation, host or device)

float* scratch_on_current_device() {
    int dev = 0;
    CLLM_HIP(hipGetDevice(&dev));
    CLLM_REQUIRE(dev >= 0 && dev < static_cast<int>(g_scratch.size()), "attention scratch: device index above 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        CLLM_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        CLLM_INTERNAL(ptr, "attention scratch: no device address");
        g_scratch[dev] = static_cast<float*>(ptr);
    }
    return g_scratch[dev];
}

}  // namespace

void launch_attention_splitk_static(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* d_pos,
                                    float* out, int nh, int nkv, int hd, int max_seq, hipStream_t s) {
    CLLM_REQUIRE(nh > 0 && max_seq > 0 && max_seq % kAttnChunk == 0,
                 "attention (static scratch): max_seq must be a positive multiple of 128");
    CLLM_REQUIRE(static_cast<long long>(nh) * (max_seq / kAttnChunk) <= kStaticAttnSlots,
                 "attention (static scratch): nh * max_seq / 128 exceeds the 8192 partial slots of the static scratch");
    float* base = scratch_on_current_device();
    // No clearing needed: every split at or before ctx writes its slots before the merge reads them, and the merge
    // reads no other slot.
    launch_attention_splitk(q, k_cache, v_cache, d_pos, base, base + static_cast<size_t>(kStaticAttnSlots) * kHd, out,
                            nh, nkv, hd, max_seq, s);
}

}  // namespace cllm
