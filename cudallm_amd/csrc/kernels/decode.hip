// Persistent batch-1 decode step for gfx950: one launch computes one token.
//
// What is computed is the fused op order of reference src/engine/engine.cpp:181-237 (embedding;
// per layer qkv with RMSNorm prologue, RoPE + fp16 KV write, split-K GQA attention with an LSE
// merge, wo + residual, gate_up with RMSNorm prologue and SwiGLU, down + residual; lm_head with
// the final RMSNorm; argmax that writes the token and advances the position).  How it is
// scheduled is this file's own:
//
//  * One workgroup of 4 waves per CU (one wave per SIMD, so each wave may use 512 registers and
//    the prefetched weight rows never go to scratch); every workgroup runs every phase.  Matvec
//    rows are dealt to waves round-robin, attention splits to workgroups.
//  * Phases exchange vectors through tagged 64-bit words (see decode.h).  A consumer loads the
//    vector it needs with relaxed agent-scope atomics and re-loads only entries whose tag is not
//    yet the current phase's.  No grid barriers, no RMW atomics and no cache flushes on the data
//    path: the dependency chain costs one store->load hop per phase.
//  * A wave issues the weight loads of its first rows (and their scales) BEFORE it waits for the
//    phase input, so the HBM stream continues while the producing phase finishes elsewhere; the
//    attention workgroups likewise pull their K/V tiles before waiting for q.
//  * Every wait is bounded.  On overrun the wave sets the sticky d_err flag and continues with
//    whatever it read; other waits notice the flag and stop waiting, so the grid always drains.
//    Indices never depend on activation values and the token is clamped, so no access can leave
//    its buffer even then.  The host reports the flag as a device error.
#include "../decode.h"
#include "../kernels.h"
#include "device.h"
#include "dot.h"

namespace cllm {
namespace dk {

using mv::Fmt;
using mv::chunk_dot;
using mv::kBias;
using mv::row_bytes;

constexpr int kThreads = kDecodeThreads, kWaves = kThreads / kWave;
constexpr int H = 2048, INTER = 8192, NH = 32, NKV = 8, HD = 64, QKV = (NH + 2 * NKV) * HD, VOCAB = 128256, NL = 16;
constexpr int kTagStride = 8;            // tag slots per layer
constexpr unsigned kEpochStride = 256;   // tag slots per step
constexpr unsigned kSpinCap = 1u << 20;  // bounded waits (~1 s of polling)
constexpr int kPartStride = HD + 2;      // o[64], m, l
constexpr int kPairs = QKV / 2;          // RoPE pairs (i, i+32) of every q/k/v head
// Units per wave when the grid has 256 workgroups (1024 waves); smaller grids loop further.
constexpr int kNW = 256 * kWaves;
constexpr int kQkvU = (kPairs + kNW - 1) / kNW;  // 2 pairs
constexpr int kWoU = (H + kNW - 1) / kNW;        // 2 rows
constexpr int kGuU = (INTER + kNW - 1) / kNW;    // 8 gate/up units
constexpr int kDownU = (H + kNW - 1) / kNW;      // 2 rows

enum : unsigned { T_QKV = 0, T_ATT_PART = 1, T_ATT = 2, T_XA = 3, T_ACT = 4, T_X = 5 };
constexpr unsigned T_ARG = NL * kTagStride;

__device__ __forceinline__ uint64_t tload(const uint64_t* a) {
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(uint64_t* a, float v, unsigned tag) {
    __hip_atomic_store(a, (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tagged(uint64_t v, unsigned tag) { return static_cast<unsigned>(v >> 32) == tag; }
__device__ __forceinline__ float tvalue(uint64_t v) { return __builtin_bit_cast(float, static_cast<uint32_t>(v)); }
__device__ __forceinline__ bool failed(unsigned* err) {
    return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void fail(unsigned* err) {
    __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// True when a wait must stop: it ran out of polls, or another wave already failed.
__device__ __forceinline__ bool give_up(unsigned& spins, unsigned* err) {
    if (++spins >= kSpinCap || ((spins & 255u) == 0 && failed(err))) {
        fail(err);
        return true;
    }
    __builtin_amdgcn_s_sleep(1);
    return false;
}

// Wait for one tagged value (per lane).
__device__ __forceinline__ float wait1(const uint64_t* a, unsigned tag, unsigned* err) {
    uint64_t v = tload(a);
    unsigned spins = 0;
    while (!tagged(v, tag) && !give_up(spins, err)) v = tload(a);
    return tvalue(v);
}

// The whole workgroup copies N tagged floats into LDS once every tag equals `tag`.
template <int N>
__device__ void fetch(const uint64_t* src, unsigned tag, float* dst, unsigned* err, int tid) {
    constexpr int PT = N / kThreads;
    static_assert(N % kThreads == 0, "fetch size");
    uint64_t v[PT];
#pragma unroll
    for (int k = 0; k < PT; ++k) v[k] = tload(src + tid + k * kThreads);
    unsigned spins = 0;
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < PT; ++k) ok = ok && tagged(v[k], tag);
        if (ok || give_up(spins, err)) break;
#pragma unroll
        for (int k = 0; k < PT; ++k)
            if (!tagged(v[k], tag)) v[k] = tload(src + tid + k * kThreads);
    }
#pragma unroll
    for (int k = 0; k < PT; ++k) dst[tid + k * kThreads] = tvalue(v[k]);
    __syncthreads();
}

// 1 / rms(x), identical in every workgroup (same partition, same order).
__device__ float rms_inv(const float* x, float eps, float* scratch, int tid) {
    float ss = 0.f;
    for (int j = tid; j < H; j += kThreads) ss += x[j] * x[j];
    ss = block_sum(ss, scratch);
    return rsqrtf(ss / static_cast<float>(H) + eps);
}

// The lane's 32 inputs of a 2048-wide row (same column mapping as the standalone matvec), scaled
// by inv * norm_w when NORM.  norm_w is read with 128-bit global loads.
typedef const __attribute__((address_space(1))) f32x4 global_f32x4;
template <WType WT, bool NORM>
__device__ __forceinline__ void lane_inputs(const float* x, const float* norm_w, float inv, float* xr, float& xsum,
                                            int lane) {
    using F = Fmt<WT>;
    xsum = 0.f;
#pragma unroll
    for (int k = 0; k < F::CPL; ++k) {
        const int c0 = (k * kWave + lane) * F::CPC;
#pragma unroll
        for (int j = 0; j < F::CPC; j += 4) {
            const f32x4 xv = *reinterpret_cast<const f32x4*>(x + c0 + j);
            f32x4 nw = {1.f, 1.f, 1.f, 1.f};
            if constexpr (NORM) nw = *((global_f32x4*)(norm_w + c0 + j));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = NORM ? xv[e] * inv * nw[e] : xv[e];
                xr[k * F::CPC + j + e] = v;
                xsum += v;
            }
        }
    }
}

// One 2048-wide weight row as this lane holds it: its 16-byte chunks and the scale it needs
// (int8: the row scale; int4: the scale of the lane's 128-column group).
template <WType WT>
struct Row {
    u32x4 w[Fmt<WT>::CPL];
    float s;
};

template <WType WT>
__device__ __forceinline__ void load_row(const void* w, const void* scales, int row, int lane, Row<WT>& r) {
    const char* p = static_cast<const char*>(w) + static_cast<size_t>(row) * row_bytes<WT>(H) + lane * 16;
#pragma unroll
    for (int k = 0; k < Fmt<WT>::CPL; ++k) r.w[k] = load_stream(p + k * 1024);
    if constexpr (WT == WType::INT8) r.s = gload(static_cast<const float*>(scales) + row);
    if constexpr (WT == WType::INT4)
        r.s = half_bits_to_float(
            gload(static_cast<const uint16_t*>(scales) + static_cast<size_t>(row) * (H / 128) + lane / 4));
}

// Complete dot of a 2048-wide row, uniform across the wave.
template <WType WT>
__device__ __forceinline__ float row_dot(const Row<WT>& r, const float* xr, float xsum) {
    using F = Fmt<WT>;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < F::CPL; ++k) s += chunk_dot<WT>(r.w[k], xr + k * F::CPC);
    if constexpr (WT == WType::INT8) s -= kBias<WT> * xsum;
    if constexpr (WT == WType::INT4) s = r.s * (s - kBias<WT> * xsum);
    s = wave_sum(s);
    if constexpr (WT == WType::INT8) s *= r.s;
    return s;
}

// One 8192-wide row (down projection): DCH chunks per lane, inputs read from LDS.
template <WType WT>
struct DRow {
    static constexpr int DCH = INTER / Fmt<WT>::CPC / kWave;
    u32x4 w[DCH];
    float s[WT == WType::INT4 ? DCH : 1];
};

template <WType WT>
__device__ __forceinline__ void load_drow(const void* w, const void* scales, int row, int lane, DRow<WT>& r) {
    constexpr int DCH = DRow<WT>::DCH;
    const char* p = static_cast<const char*>(w) + static_cast<size_t>(row) * row_bytes<WT>(INTER) + lane * 16;
#pragma unroll
    for (int k = 0; k < DCH; ++k) r.w[k] = load_stream(p + k * 1024);
    if constexpr (WT == WType::INT8) r.s[0] = gload(static_cast<const float*>(scales) + row);
    if constexpr (WT == WType::INT4) {
        const uint16_t* sc = static_cast<const uint16_t*>(scales) + static_cast<size_t>(row) * (INTER / 128);
#pragma unroll
        for (int k = 0; k < DCH; ++k) r.s[k] = half_bits_to_float(gload(sc + (k * kWave + lane) / 4));
    }
}

template <WType WT>
__device__ __forceinline__ float drow_dot(const DRow<WT>& r, const float* x, int lane) {
    using F = Fmt<WT>;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < DRow<WT>::DCH; ++k) {
        if (k % 4 == 0) __builtin_amdgcn_sched_barrier(0);
        const float* xc = x + (k * kWave + lane) * F::CPC;
        float t = chunk_dot<WT>(r.w[k], xc);
        if constexpr (WT != WType::BF16) {
            float cs = 0.f;
#pragma unroll
            for (int j = 0; j < F::CPC; ++j) cs += xc[j];
            t -= kBias<WT> * cs;
        }
        if constexpr (WT == WType::INT4) t *= r.s[k];
        s += t;
    }
    s = wave_sum(s);
    if constexpr (WT == WType::INT8) s *= r.s[0];
    return s;
}

template <WType WT>
__device__ __forceinline__ float embed(const void* w, const void* s, int tok, int j) {
    const size_t t = static_cast<size_t>(tok);
    if constexpr (WT == WType::BF16) {
        return __builtin_bit_cast(float, static_cast<uint32_t>(gload(static_cast<const uint16_t*>(w) + t * H + j)) << 16);
    } else if constexpr (WT == WType::INT8) {
        return static_cast<float>(gload(static_cast<const int8_t*>(w) + t * H + j)) *
               gload(static_cast<const float*>(s) + t);
    } else {
        const uint8_t b = gload(static_cast<const uint8_t*>(w) + t * (H / 2) + j / 2);
        const int q = static_cast<int>((j & 1) ? (b >> 4) : (b & 0x0F)) - 8;
        return static_cast<float>(q) *
               half_bits_to_float(gload(static_cast<const uint16_t*>(s) + t * (H / 128) + j / 128));
    }
}

// Phase-end timestamp of this workgroup (thread 0), when stamping is enabled.
__device__ __forceinline__ void stamp(const DecodeParams& p, int slot) {
    if (p.stamps && threadIdx.x == 0) p.stamps[blockIdx.x * kStampSlots + slot] = __builtin_amdgcn_s_memrealtime();
}
// In-phase timestamp, recorded for layer 1 only (slots kInPhase + 2 * phase + {0: input arrived, 1: prologue done}).
constexpr int kInPhase = 100;
__device__ __forceinline__ void stamp_in(const DecodeParams& p, int l, int phase, int k) {
    if (l == 1) stamp(p, kInPhase + 2 * phase + k);
}

// Argmax order: larger value first, then lower index (numpy's tie rule).  NaN never wins.
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int CTRL>
__device__ __forceinline__ void arg_dpp(float& v, int& i) {
    const float ov = dpp<CTRL>(v);
    const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xf, 0xf, true);
    if (arg_better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}

// Argmax over the 64 lanes of a wave; the result is uniform across the wave.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    arg_dpp<kDppXor1>(v, i);
    arg_dpp<kDppXor2>(v, i);
    arg_dpp<kDppHalfMirror>(v, i);
    arg_dpp<kDppMirror>(v, i);
    float bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float ov = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), r));
        const int oi = __builtin_amdgcn_readlane(i, r);
        if (arg_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    v = bv;
    i = bi;
}

template <WType WT>
__global__ void __launch_bounds__(kThreads) decode_kernel(DecodeParams p) {
    using F = Fmt<WT>;
    constexpr int NX = F::CPL * F::CPC;
    // LDS: layer input, post-attention residual, this step's RoPE cos/sin, and one 36 KiB region
    // that holds either the attention tiles, the attention output or the SwiGLU output.
    __shared__ float xin[H];
    __shared__ float xa[H];
    __shared__ __align__(16) float big[9216];
    __shared__ float rope_c[HD / 2], rope_s[HD / 2];
    __shared__ float scratch[16];
    __shared__ float red_v[kWaves];
    __shared__ int red_i[kWaves];

    const int G = gridDim.x, NW = G * kWaves;
    unsigned* err = p.d_err;
    const int pos = *p.d_pos;
    const int tok = min(max(*p.d_token, 0), VOCAB - 1);
    const unsigned step = *p.d_step;
    const unsigned base = step * kEpochStride;
    const int ctx = pos + 1;
    const int nsplit = (ctx + kAttnChunk - 1) / kAttnChunk;
    const int NS = p.max_seq / kAttnChunk;
    const size_t layer_cache = static_cast<size_t>(NKV) * p.max_seq * HD;

    stamp(p, 0);
    for (int j = threadIdx.x; j < H; j += kThreads) xin[j] = embed<WT>(p.emb, p.emb_s, tok, j);
    if (threadIdx.x < HD / 2) {  // the angles depend only on the position: one sincos per pair per step
        float sn, cs;
        sincosf(static_cast<float>(pos) * gload(p.inv_freq + threadIdx.x), &sn, &cs);
        rope_s[threadIdx.x] = sn;
        rope_c[threadIdx.x] = cs;
    }
    if (p.residuals && blockIdx.x == 0)
        for (int j = threadIdx.x; j < H; j += kThreads) p.residuals[j] = xin[j];
    __syncthreads();

    // An opaque copy of the thread index, renewed at every phase: without it the compiler computes
    // the per-thread addresses of all phases up front and keeps them live across the whole layer.
    int tid = 0, wave = 0, lane = 0, gw = 0;
    auto renew = [&] {
        tid = threadIdx.x;
        asm volatile("" : "+v"(tid)::"memory");
        wave = tid / kWave;
        lane = tid % kWave;
        gw = blockIdx.x * kWaves + wave;
    };

#pragma unroll 1
    for (int l = 0; l < NL; ++l) {
        const DecodeLayer Lw = p.layers[l];
        const unsigned tg = base + l * kTagStride;
        uint64_t* tqkv = p.tqkv + static_cast<size_t>(l) * QKV;
        uint64_t* tatt = p.tatt + static_cast<size_t>(l) * H;
        uint64_t* tpart = p.tpart + static_cast<size_t>(l) * NH * NS * kPartStride;
        uint64_t* txa = p.txa + static_cast<size_t>(l) * H;
        uint64_t* tact = p.tact + static_cast<size_t>(l) * INTER;
        uint64_t* txo = p.tx + static_cast<size_t>(l + 1) * H;

        // ---- qkv (+ attn_norm prologue, RoPE, fp16 KV write); unit = RoPE pair (i, i+32) of a head ----
        renew();
        {
            Row<WT> ra[kQkvU], rb[kQkvU];
#pragma unroll
            for (int i = 0; i < kQkvU; ++i) {
                const int u = gw + i * NW;
                if (u < kPairs) {
                    const int r0 = (u / 32) * HD + u % 32;
                    load_row<WT>(Lw.wqkv, Lw.sqkv, r0, lane, ra[i]);
                    load_row<WT>(Lw.wqkv, Lw.sqkv, r0 + 32, lane, rb[i]);
                }
            }
            if (l > 0) fetch<H>(p.tx + static_cast<size_t>(l) * H, tg - kTagStride + T_X, xin, err, tid);
            stamp_in(p, l, 0, 0);
            const float inv = rms_inv(xin, p.eps, scratch, tid);
            float xr[NX], xsum;
            lane_inputs<WT, true>(xin, Lw.attn_norm, inv, xr, xsum, lane);
            stamp_in(p, l, 0, 1);
            auto finish = [&](int u, float d0, float d1) {
                const int h = u / 32, i = u % 32, r0 = h * HD + i;
                float o0 = d0, o1 = d1;
                if (h < NH + NKV) {
                    o0 = d0 * rope_c[i] - d1 * rope_s[i];
                    o1 = d1 * rope_c[i] + d0 * rope_s[i];
                }
                tstore(tqkv + r0, o0, tg + T_QKV);
                tstore(tqkv + r0 + 32, o1, tg + T_QKV);
                if (h >= NH) {
                    uint16_t* cache = h < NH + NKV ? p.k_cache : p.v_cache;
                    const size_t off = l * layer_cache + (static_cast<size_t>((h - NH) % NKV) * p.max_seq + pos) * HD;
                    cache[off + i] = float_to_half_bits(o0);
                    cache[off + i + 32] = float_to_half_bits(o1);
                }
            };
#pragma unroll
            for (int i = 0; i < kQkvU; ++i) {
                const int u = gw + i * NW;
                __builtin_amdgcn_sched_barrier(0);
                if (u < kPairs) {
                    const float d0 = row_dot<WT>(ra[i], xr, xsum);
                    const float d1 = row_dot<WT>(rb[i], xr, xsum);
                    if (lane == 0) finish(u, d0, d1);
                }
            }
#pragma unroll 1
            for (int u = gw + kQkvU * NW; u < kPairs; u += NW) {  // grids below 256 workgroups
                const int r0 = (u / 32) * HD + u % 32;
                load_row<WT>(Lw.wqkv, Lw.sqkv, r0, lane, ra[0]);
                load_row<WT>(Lw.wqkv, Lw.sqkv, r0 + 32, lane, rb[0]);
                const float d0 = row_dot<WT>(ra[0], xr, xsum);
                const float d1 = row_dot<WT>(rb[0], xr, xsum);
                if (lane == 0) finish(u, d0, d1);
            }
        }
        stamp(p, 1 + 6 * l + 0);

        // ---- split-K attention: task = (kv head, 128-token split), one workgroup per task ----
        renew();
        {
            uint32_t* Ks = reinterpret_cast<uint32_t*>(big);  // [128][33]
            u32x4* Vs = reinterpret_cast<u32x4*>(big + 4224);  // [128][8]
            float* ps = big + 8320;                            // [4][128]
            float* qs = big + 8832;                            // [4][64]
            float* kvc = big + 9088;                           // [2][64] this token's k, v
            constexpr int kTile = kAttnChunk * 8 / kThreads;   // 16-byte chunks per thread
            const int T = NKV * nsplit;
#pragma unroll 1
            for (int t = blockIdx.x; t < T; t += G) {
                const int kvh = t % NKV, split = t / NKV;
                const int t0 = split * kAttnChunk, n = min(kAttnChunk, ctx - t0);
                const uint16_t* Kg = p.k_cache + l * layer_cache + static_cast<size_t>(kvh) * p.max_seq * HD;
                const uint16_t* Vg = p.v_cache + l * layer_cache + static_cast<size_t>(kvh) * p.max_seq * HD;
                // Earlier tokens come from the cache and do not depend on this step: request them first.
                u32x4 kt[kTile], vt[kTile];
#pragma unroll
                for (int k = 0; k < kTile; ++k) {
                    const int idx = tid + k * kThreads, r = idx / 8, c = idx % 8;
                    if (r < n && t0 + r < pos) {
                        kt[k] = load_stream(Kg + static_cast<size_t>(t0 + r) * HD + c * 8);
                        vt[k] = load_stream(Vg + static_cast<size_t>(t0 + r) * HD + c * 8);
                    }
                }
                // q of the group's 4 heads and (last split only) this token's k and v: one wait per thread.
                qs[tid] = wait1(tqkv + (kvh * 4) * HD + tid, tg + T_QKV, err);
                if (tid < 2 * HD && t0 + n - 1 == pos)
                    kvc[tid] = wait1(tqkv + (tid < HD ? NH * HD : (NH + NKV) * HD - HD) + kvh * HD + tid, tg + T_QKV, err);
                __syncthreads();
                if (t == static_cast<int>(blockIdx.x)) stamp_in(p, l, 1, 0);
#pragma unroll
                for (int k = 0; k < kTile; ++k) {
                    const int idx = tid + k * kThreads, r = idx / 8, c = idx % 8;
                    if (r < n) {
                        u32x4 kv = kt[k], vv = vt[k];
                        if (t0 + r == pos) {  // rounded to fp16 exactly as the qkv phase wrote the cache
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                kv[e] = static_cast<uint32_t>(float_to_half_bits(kvc[c * 8 + 2 * e])) |
                                        (static_cast<uint32_t>(float_to_half_bits(kvc[c * 8 + 2 * e + 1])) << 16);
                                vv[e] = static_cast<uint32_t>(float_to_half_bits(kvc[HD + c * 8 + 2 * e])) |
                                        (static_cast<uint32_t>(float_to_half_bits(kvc[HD + c * 8 + 2 * e + 1])) << 16);
                            }
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) Ks[r * 33 + c * 4 + e] = kv[e];
                        Vs[r * 8 + c] = vv;
                    }
                }
                __syncthreads();
                // wave w = query head kvh*4 + w; lane scores tokens lane and lane + 64.
                float s[2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int j = lane + kWave * k;
                    if (j < n) {
                        float dot = 0.f;
#pragma unroll
                        for (int d2 = 0; d2 < HD / 2; ++d2) {
                            const uint32_t kk = Ks[j * 33 + d2];
                            dot = fmaf(half_bits_to_float(static_cast<uint16_t>(kk)), qs[wave * HD + 2 * d2], dot);
                            dot = fmaf(half_bits_to_float(static_cast<uint16_t>(kk >> 16)), qs[wave * HD + 2 * d2 + 1], dot);
                        }
                        s[k] = 0.125f * dot;
                    } else {
                        s[k] = -INFINITY;
                    }
                }
                const float m = wave_max(fmaxf(s[0], s[1]));
                const float p0 = lane < n ? expf(s[0] - m) : 0.f;
                const float p1 = lane + kWave < n ? expf(s[1] - m) : 0.f;
                const float lsum = wave_sum(p0 + p1);
                ps[wave * kAttnChunk + lane] = p0;
                ps[wave * kAttnChunk + lane + kWave] = p1;
                __syncthreads();
                const uint16_t* vrow = reinterpret_cast<const uint16_t*>(Vs);
                float o = 0.f;
                for (int j = 0; j < n; ++j) o = fmaf(ps[wave * kAttnChunk + j], half_bits_to_float(vrow[j * HD + lane]), o);
                const int h = kvh * 4 + wave;
                if (nsplit == 1) {
                    tstore(tatt + h * HD + lane, o / lsum, tg + T_ATT);
                } else {
                    uint64_t* pp = tpart + (static_cast<size_t>(h) * NS + split) * kPartStride;
                    tstore(pp + lane, o, tg + T_ATT_PART);
                    if (lane == 0) {
                        tstore(pp + HD, m, tg + T_ATT_PART);
                        tstore(pp + HD + 1, lsum, tg + T_ATT_PART);
                    }
                }
                __syncthreads();
            }
        }
        stamp(p, 1 + 6 * l + 1);

        // ---- LSE merge of the splits: one wave per head, lane s holds split s (nsplit <= 64) ----
        renew();
        if (nsplit > 1) {
#pragma unroll 1
            for (int h = gw; h < NH; h += NW) {
                const uint64_t* pp = tpart + static_cast<size_t>(h) * NS * kPartStride;
                float ms = -INFINITY, ls = 0.f;
                if (lane < nsplit) {
                    ms = wait1(pp + lane * kPartStride + HD, tg + T_ATT_PART, err);
                    ls = wait1(pp + lane * kPartStride + HD + 1, tg + T_ATT_PART, err);
                }
                const float M = wave_max(ms);
                const float e = lane < nsplit ? expf(ms - M) : 0.f;
                const float Lsum = wave_sum(ls * e);
                float acc = 0.f;
#pragma unroll 1
                for (int sb = 0; sb < nsplit; sb += 16) {
                    uint64_t v[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k)
                        v[k] = sb + k < nsplit ? tload(pp + (sb + k) * kPartStride + lane)
                                               : (static_cast<uint64_t>(tg + T_ATT_PART) << 32);
                    unsigned spins = 0;
                    for (;;) {
                        bool ok = true;
#pragma unroll
                        for (int k = 0; k < 16; ++k) ok = ok && tagged(v[k], tg + T_ATT_PART);
                        if (ok || give_up(spins, err)) break;
#pragma unroll
                        for (int k = 0; k < 16; ++k)
                            if (sb + k < nsplit && !tagged(v[k], tg + T_ATT_PART))
                                v[k] = tload(pp + (sb + k) * kPartStride + lane);
                    }
#pragma unroll
                    for (int k = 0; k < 16; ++k)
                        if (sb + k < nsplit) acc = fmaf(tvalue(v[k]), __shfl(e, sb + k), acc);
                }
                tstore(tatt + h * HD + lane, acc / Lsum, tg + T_ATT);
            }
        }
        stamp(p, 1 + 6 * l + 2);

        // ---- wo + residual ----
        renew();
        {
            Row<WT> rw[kWoU];
#pragma unroll
            for (int i = 0; i < kWoU; ++i)
                if (gw + i * NW < H) load_row<WT>(Lw.wo, Lw.so, gw + i * NW, lane, rw[i]);
            fetch<H>(tatt, tg + T_ATT, big, err, tid);
            stamp_in(p, l, 3, 0);
            float xr[NX], xsum;
            lane_inputs<WT, false>(big, nullptr, 1.f, xr, xsum, lane);
            stamp_in(p, l, 3, 1);
#pragma unroll
            for (int i = 0; i < kWoU; ++i) {
                const int r = gw + i * NW;
                __builtin_amdgcn_sched_barrier(0);
                if (r < H) {
                    const float d = row_dot<WT>(rw[i], xr, xsum);
                    if (lane == 0) tstore(txa + r, xin[r] + d, tg + T_XA);
                }
            }
#pragma unroll 1
            for (int r = gw + kWoU * NW; r < H; r += NW) {
                load_row<WT>(Lw.wo, Lw.so, r, lane, rw[0]);
                const float d = row_dot<WT>(rw[0], xr, xsum);
                if (lane == 0) tstore(txa + r, xin[r] + d, tg + T_XA);
            }
        }
        stamp(p, 1 + 6 * l + 3);

        // ---- gate_up (+ ffn_norm prologue, SwiGLU); unit = gate row u and up row u + inter ----
        // PF units in flight per wave (a ring): each consumed slot is refilled with the unit PF ahead.
        renew();
        {
            constexpr int PF = WT == WType::BF16 ? 2 : WT == WType::INT8 ? 4 : kGuU;  // 16 KiB per wave
            Row<WT> rg[PF], ru[PF];
#pragma unroll
            for (int i = 0; i < PF; ++i) {
                const int u = gw + i * NW;
                if (u < INTER) {
                    load_row<WT>(Lw.wgu, Lw.sgu, u, lane, rg[i]);
                    load_row<WT>(Lw.wgu, Lw.sgu, u + INTER, lane, ru[i]);
                }
            }
            fetch<H>(txa, tg + T_XA, xa, err, tid);
            stamp_in(p, l, 4, 0);
            const float inv = rms_inv(xa, p.eps, scratch, tid);
            float xr[NX], xsum;
            lane_inputs<WT, true>(xa, Lw.ffn_norm, inv, xr, xsum, lane);
            stamp_in(p, l, 4, 1);
#pragma unroll
            for (int i = 0; i < kGuU; ++i) {
                const int u = gw + i * NW;
                __builtin_amdgcn_sched_barrier(0);
                if (u < INTER) {
                    const float gv = row_dot<WT>(rg[i % PF], xr, xsum);
                    const float uv = row_dot<WT>(ru[i % PF], xr, xsum);
                    if (lane == 0) tstore(tact + u, silu(gv) * uv, tg + T_ACT);
                }
                const int un = gw + (i + PF) * NW;
                if (i + PF < kGuU && un < INTER) {
                    load_row<WT>(Lw.wgu, Lw.sgu, un, lane, rg[i % PF]);
                    load_row<WT>(Lw.wgu, Lw.sgu, un + INTER, lane, ru[i % PF]);
                }
            }
#pragma unroll 1
            for (int u = gw + kGuU * NW; u < INTER; u += NW) {
                load_row<WT>(Lw.wgu, Lw.sgu, u, lane, rg[0]);
                load_row<WT>(Lw.wgu, Lw.sgu, u + INTER, lane, ru[0]);
                const float gv = row_dot<WT>(rg[0], xr, xsum);
                const float uv = row_dot<WT>(ru[0], xr, xsum);
                if (lane == 0) tstore(tact + u, silu(gv) * uv, tg + T_ACT);
            }
        }
        stamp(p, 1 + 6 * l + 4);

        // ---- down + residual (8192-wide rows, inputs read from LDS) ----
        renew();
        {
            constexpr int PD = WT == WType::BF16 ? 1 : kDownU;  // rows in flight (16 KiB per wave for bf16)
            DRow<WT> rd[PD];
#pragma unroll
            for (int i = 0; i < PD; ++i)
                if (gw + i * NW < H) load_drow<WT>(Lw.wd, Lw.sd, gw + i * NW, lane, rd[i]);
            fetch<INTER>(tact, tg + T_ACT, big, err, tid);
            stamp_in(p, l, 5, 0);
            auto finish = [&](int r, float d) {
                const float xn = xa[r] + d;
                tstore(txo + r, xn, tg + T_X);
                if (p.residuals) p.residuals[static_cast<size_t>(l + 1) * H + r] = xn;
            };
#pragma unroll
            for (int i = 0; i < PD; ++i) {
                const int r = gw + i * NW;
                if (r < H) {
                    const float d = drow_dot<WT>(rd[i], big, lane);
                    if (lane == 0) finish(r, d);
                }
            }
#pragma unroll 1
            for (int r = gw + PD * NW; r < H; r += NW) {
                load_drow<WT>(Lw.wd, Lw.sd, r, lane, rd[0]);
                const float d = drow_dot<WT>(rd[0], big, lane);
                if (lane == 0) finish(r, d);
            }
            __syncthreads();  // `big` is reused by the next layer's attention tiles
        }
        stamp(p, 1 + 6 * l + 5);
    }

    // ---- lm_head (+ final norm) with the argmax folded in; R rows per wave per step, double-buffered ----
    renew();
    {
        constexpr int R = 2;
        Row<WT> cur[R], nxt[R];
        const int step_rows = NW * R;
        int r0 = gw * R;
#pragma unroll
        for (int i = 0; i < R; ++i)
            if (r0 + i < VOCAB) load_row<WT>(p.emb, p.emb_s, r0 + i, lane, cur[i]);
        fetch<H>(p.tx + static_cast<size_t>(NL) * H, base + (NL - 1) * kTagStride + T_X, xin, err, tid);
        const float inv = rms_inv(xin, p.eps, scratch, tid);
        float xr[NX], xsum;
        lane_inputs<WT, true>(xin, p.final_norm, inv, xr, xsum, lane);
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll 1
        for (; r0 < VOCAB; r0 += step_rows) {
            const int rn = r0 + step_rows;
#pragma unroll
            for (int i = 0; i < R; ++i)
                if (rn + i < VOCAB) load_row<WT>(p.emb, p.emb_s, rn + i, lane, nxt[i]);
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int r = r0 + i;
                if (r < VOCAB) {
                    const float d = row_dot<WT>(cur[i], xr, xsum);
                    if (lane == 0) p.logits[r] = d;
                    if (arg_better(d, r, bv, bi)) {
                        bv = d;
                        bi = r;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < R; ++i) cur[i] = nxt[i];
        }
        if (lane == 0) {
            red_v[wave] = bv;
            red_i[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < kWaves; ++w)
                if (arg_better(red_v[w], red_i[w], bv, bi)) {
                    bv = red_v[w];
                    bi = red_i[w];
                }
            tstore(p.targ + 2 * blockIdx.x, bv, base + T_ARG);
            tstore(p.targ + 2 * blockIdx.x + 1, __builtin_bit_cast(float, bi), base + T_ARG);
        }
        __syncthreads();
    }
    stamp(p, 97);

    // ---- final argmax over the workgroups' partials (wave trees); token and position advance on device ----
    if (blockIdx.x == 0) {
        float v = -INFINITY;
        int i = 0x7fffffff;
        for (int g = tid; g < G; g += kThreads) {
            const float gv = wait1(p.targ + 2 * g, base + T_ARG, err);
            const int gi = __builtin_bit_cast(int, wait1(p.targ + 2 * g + 1, base + T_ARG, err));
            if (arg_better(gv, gi, v, i)) {
                v = gv;
                i = gi;
            }
        }
        wave_argmax(v, i);
        if (lane == 0) {
            red_v[wave] = v;
            red_i[wave] = i;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < kWaves; ++w)
                if (arg_better(red_v[w], red_i[w], v, i)) {
                    v = red_v[w];
                    i = red_i[w];
                }
            *p.d_token = min(max(i, 0), VOCAB - 1);
            *p.d_pos = pos + 1;
            *p.d_step = step + 1;
        }
        stamp(p, 98);
    }
}

}  // namespace dk

int decode_max_grid(WType wt) {
    int b = 0;
    switch (wt) {
        case WType::BF16:
            CLLM_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, dk::decode_kernel<WType::BF16>, kDecodeThreads, 0));
            break;
        case WType::INT8:
            CLLM_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, dk::decode_kernel<WType::INT8>, kDecodeThreads, 0));
            break;
        case WType::INT4:
            CLLM_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, dk::decode_kernel<WType::INT4>, kDecodeThreads, 0));
            break;
    }
    return b * device_cu_count();
}

void launch_decode(WType wt, const DecodeParams& p, int grid, hipStream_t s) {
    CLLM_REQUIRE(grid > 0 && grid <= 4096, "decode: bad grid");
    CLLM_REQUIRE(p.max_seq > 0 && p.max_seq % kAttnChunk == 0 && p.max_seq <= 64 * kAttnChunk,
                 "decode: max_seq must be a multiple of 128 and at most 8192");
    switch (wt) {
        case WType::BF16:
            hipLaunchKernelGGL(dk::decode_kernel<WType::BF16>, dim3(grid), dim3(kDecodeThreads), 0, s, p);
            break;
        case WType::INT8:
            hipLaunchKernelGGL(dk::decode_kernel<WType::INT8>, dim3(grid), dim3(kDecodeThreads), 0, s, p);
            break;
        case WType::INT4:
            hipLaunchKernelGGL(dk::decode_kernel<WType::INT4>, dim3(grid), dim3(kDecodeThreads), 0, s, p);
            break;
    }
    CLLM_HIP(hipGetLastError());
}

}  // namespace cllm
