// Batch-1 weight-streaming matvec for gfx950 (wave64), included by one translation unit per weight
// type.  Behaviour follows reference src/kernels/matvec_opt.cu:43-157 (y = W x^ with an fp32
// accumulator, optional fused RMSNorm prologue, STORE / ADD / SWIGLU epilogue, int8 scale per row,
// int4 fp16 scale per 128 columns); the work decomposition is this file's own:
//
//  * A workgroup is 4 waves.  Columns are cut into 2048-wide slices; KS = cols/2048 waves share
//    one row (one slice each), so the 4 waves of a workgroup cover 4/KS row groups.
//  * Every lane owns a fixed set of 32 columns of its slice: the 16-byte chunks lane, lane+64, ...
//    (8 bf16 / 16 int8 / 32 int4 columns per chunk).  Those 32 inputs - normalised when the norm
//    is fused - are loaded ONCE into VGPRs and reused for every row the wave touches, so the inner
//    loop reads no LDS at all: only 128-bit non-temporal weight loads, 64 lanes x 16 B = 1 KiB
//    contiguous per load instruction.
//  * R rows (rpb) are loaded before any is consumed, for R x (4 KiB bf16 | 2 KiB int8 | 1 KiB int4)
//    of loads per pass; a wave issues the next pass's loads before it multiplies the current one,
//    so up to 2R rows are in flight.  The first pass's weights are requested right after the lane's
//    inputs, before the norm and digit prologue.  No load sits under a branch (rows past the end
//    re-read the last row) and, with KS = 1, no store sits in the loop (each wave's row sums wait in
//    its lanes until its last pass): either made the compiler's wait counts conservative, so that a
//    pass also waited for the next pass's loads.  Measured on MI355X against the earlier form: lm_head
//    bf16 82.5 -> 80.0 us, int8 44.6 -> 40.5 us, int4 32.2 -> 28.0 us; bf16 and int8 lm_head then run
//    within 1 % of a plain stream read of the same bytes.
//  * Quantised 2048-wide rows (KS = 1) use integer digit dots: each lane turns its 32 inputs into
//    fixed-point digit words once (one scale per wave from max |x^|, the same in every wave since each
//    covers the whole row), and a row then costs 24 v_dot8_i32_i4 / v_dot4_i32_i8 per lane instead of
//    a conversion and an FMA per column.  The 8192-wide down rows (KS = 4) keep the float path.
//  * Row sums are wave64 DPP butterflies (deterministic order); with KS > 1 the slice partials
//    meet in LDS and are added in slice order.  No atomics anywhere.
//  * The grid: min(row blocks, CUs x the shape class's workgroups per CU (grid_per_cu; by default as
//    many as can be resident)), but with KS = 1 at least enough workgroups that none takes more than
//    64 / R passes.
//
// Widths with cols % 2048 != 0 or cols/2048 not in {1,4} use matvec_generic, which stages x in LDS.
#pragma once

#include <algorithm>

#include <hip/hip_ext.h>

#include "../kernels.h"
#include "device.h"
#include "digits.h"
#include "dot.h"

namespace cllm {
namespace mv {

constexpr int kSlice = 2048;
constexpr int kThreads = 256;
// Passes of R rows per wave with KS = 1: the wave's row sums wait in its 64 lanes until the end.
template <int R>
constexpr int kMaxPasses = kWave / R;

template <Epilogue EP>
__device__ __forceinline__ void store_out(float* y, int r, float d, float du) {
    if constexpr (EP == Epilogue::STORE) {
        y[r] = d;
    } else if constexpr (EP == Epilogue::ADD) {
        y[r] = y[r] + d;
    } else {
        y[r] = silu(d) * du;
    }
}

template <WType WT, Epilogue EP, bool NORM, int KS, int R>
__global__ void __launch_bounds__(kThreads) matvec_fast(MatvecArgs a) {
    using F = Fmt<WT>;
    constexpr int NX = F::CPL * F::CPC;  // 32 inputs per lane
    constexpr int GROUPS = 4 / KS;
    constexpr int ROWS_WG = GROUPS * R;
    constexpr bool GLU = EP == Epilogue::SWIGLU;
    constexpr int NP = GLU ? 2 : 1;
    constexpr bool DIG = WT != WType::BF16 && KS == 1;
    __shared__ float scratch[16];
    __shared__ float part[KS > 1 ? KS * ROWS_WG * NP : 1];

    const int tid = threadIdx.x;
    // The wave index through readfirstlane: the compiler then knows it is uniform, so every row index and weight
    // address derived from it is computed once per wave in scalar registers instead of in every lane.
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
    const int slice = wave % KS, grp = wave / KS;
    const int out_rows = GLU ? a.rows / 2 : a.rows;
    // Row blocks are dealt to the workgroups in turn; base is the same for every wave of a workgroup, so the
    // barriers below (block_sum, and pass() with KS > 1) are reached by all of them.
    const int stride = gridDim.x * ROWS_WG;
    int base = blockIdx.x * ROWS_WG;
    if (base >= out_rows) return;
    int left = (out_rows - base + stride - 1) / stride;  // passes of this workgroup, >= 1

    // The lane's 32 inputs (and norm weights) are requested first, then the first pass's weights, so that the
    // prologue below waits only for the short input loads while the weight bytes are already in flight (loads
    // complete in order, so requesting the weights first would make the prologue wait for them).
    f32x4 xin[NX / 4], nwin[NORM ? NX / 4 : 1];
#pragma unroll
    for (int k = 0; k < F::CPL; ++k) {
        const int c0 = slice * kSlice + (k * kWave + lane) * F::CPC;
#pragma unroll
        for (int j = 0; j < F::CPC; j += 4) {
            xin[(k * F::CPC + j) / 4] = *reinterpret_cast<const f32x4*>(a.x + c0 + j);
            if constexpr (NORM) nwin[(k * F::CPC + j) / 4] = *reinterpret_cast<const f32x4*>(a.norm_w + c0 + j);
        }
    }
    const size_t rb = row_bytes<WT>(a.cols);
    // Addresses are a row base that is uniform across the wave (scalar registers) plus a 32-bit lane offset, the
    // form of a load with a scalar base: one offset register per lane instead of a 64-bit address per row.
    const char* wbase = static_cast<const char*>(a.w);
    const uint32_t woff = static_cast<uint32_t>(slice * (kSlice * 16 / F::CPC) + lane * 16);
    const int groups_per_row = a.cols / 128;
    // int4: one 128-column group per lane; lanes 4g..4g+3 share scale g of the slice.
    const uint16_t* sbase = static_cast<const uint16_t*>(a.scales);
    const uint32_t soff = static_cast<uint32_t>(slice * (kSlice / 128) + lane / 4);

    // The R rows of one pass: weight chunks and, for int4, the lane's group scales.  Two of these alternate, so the
    // next pass's loads are in flight while this pass is multiplied.
    struct Block {
        u32x4 v[R][F::CPL];
        u32x4 vu[GLU ? R : 1][F::CPL];
        uint16_t g[R], gu[R];
    };
    // Rows past the end load the last row again (their sums are never stored): with no branch around the loads the
    // compiler counts them exactly, so a pass waits only for its own loads and not for the next pass's as well.
    auto load = [&](Block& b, int r0) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int rc = min(r0 + i, out_rows - 1);
            const char* row = wbase + static_cast<size_t>(rc) * rb;
            const char* row_u = wbase + static_cast<size_t>(rc + out_rows) * rb;
#pragma unroll
            for (int k = 0; k < F::CPL; ++k) {
                b.v[i][k] = load_stream(row + woff + k * 1024);
                if constexpr (GLU) b.vu[i][k] = load_stream(row_u + woff + k * 1024);
            }
            if constexpr (WT == WType::INT4) {
                b.g[i] = gload(sbase + static_cast<size_t>(rc) * groups_per_row + soff);
                if constexpr (GLU) b.gu[i] = gload(sbase + static_cast<size_t>(rc + out_rows) * groups_per_row + soff);
            }
        }
    };
    Block A, B;
    load(A, base + grp * R);
    __builtin_amdgcn_sched_barrier(0);  // keep the weight loads ahead of the prologue

    // RMSNorm: with KS = 1 every wave holds the whole row (64 lanes x 32 columns), so a wave sum gives the sum of
    // squares; with KS > 1 the workgroup's waves hold one slice each.
    float inv = 1.f;
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < NX / 4; ++q)
            ss += xin[q][0] * xin[q][0] + xin[q][1] * xin[q][1] + xin[q][2] * xin[q][2] + xin[q][3] * xin[q][3];
        ss = KS == 1 ? wave_sum(ss) : block_sum(ss, scratch);
        inv = rsqrtf(ss / static_cast<float>(a.cols) + a.eps);
    }
    float xr[NX];
    float xsum = 0.f;
#pragma unroll
    for (int q = 0; q < NX / 4; ++q) {
        f32x4 v = xin[q];
        if constexpr (NORM) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = v[e] * inv * nwin[q][e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xr[4 * q + e] = v[e];
            xsum += v[e];
        }
    }

    // Digit words of the lane's inputs in its weight words' layout: int8 digit k of chunk c, word t (columns
    // 4t .. 4t + 3) at dg[(2k + c) 4 + t]; int4 digit k of word t (columns 8t .. 8t + 7) at dg[4k + t].
    [[maybe_unused]] uint32_t dg[DIG ? 24 : 1];
    [[maybe_unused]] float dsc = 1.f;
    if constexpr (DIG) {
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < NX; ++j) m = fmaxf(m, fabsf(xr[j]));
        const int e = dig_exponent(wave_max(m));
        dsc = ldexpf(1.f, -e);
        const float scale = ldexpf(1.f, e);
        if constexpr (WT == WType::INT8) {
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float* xc = xr + c * 16 + 4 * t;
                    uint32_t P[3];
                    byte_planes(fixed_word(xc[0], scale, 0x808080u), fixed_word(xc[1], scale, 0x808080u),
                                fixed_word(xc[2], scale, 0x808080u), fixed_word(xc[3], scale, 0x808080u), P);
#pragma unroll
                    for (int k = 0; k < 3; ++k) dg[(2 * k + c) * 4 + t] = P[k] ^ 0x80808080u;
                }
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t u[8], w[6];
#pragma unroll
                for (int b = 0; b < 8; ++b) u[b] = fixed_word(xr[8 * t + b], scale, 0x888888u);
                nibble_words(u, w);
#pragma unroll
                for (int k = 0; k < 6; ++k) dg[4 * k + t] = w[k] ^ 0x88888888u;
            }
        }
    }

    // KS = 1: the row sums wait in lanes (lane j: the wave's j-th row) and are stored after the last pass, so no store
    // sits in the loop (a store there made the loop's head wait for the previous pass's loads).  The host keeps every
    // wave within kMaxPasses<R> passes, so 64 lanes hold them all.
    [[maybe_unused]] float acc = 0.f, acc_u = 0.f;
    [[maybe_unused]] int acc_row = -1, held = 0;
    auto pass = [&](const Block& b, int base) {
        const int r0 = base + grp * R;
        float d[R], du[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if constexpr (DIG) {
                // Per lane: int8 sum_k 256^k sum(q d_k); int4 sum_k 16^k sum(q d_k) (nibble u = q + 8, so q = u xor 8)
                // times the lane's group scale.  The row's sum times 2^-e (and the int8 row scale at the store).
                auto dot = [&](const u32x4* v, uint16_t g) {
                    if constexpr (WT == WType::INT8) {
                        int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
                        for (int c = 0; c < 2; ++c)
#pragma unroll
                            for (int t = 0; t < 4; ++t) {
                                const int w = static_cast<int>(v[c][t]);
                                a0 = __builtin_amdgcn_sdot4(w, static_cast<int>(dg[(0 + c) * 4 + t]), a0, false);
                                a1 = __builtin_amdgcn_sdot4(w, static_cast<int>(dg[(2 + c) * 4 + t]), a1, false);
                                a2 = __builtin_amdgcn_sdot4(w, static_cast<int>(dg[(4 + c) * 4 + t]), a2, false);
                            }
                        return fmaf(fmaf(static_cast<float>(a2), 256.f, static_cast<float>(a1)), 256.f, static_cast<float>(a0));
                    } else {
                        int ac[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            const int w = static_cast<int>(v[0][t] ^ 0x88888888u);
#pragma unroll
                            for (int k = 0; k < 6; ++k) ac[k] = __builtin_amdgcn_sdot8(w, static_cast<int>(dg[4 * k + t]), ac[k], false);
                        }
                        const int p0 = ac[0] + 16 * ac[1], p1 = ac[2] + 16 * ac[3], p2 = ac[4] + 16 * ac[5];
                        return fmaf(static_cast<float>(p2), 65536.f, static_cast<float>(p0 + 256 * p1)) * half_bits_to_float(g);
                    }
                };
                d[i] = dot(b.v[i], b.g[i]);
                du[i] = 0.f;
                if constexpr (GLU) du[i] = dot(b.vu[i], b.gu[i]);
            } else {
                float s = 0.f, su = 0.f;
#pragma unroll
                for (int k = 0; k < F::CPL; ++k) {
                    s += chunk_dot<WT>(b.v[i][k], xr + k * F::CPC);
                    if constexpr (GLU) su += chunk_dot<WT>(b.vu[i][k], xr + k * F::CPC);
                }
                if constexpr (WT == WType::INT8) {
                    s -= kBias<WT> * xsum;
                    if constexpr (GLU) su -= kBias<WT> * xsum;
                }
                if constexpr (WT == WType::INT4) {
                    s = half_bits_to_float(b.g[i]) * (s - 8.f * xsum);
                    if constexpr (GLU) su = half_bits_to_float(b.gu[i]) * (su - 8.f * xsum);
                }
                d[i] = s;
                du[i] = su;
            }
        }
        // Lane l: the sums of row r0 + (l mod R) (times 2^-e for the digit dots).  int4's 2048-wide rows (1 KiB, the
        // most rows per byte) reduce all R rows at once (rows_sum: int4 lm_head 28.2 -> 26.2 us, gate_up 8.0 -> 7.3 us
        // on MI355X); the other forms keep a full reduction per row, which measured as fast or faster for them (bf16
        // down 7.3 against 8.4 us).
        float tot = 0.f, tot_u = 0.f;
        if constexpr (WT == WType::INT4 && KS == 1) {
            tot = rows_sum<R>(d, lane);
            if constexpr (GLU) tot_u = rows_sum<R>(du, lane);
        } else {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const float si = wave_sum(d[i]);
                const float sui = GLU ? wave_sum(du[i]) : 0.f;
                if (lane % R == i) {
                    tot = si;
                    tot_u = sui;
                }
            }
        }
        if constexpr (DIG) {
            tot *= dsc;
            tot_u *= dsc;
        }

        if constexpr (KS == 1) {
            // Lane held + i keeps row r0 + i until the wave's last pass (no store inside the loop); held is a multiple
            // of R, so that lane already holds row i's sum.
            if (lane >= held && lane < held + R) {
                acc = tot;
                acc_u = tot_u;
                acc_row = r0 + lane - held;
            }
            held += R;
        } else {
            // Lane i (< R) holds row r0 + i.
            const float mine = tot, mine_u = tot_u;
            if (lane < R) {
                const int slot = (slice * ROWS_WG + grp * R + lane) * NP;
                part[slot] = mine;
                if constexpr (GLU) part[slot + 1] = mine_u;
            }
            __syncthreads();
            if (tid < ROWS_WG && base + tid < out_rows) {
                const int r = base + tid;
                float s = 0.f, su = 0.f;
#pragma unroll
                for (int q = 0; q < KS; ++q) {
                    s += part[(q * ROWS_WG + tid) * NP];
                    if constexpr (GLU) su += part[(q * ROWS_WG + tid) * NP + 1];
                }
                if constexpr (WT == WType::INT8) {
                    const float* sc = static_cast<const float*>(a.scales);
                    s *= sc[r];
                    if constexpr (GLU) su *= sc[r + out_rows];
                }
                store_out<EP>(a.y, r, s, su);
            }
            __syncthreads();
        }
    };

    // One pass's loads are outstanding at the top of each half; the next pass is requested before this one is
    // multiplied.  No load sits under a branch, so each pass waits only for its own loads.
    for (;;) {
        if (left == 1) {
            pass(A, base);
            break;
        }
        load(B, base + stride + grp * R);
        __builtin_amdgcn_sched_barrier(0);  // issue the next pass's loads before this pass's math
        pass(A, base);
        base += stride;
        --left;
        if (left == 1) {
            pass(B, base);
            break;
        }
        load(A, base + stride + grp * R);
        __builtin_amdgcn_sched_barrier(0);
        pass(B, base);
        base += stride;
        --left;
    }
    if constexpr (KS == 1) {
        if (lane < held && acc_row < out_rows) {
            if constexpr (WT == WType::INT8) {
                const float* sc = static_cast<const float*>(a.scales);
                acc *= sc[acc_row];
                if constexpr (GLU) acc_u *= sc[acc_row + out_rows];
            }
            store_out<EP>(a.y, acc_row, acc, acc_u);
        }
    }
}

// Any cols that is a multiple of 1024 (up to 12288): x^ staged in LDS, one wave per row.
template <WType WT, Epilogue EP, bool NORM>
__global__ void __launch_bounds__(kThreads) matvec_generic(MatvecArgs a) {
    using F = Fmt<WT>;
    extern __shared__ float xs[];
    __shared__ float scratch[16];
    constexpr bool GLU = EP == Epilogue::SWIGLU;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int out_rows = GLU ? a.rows / 2 : a.rows;
    float inv = 1.f;
    if constexpr (NORM) {
        float ss = 0.f;
        for (int j = tid; j < a.cols; j += kThreads) ss += a.x[j] * a.x[j];
        ss = block_sum(ss, scratch);
        inv = rsqrtf(ss / static_cast<float>(a.cols) + a.eps);
    }
    for (int j = tid; j < a.cols; j += kThreads) xs[j] = NORM ? a.x[j] * inv * a.norm_w[j] : a.x[j];
    __syncthreads();

    const size_t rb = row_bytes<WT>(a.cols);
    const int nchunk = a.cols / F::CPC;
    const int groups_per_row = a.cols / 128;
    for (int r = blockIdx.x * 4 + wave; r < out_rows; r += gridDim.x * 4) {
        float s = 0.f, su = 0.f;
        for (int c = lane; c < nchunk; c += kWave) {
            const float* x = xs + c * F::CPC;
            const char* p = static_cast<const char*>(a.w) + static_cast<size_t>(r) * rb + c * 16;
            float t = chunk_dot<WT>(load_stream(p), x);
            float tu = GLU ? chunk_dot<WT>(load_stream(p + static_cast<size_t>(out_rows) * rb), x) : 0.f;
            if constexpr (WT != WType::BF16) {
                float xsum = 0.f;
#pragma unroll
                for (int j = 0; j < F::CPC; ++j) xsum += x[j];
                t -= kBias<WT> * xsum;
                if constexpr (GLU) tu -= kBias<WT> * xsum;
            }
            if constexpr (WT == WType::INT4) {
                const uint16_t* sc = static_cast<const uint16_t*>(a.scales);
                const int gi = c * F::CPC / 128;
                t *= half_bits_to_float(sc[static_cast<size_t>(r) * groups_per_row + gi]);
                if constexpr (GLU) tu *= half_bits_to_float(sc[static_cast<size_t>(r + out_rows) * groups_per_row + gi]);
            }
            s += t;
            su += tu;
        }
        s = wave_sum(s);
        su = GLU ? wave_sum(su) : 0.f;
        if (lane == 0) {
            if constexpr (WT == WType::INT8) {
                const float* sc = static_cast<const float*>(a.scales);
                s *= sc[r];
                if constexpr (GLU) su *= sc[r + out_rows];
            }
            store_out<EP>(a.y, r, s, su);
        }
    }
}

// Launches a matvec kernel; when the thread has armed kernel events (arm_kernel_events), the dispatch itself
// records them at the kernel's start and end, so a benchmark times the kernel without the launch gap.
template <typename K>
void dispatch(K kernel, int grid, size_t smem, hipStream_t s, const MatvecArgs& a) {
    KernelEvents ev = take_kernel_events();
    if (ev.start)
        hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), static_cast<uint32_t>(smem), s, ev.start, ev.stop, 0u, a);
    else
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), smem, s, a);
    CLLM_HIP(hipGetLastError());
}

template <typename K>
int resident_blocks(K kernel, size_t smem) {
    int b = 0;
    CLLM_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, kernel, kThreads, smem));
    CLLM_INTERNAL(b > 0, "matvec kernel cannot be resident");
    return b;
}

template <WType WT, Epilogue EP, bool NORM, int KS, int R>
void launch_fast(const MatvecArgs& a, hipStream_t s) {
    auto k = matvec_fast<WT, EP, NORM, KS, R>;
    static const int occ = resident_blocks(k, 0);
    const int out_rows = EP == Epilogue::SWIGLU ? a.rows / 2 : a.rows;
    constexpr int ROWS_WG = (4 / KS) * R;
    const int need = (out_rows + ROWS_WG - 1) / ROWS_WG;
    // Workgroups per CU: the shape class's choice, else as many as can be resident; but with KS = 1 no workgroup may
    // take more than kMaxPasses<R> passes.
    const int per_cu = grid_per_cu(WT, EP, a.rows, a.cols);
    const int grid = std::max(std::min(need, device_cu_count() * (per_cu > 0 ? per_cu : occ)),
                              KS == 1 ? (need + kMaxPasses<R> - 1) / kMaxPasses<R> : 0);
    dispatch(k, grid, 0, s, a);
}

template <WType WT, Epilogue EP, bool NORM>
void launch_generic(const MatvecArgs& a, hipStream_t s) {
    auto k = matvec_generic<WT, EP, NORM>;
    const size_t smem = static_cast<size_t>(a.cols) * sizeof(float);
    const int occ = resident_blocks(k, smem);
    const int out_rows = EP == Epilogue::SWIGLU ? a.rows / 2 : a.rows;
    const int grid = std::min((out_rows + 3) / 4, device_cu_count() * occ);
    dispatch(k, grid, smem, s, a);
}

template <WType WT, Epilogue EP, bool NORM, int KS>
void pick_r(int rpb, const MatvecArgs& a, hipStream_t s) {
    switch (rpb) {
        case 1: return launch_fast<WT, EP, NORM, KS, 1>(a, s);
        case 2: return launch_fast<WT, EP, NORM, KS, 2>(a, s);
        case 4: return launch_fast<WT, EP, NORM, KS, 4>(a, s);
        case 8: return launch_fast<WT, EP, NORM, KS, 8>(a, s);
    }
    throw ArgError("matvec: rpb must be 1, 2, 4 or 8");
}

template <WType WT, Epilogue EP, bool NORM>
void pick_shape(int rpb, const MatvecArgs& a, hipStream_t s) {
    if (a.cols == 2048) return pick_r<WT, EP, NORM, 1>(rpb, a, s);
    if (a.cols == 8192) return pick_r<WT, EP, NORM, 4>(rpb, a, s);
    return launch_generic<WT, EP, NORM>(a, s);
}

template <WType WT>
void launch_wt(Epilogue ep, const MatvecArgs& a, int rpb, hipStream_t s) {
    const bool norm = a.norm_w != nullptr;
    switch (ep) {
        case Epilogue::STORE:
            return norm ? pick_shape<WT, Epilogue::STORE, true>(rpb, a, s) : pick_shape<WT, Epilogue::STORE, false>(rpb, a, s);
        case Epilogue::ADD:
            return norm ? pick_shape<WT, Epilogue::ADD, true>(rpb, a, s) : pick_shape<WT, Epilogue::ADD, false>(rpb, a, s);
        case Epilogue::SWIGLU:
            return norm ? pick_shape<WT, Epilogue::SWIGLU, true>(rpb, a, s) : pick_shape<WT, Epilogue::SWIGLU, false>(rpb, a, s);
    }
    throw ArgError("matvec: bad epilogue");
}

}  // namespace mv

template <WType WT>
void launch_matvec_wt(Epilogue ep, const MatvecArgs& a, int rpb, hipStream_t s);

}  // namespace cllm
