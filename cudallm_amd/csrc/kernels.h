// Host-side launch functions of the gfx950 kernels.  Each validates the shapes its kernel and
// grid assume before launching (a wrong shape becomes an ArgError, never a device fault).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace cllm {

constexpr int kAttnChunk = 128;    // tokens per split-K attention chunk
constexpr int kArgmaxParts = 256;  // partial results of the two-pass argmax

struct MatvecArgs {
    const void* w;
    const void* scales;
    const float* x;
    const float* norm_w;  // non-null when the RMSNorm prologue is fused
    float eps;
    float* y;
    int rows, cols;
};

// rpb of the fast matvec when the caller passes 0 (per weight type and shape).
int default_rpb(WType wt, Epilogue ep, int rows, int cols);
// Workgroups per CU in the standalone matvec's grid for that shape class (0: as many as can be resident).
int grid_per_cu(WType wt, Epilogue ep, int rows, int cols);
// Events the next matvec launch on this thread records at its kernel's start and end (benchmarks: the interval
// excludes the launch gap).  take_kernel_events() returns and clears them.
struct KernelEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
void arm_kernel_events(hipEvent_t start, hipEvent_t stop);
KernelEvents take_kernel_events();
// y (= | +=) W x^ with the selected epilogue; x^ = rmsnorm(x) * norm_w when norm_w != null.
void launch_matvec(WType wt, Epilogue ep, const MatvecArgs& a, int rpb, hipStream_t s);
// One thread per row, bf16, STORE only: the deliberately uncoalesced ablation baseline.
void launch_matvec_naive(const MatvecArgs& a, hipStream_t s);

void launch_rmsnorm(const float* x, const float* w, float eps, float* y, int n, hipStream_t s);
void launch_add_inplace(float* x, const float* y, int n, hipStream_t s);
void launch_silu_mul(const float* gu, float* act, int inter, hipStream_t s);
void launch_set_token(int* d_token, int token, hipStream_t s);
void launch_embedding(WType wt, const void* w, const void* scales, const int* d_token, float* x, int hidden,
                      int vocab, int group_size, hipStream_t s);

// RoPE on the q (and k) heads of qkv = [q(nh*hd) | k(nkv*hd) | v(nkv*hd)] at position *d_pos.
// fused: q rotated in place, rotated k and v written to the fp16 caches (k in qkv left as is).
void launch_rope_kv_fused(float* qkv, const float* inv_freq, uint16_t* k_cache, uint16_t* v_cache, const int* d_pos,
                          int nh, int nkv, int hd, int max_seq, hipStream_t s);
void launch_rope_inplace(float* qkv, const float* inv_freq, const int* d_pos, int nh, int nkv, int hd, hipStream_t s);
void launch_kv_write(const float* qkv, uint16_t* k_cache, uint16_t* v_cache, const int* d_pos, int nh, int nkv,
                     int hd, int max_seq, hipStream_t s);

// Split-K GQA decode attention over ctx = *d_pos + 1 tokens of the fp16 caches [nkv][max_seq][hd].
void launch_attention_splitk(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* d_pos,
                             float* part_o, float* part_ml, float* out, int nh, int nkv, int hd, int max_seq,
                             hipStream_t s);
// The same split-K attention with its partials in a static device array of kStaticAttnSlots slots
// (nh * max_seq / 128 <= 8192): no allocation on any call (the array's address on a device is resolved on the first
// call there).  Calls that overlap on one device share that array and race.
constexpr int kStaticAttnSlots = 8192;
void launch_attention_splitk_static(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* d_pos,
                                    float* out, int nh, int nkv, int hd, int max_seq, hipStream_t s);
void launch_attention_naive(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* d_pos,
                            float* out, int nh, int nkv, int hd, int max_seq, hipStream_t s);

// Deterministic argmax (ties -> lowest index); writes *d_token and advances *d_pos by one.
void launch_argmax(const float* logits, int n, float* part_v, int* part_i, int* d_token, int* d_pos, hipStream_t s);

// Weight quantisers (bit-identical to the numpy definitions).
void launch_quantize_int8_rows(const float* w, int rows, int cols, int8_t* q, float* scales, hipStream_t s);
void launch_quantize_int4_groups(const float* w, int rows, int cols, uint8_t* packed, uint16_t* scales, hipStream_t s);
void launch_unpack_int4(const uint8_t* packed, int rows, int cols, int8_t* q, hipStream_t s);

int device_cu_count();

// Stream-read bandwidth of device memory over a `bytes` buffer: best and median GB/s of `reps` timed reads
// for the best of a few launch shapes (the read peak the roofline fractions are also quoted against).
struct ReadBandwidth {
    double best_gbps = 0, median_gbps = 0;
    int blocks_per_cu = 0, loads_in_flight = 0;
};
ReadBandwidth measure_read_bandwidth(size_t bytes, int reps);
// One stream read of `bytes` at `src` (the bandwidth kernel: blocks_per_cu x CUs workgroups, 8 loads in flight per
// thread; sink: blocks_per_cu x CUs words, written only for a value the data never holds in practice).  Records the
// armed kernel events, like launch_matvec.
void launch_stream_read(const void* src, size_t bytes, int blocks_per_cu, unsigned* sink, size_t sink_words,
                        hipStream_t s);

}  // namespace cllm
