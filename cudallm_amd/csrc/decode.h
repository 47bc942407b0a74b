// Parameters of the persistent decode-step kernel (shared by host and device code).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace cllm {

// Per-layer weight pointers, kept in device memory.
struct DecodeLayer {
    const float* attn_norm;
    const void* wqkv;
    const void* sqkv;
    const void* wo;
    const void* so;
    const float* ffn_norm;
    const void* wgu;
    const void* sgu;
    const void* wd;
    const void* sd;
};

// Tagged vectors: every element is a 64-bit word (fp32 value in the low half, the epoch tag of
// the phase that produced it in the high half), written and read with relaxed agent-scope 64-bit
// atomics.  A reader waits for the tag of the current phase, so one read both synchronises with
// the producing workgroup and delivers the value.
struct DecodeParams {
    const DecodeLayer* layers;
    const void* emb;
    const void* emb_s;
    const float* inv_freq;
    const float* final_norm;
    uint16_t* k_cache;  // fp16 [layer][kv_head][max_seq][head_dim]
    uint16_t* v_cache;
    int max_seq;
    uint64_t* tx;    // [n_layers + 1][hidden]  residual stream at each layer input (index l+1 = after layer l)
    uint64_t* txa;   // [n_layers][hidden]      residual after the attention block
    uint64_t* tqkv;  // [n_layers][3072]        q|k (rotated) | v
    uint64_t* tatt;  // [n_layers][2048]        attention output
    uint64_t* tpart; // [n_layers][32][max_seq/128][66]  split partials: o[64], m, l
    uint64_t* tact;  // [n_layers][inter]       SwiGLU output
    uint64_t* targ;  // [grid][2]               per-workgroup argmax (value, index)
    float* logits;
    int* d_token;
    int* d_pos;
    unsigned* d_step;  // launch counter: epoch base of the tags, never reset
    unsigned* d_err;   // sticky: set when a wait exceeded its bound
    float* residuals;  // optional [(n_layers + 1) * hidden] snapshots (step_debug)
    unsigned long long* stamps;  // optional [grid][kStampSlots] phase-end timestamps (100 MHz clock)
    float eps;
    // Timing perturbation for tests, 0 in normal use (the CUDALLM_STALL environment variable): bit k
    // (kStall*) makes each workgroup's compute waves sleep about 13 us before that phase waits for its
    // input, kStallLoader makes each loader wave sleep at every segment switch, and kStallOdd limits
    // the sleeps to odd workgroups.  Results must stay bit-identical under any mask.
    unsigned stall;
    // Co-residency probe (engine set-up only, null in a decode step): every workgroup adds 1 to probe[0] and waits,
    // with a bound, until all gridDim.x have arrived; a workgroup that gives up sets probe[1].  Nothing else runs.
    unsigned* probe;
};

enum : unsigned {
    kStallQkv = 1u << 0,
    kStallAttn = 1u << 1,
    kStallWo = 1u << 2,
    kStallGateUp = 1u << 3,
    kStallDown = 1u << 4,
    kStallLmHead = 1u << 5,
    kStallLoader = 1u << 6,
    kStallOdd = 1u << 7,
    kStallInputs = 1u << 8,  // after a phase's input barrier, before the waves read the input from LDS
    kStallWave0 = 1u << 9,   // only compute wave 0 of a selected workgroup sleeps (skew inside the workgroup)
};

// Timestamp slots per workgroup: 0 = start, 1 + 6 l + k = end of phase k of layer l
// (k: 0 qkv, 1 attention, 2 split merge, 3 wo, 4 gate_up, 5 down), 97 = lm_head end,
// 98 = final argmax end (workgroup 0 only); for layer 1, 100 + 2 k = phase k's input arrived and
// 101 + 2 k = its prologue done.
constexpr int kStampSlots = 128;

constexpr int kDecodeThreads = 512;  // 4 compute waves + 4 loader waves
// Grid bounds of the decode kernel: each compute wave keeps the residual inputs of its wo/down rows in
// LDS for at most 8 rows (2048 rows over >= 64 x 4 waves).
// The loader's row walk needs NW = 4 * grid to be a multiple of 32 (grid % 8 == 0).
constexpr int kDecodeMinGrid = 64, kDecodeMaxGrid = 4096;
// Longest context of the decode kernel (Llama-3.2's 131072 positions): 1024 attention splits.
constexpr int kDecodeMaxSeq = 131072;
// Tags are (step + 1) * 256 + layer * 8 + phase in 32 bits, so the step counter must stay below 2^24 - 1.  The
// host clears every tagged buffer and restarts the counter before it gets there.
constexpr unsigned kDecodeStepLimit = (1u << 24) - 2;

// Enqueue one decode step: one plain launch of `grid` workgroups, which must all be co-resident (the engine checks
// that once with a probe launch, decode_grid_is_resident; every cross-workgroup wait is bounded besides).
void launch_decode(WType wt, const DecodeParams& p, int grid, hipStream_t s);
// Launches the decode kernel in probe mode with `grid` workgroups and reports whether all of them were resident at
// once.  `probe` is two zeroed device words.
bool decode_grid_is_resident(WType wt, const DecodeParams& p, int grid, unsigned* probe, hipStream_t s);
// Workgroups of the decode kernel that fit on the device at once for this weight type.
int decode_max_grid(WType wt);

}  // namespace cllm
