// Batch-1 decode engine: owns the weights, the activations, the fp16 KV cache and the decode step.
//
// Two ways to run a step:
//  * the persistent decode kernel (decode.h), one launch per token, for the default
//    options (opt matvec, opt attention, fused);
//  * the multi-kernel step, for the reference's ablation options: a fixed program of kernel
//    launches built once at construction, replayed from a captured hipGraph when cuda_graph is set.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "decode.h"
#include "kernels.h"
#include "weights.h"

namespace cllm {

struct EngineOptions {
    int matvec = 1;        // 0 naive, 1 opt
    int attn = 1;          // 0 naive, 1 split-K
    bool fuse = true;
    bool graph = true;
    int max_seq_len = 0;   // 0 = file value
    int matvec_rpb = 0;    // 0 = default per weight type
};

// The option rules of reference src/engine/engine.cpp:10-21, plus max_seq_len <= the file's value.
void validate_options(const EngineOptions& o, const ModelConfig& c);

// Layout of cudallm_step_trace's output, in floats: the residual stream at every layer boundary, then per
// layer the vectors the persistent kernel exchanges between its phases.
struct TraceLayout {
    size_t residuals, qkv, att, xa, act, total;
    static TraceLayout of(const ModelConfig& c);
};

class Engine {
public:
    Engine(const std::string& path, const EngineOptions& opts);
    ~Engine();
    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;

    const ModelConfig& config() const { return weights_->config(); }
    const EngineOptions& options() const { return opts_; }
    int max_seq() const { return max_seq_; }
    uint64_t weight_bytes() const { return weights_->weight_bytes(); }
    int pos() const { return host_pos_; }
    bool persistent() const { return persistent_; }
    int grid() const { return grid_; }
    hipStream_t stream() const { return stream_; }

    void reset();
    void step(int token, float* logits_out, int* next_token_out);
    void step_debug(int token, float* residuals_out, float* logits_out, int* next_token_out);
    // One step of the persistent kernel with per-phase timestamps; returns the grid size.
    int step_profile(int token, unsigned long long* stamps_out, long capacity);
    // One step of the persistent kernel that also copies out the vectors of every phase (TraceLayout).
    void step_trace(int token, float* trace_out, long capacity, float* logits_out, int* next_token_out);

private:
    // Common head of every step: the sequence must have room and the token must be a vocabulary index
    // or -1 (reuse the device argmax).
    void begin_step(const char* who, int token);
    void launch_persistent(const DecodeParams& p);
    void read_outputs(float* logits_out, int* next_token_out);
    void raise_if_kernel_failed();
    void build_program();
    void run_program(bool debug);
    void release() noexcept;

    std::unique_ptr<Weights> weights_;
    EngineOptions opts_;
    int max_seq_ = 0;
    int host_pos_ = 0;
    int rpb_ = 0;
    hipStream_t stream_ = nullptr;

    // Multi-kernel step: launches in op order; debug-only entries copy the residual stream into d_res_.
    struct Op {
        bool debug_only;
        std::function<void(hipStream_t)> enqueue;
    };
    std::vector<Op> program_;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t graph_exec_ = nullptr;

    void* arena_ = nullptr;  // every activation buffer, one allocation
    float *x_ = nullptr, *xb_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *tmp_ = nullptr, *gu_ = nullptr,
          *act_ = nullptr, *logits_ = nullptr, *part_o_ = nullptr, *part_ml_ = nullptr, *arg_v_ = nullptr;
    int *arg_i_ = nullptr, *d_token_ = nullptr, *d_pos_ = nullptr;
    uint16_t *k_cache_ = nullptr, *v_cache_ = nullptr;  // fp16 [layer][kv_head][max_seq][head_dim]
    float* d_res_ = nullptr;  // residual snapshots for step_debug, (n_layers + 1) x hidden

    // Persistent decode kernel.
    bool persistent_ = false;
    int grid_ = 0;
    DecodeParams dp_{};
    void* tags_begin_ = nullptr;  // the tagged buffers, one contiguous range
    size_t tags_bytes_ = 0;
    unsigned launches_ = 0;       // launches since the tags were last cleared
    unsigned step_limit_ = kDecodeStepLimit;
    unsigned long long* d_stamps_ = nullptr;
};

}  // namespace cllm
