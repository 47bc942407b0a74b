// Batch-1 decode engine: owns the weights, the activations, the fp16 KV cache and the decode graph.
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <string>

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

// Option rules of reference src/engine/engine.cpp:10-21 plus max_seq_len <= the file's value.
void validate_options(const EngineOptions& o, const ModelConfig& c);

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

    void reset();
    void step(int token, float* logits_out, int* next_token_out);
    void step_debug(int token, float* residuals_out, float* logits_out, int* next_token_out);
    // One step of the persistent kernel with per-phase timestamps; returns the grid size.
    int step_profile(int token, unsigned long long* stamps_out, long capacity);
    hipStream_t stream() const { return stream_; }

private:
    void enqueue_forward(float* residuals_out);
    void linear(const Linear& L, const float* x, float* y, Epilogue ep, const float* norm_w);
    void check_device_error();
    void release() noexcept;

    std::unique_ptr<Weights> weights_;
    EngineOptions opts_;
    int max_seq_ = 0;
    int host_pos_ = 0;
    int rpb_ = 0;
    hipStream_t stream_ = nullptr;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;

    void* arena_ = nullptr;  // every activation buffer, one allocation
    float *x_ = nullptr, *xb_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *tmp_ = nullptr, *gu_ = nullptr,
          *act_ = nullptr, *logits_ = nullptr, *part_o_ = nullptr, *part_ml_ = nullptr, *arg_v_ = nullptr;
    int *arg_i_ = nullptr, *d_token_ = nullptr, *d_pos_ = nullptr;
    uint16_t *k_cache_ = nullptr, *v_cache_ = nullptr;  // fp16 [layer][kv_head][max_seq][head_dim]

    // Persistent decode kernel (fused + opt options): one launch per token.
    bool persistent_ = false;
    int grid_ = 0;
    DecodeParams dp_{};
    float* d_res_ = nullptr;  // residual snapshots for step_debug
    unsigned* d_err_ = nullptr;
    unsigned long long* d_stamps_ = nullptr;
};

}  // namespace cllm
