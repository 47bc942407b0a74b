// .cudallm file parsing, validation and upload to one HBM allocation.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "common.h"

namespace cllm {

#pragma pack(push, 1)
// On-disk header, 256 bytes little-endian (reference src/model/cudallm_format.h:12-31).
struct FileHeader {
    char magic[4];
    uint32_t version, weight_dtype, hidden, inter, n_layers, n_heads, n_kv_heads, head_dim, vocab, max_seq_len;
    float rms_eps, rope_theta;
    uint32_t group_size, n_tensors, reserved0;
    uint64_t table_offset;
    uint8_t pad[184];
};
// On-disk tensor table entry, 80 bytes (reference src/model/cudallm_format.h:33-41).
struct FileEntry {
    char name[48];
    uint32_t dtype, rows, cols, reserved;
    uint64_t offset, nbytes;
};
#pragma pack(pop)
static_assert(sizeof(FileHeader) == 256, "header is 256 bytes");
static_assert(sizeof(FileEntry) == 80, "entry is 80 bytes");

// One matrix operand as it sits in HBM.
struct Linear {
    const void* w = nullptr;       // bf16 bits / int8 / packed int4, row-major
    const void* scales = nullptr;  // int8: fp32 [rows]; int4: fp16 [rows][cols/128]; bf16: null
    int rows = 0, cols = 0;
    WType wt = WType::BF16;
};

struct LayerWeights {
    const float* attn_norm = nullptr;
    Linear wqkv, wo;
    const float* ffn_norm = nullptr;
    Linear w_gate_up, w_down;
};

struct ModelConfig {
    WType wt = WType::BF16;
    int hidden = 0, inter = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, vocab = 0;
    int max_seq_len = 0, group_size = 0;
    float rms_eps = 0.f;
};

// Parses the header and table and checks them completely before touching the device, so every
// FORMAT / IO error is reported without a GPU.
struct ParsedFile {
    FileHeader header{};
    std::vector<FileEntry> table;
    ModelConfig config;
    uint64_t data_begin = 0, data_end = 0, weight_bytes = 0;
};
ParsedFile parse_file(const std::string& path);

class Weights {
public:
    explicit Weights(const std::string& path);
    ~Weights();
    Weights(const Weights&) = delete;
    Weights& operator=(const Weights&) = delete;

    const ModelConfig& config() const { return cfg_; }
    uint64_t weight_bytes() const { return weight_bytes_; }

    const float* inv_freq = nullptr;
    const float* final_norm = nullptr;
    Linear tok_embeddings;  // tied: also the lm_head
    std::vector<LayerWeights> layers;

private:
    ModelConfig cfg_;
    void* base_ = nullptr;
    uint64_t weight_bytes_ = 0;
};

}  // namespace cllm
