// .cudallm loader: the validation rules of reference src/model/weights.cpp:99-219, re-implemented.
//
// The loader accepts only Llama-3.2-1B dimensions (hidden 2048, inter 8192, 16 layers, 32 heads,
// 8 kv heads, head_dim 64, vocab 128256), like the reference (weights.cpp:19-27,116-128), because
// the decode kernels are specialised for that shape.  All tensors go into ONE device allocation;
// the file is streamed through two pinned 64 MiB buffers so the disk read of chunk i+1 overlaps
// the host-to-device copy of chunk i.
#include "weights.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>

namespace cllm {

namespace {

constexpr uint32_t kHidden = 2048, kInter = 8192, kLayers = 16, kHeads = 32, kKvHeads = 8, kHeadDim = 64;
constexpr uint32_t kVocab = 128256, kGroup = 128;
constexpr uint64_t kAlign = 256;
constexpr size_t kStage = 64ull << 20;

struct Want {
    std::string name;
    TDType dt;
    uint32_t rows, cols;
};

uint64_t nbytes_of(TDType dt, uint64_t rows, uint64_t cols) {
    switch (dt) {
        case TDType::F32: return rows * cols * 4;
        case TDType::BF16:
        case TDType::F16: return rows * cols * 2;
        case TDType::I8: return rows * cols;
        case TDType::I4X2: return rows * cols / 2;
    }
    throw FormatError("unknown tensor dtype");
}

void want_linear(std::vector<Want>& v, const std::string& n, WType wt, uint32_t rows, uint32_t cols) {
    if (wt == WType::BF16) {
        v.push_back({n + ".weight", TDType::BF16, rows, cols});
    } else if (wt == WType::INT8) {
        v.push_back({n + ".weight", TDType::I8, rows, cols});
        v.push_back({n + ".scales", TDType::F32, rows, 1});
    } else {
        v.push_back({n + ".weight", TDType::I4X2, rows, cols});
        v.push_back({n + ".scales", TDType::F16, rows, cols / kGroup});
    }
}

// The exact tensor sequence of a file with weight type wt (reference weights.cpp:66-81).
std::vector<Want> wanted(WType wt) {
    std::vector<Want> v;
    v.push_back({"rope.inv_freq", TDType::F32, kHeadDim / 2, 1});
    want_linear(v, "tok_embeddings", wt, kVocab, kHidden);
    v.push_back({"norm.weight", TDType::F32, kHidden, 1});
    for (uint32_t i = 0; i < kLayers; ++i) {
        const std::string p = "layers." + std::to_string(i) + ".";
        v.push_back({p + "attn_norm.weight", TDType::F32, kHidden, 1});
        want_linear(v, p + "wqkv", wt, (kHeads + 2 * kKvHeads) * kHeadDim, kHidden);
        want_linear(v, p + "wo", wt, kHidden, kHeads * kHeadDim);
        v.push_back({p + "ffn_norm.weight", TDType::F32, kHidden, 1});
        want_linear(v, p + "w_gate_up", wt, 2 * kInter, kHidden);
        want_linear(v, p + "w_down", wt, kHidden, kInter);
    }
    return v;
}

void field(uint64_t got, uint64_t want, const char* what) {
    if (got != want)
        throw FormatError(std::string("header ") + what + " is " + std::to_string(got) + ", this engine needs " +
                          std::to_string(want));
}

void read_all(std::ifstream& f, void* dst, size_t n, const std::string& path, const char* what) {
    f.read(static_cast<char*>(dst), static_cast<std::streamsize>(n));
    if (static_cast<size_t>(f.gcount()) != n) throw IoError(path + ": short read of the " + what);
}

}  // namespace

ParsedFile parse_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw IoError("cannot open " + path);
    f.seekg(0, std::ios::end);
    const uint64_t size = static_cast<uint64_t>(f.tellg());
    f.seekg(0);

    ParsedFile pf;
    FileHeader& h = pf.header;
    if (size < sizeof(h)) throw FormatError(path + ": too small to hold the 256-byte header");
    read_all(f, &h, sizeof(h), path, "header");
    if (std::memcmp(h.magic, "CLLM", 4) != 0) throw FormatError(path + ": bad magic (not a .cudallm file)");
    field(h.version, 1, "version");
    if (h.weight_dtype != 1 && h.weight_dtype != 3 && h.weight_dtype != 4)
        throw FormatError("weight_dtype " + std::to_string(h.weight_dtype) + " is not 1 (bf16), 3 (int8) or 4 (int4)");
    const WType wt = static_cast<WType>(h.weight_dtype);
    field(h.hidden, kHidden, "hidden_size");
    field(h.inter, kInter, "intermediate_size");
    field(h.n_layers, kLayers, "n_layers");
    field(h.n_heads, kHeads, "n_heads");
    field(h.n_kv_heads, kKvHeads, "n_kv_heads");
    field(h.head_dim, kHeadDim, "head_dim");
    field(h.vocab, kVocab, "vocab_size");
    if (h.max_seq_len == 0 || h.max_seq_len % 128 != 0)
        throw FormatError("header max_seq_len must be a positive multiple of 128");
    field(h.n_tensors, wt == WType::BF16 ? 99 : 164, "n_tensors");
    field(h.table_offset, 256, "table_offset");
    field(h.group_size, wt == WType::INT4 ? kGroup : 0, "group_size");

    const std::vector<Want> want = wanted(wt);
    CLLM_INTERNAL(want.size() == h.n_tensors, "tensor list size");
    const uint64_t table_end = h.table_offset + uint64_t(h.n_tensors) * sizeof(FileEntry);
    if (size < table_end) throw FormatError(path + ": too small to hold the tensor table");
    pf.table.resize(h.n_tensors);
    f.seekg(static_cast<std::streamoff>(h.table_offset));
    read_all(f, pf.table.data(), pf.table.size() * sizeof(FileEntry), path, "tensor table");

    uint64_t end = table_end;
    for (size_t k = 0; k < pf.table.size(); ++k) {
        const FileEntry& e = pf.table[k];
        const Want& w = want[k];
        const std::string name(e.name, strnlen(e.name, sizeof(e.name)));
        if (name != w.name) throw FormatError("tensor #" + std::to_string(k) + " is '" + name + "', expected '" + w.name + "'");
        if (e.dtype != static_cast<uint32_t>(w.dt) || e.rows != w.rows || e.cols != w.cols)
            throw FormatError("tensor '" + name + "': dtype or shape does not match the format");
        if (e.offset % kAlign) throw FormatError("tensor '" + name + "': offset is not 256-byte aligned");
        if (e.offset < end) throw FormatError("tensor '" + name + "': overlaps the data before it");
        if (e.nbytes != nbytes_of(w.dt, w.rows, w.cols)) throw FormatError("tensor '" + name + "': wrong nbytes");
        end = e.offset + e.nbytes;
        pf.weight_bytes += e.nbytes;
    }
    pf.data_begin = pf.table.front().offset;
    pf.data_end = end;
    if (size < pf.data_end) throw FormatError(path + ": truncated inside the tensor data");

    ModelConfig& c = pf.config;
    c.wt = wt;
    c.hidden = kHidden;
    c.inter = kInter;
    c.n_layers = kLayers;
    c.n_heads = kHeads;
    c.n_kv_heads = kKvHeads;
    c.head_dim = kHeadDim;
    c.vocab = kVocab;
    c.max_seq_len = static_cast<int>(h.max_seq_len);
    c.group_size = static_cast<int>(h.group_size);
    c.rms_eps = h.rms_eps;
    return pf;
}

Weights::Weights(const std::string& path) {
    const ParsedFile pf = parse_file(path);
    cfg_ = pf.config;
    weight_bytes_ = pf.weight_bytes;
    const uint64_t span = pf.data_end - pf.data_begin;

    std::ifstream f(path, std::ios::binary);
    if (!f) throw IoError("cannot open " + path);
    CLLM_HIP(hipMalloc(&base_, span));
    void* pin[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipStream_t s = nullptr;
    auto cleanup = [&] {
        if (s) (void)hipStreamSynchronize(s);
        for (int i = 0; i < 2; ++i) {
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (pin[i]) (void)hipHostFree(pin[i]);
        }
        if (s) (void)hipStreamDestroy(s);
    };
    try {
        CLLM_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        for (int i = 0; i < 2; ++i) {
            CLLM_HIP(hipHostMalloc(&pin[i], kStage, hipHostMallocDefault));
            CLLM_HIP(hipEventCreateWithFlags(&done[i], hipEventDisableTiming));
        }
        f.seekg(static_cast<std::streamoff>(pf.data_begin));
        int b = 0;
        for (uint64_t off = 0; off < span; off += kStage, b ^= 1) {
            const size_t n = static_cast<size_t>(std::min<uint64_t>(kStage, span - off));
            CLLM_HIP(hipEventSynchronize(done[b]));  // the copy that last used this buffer is finished
            read_all(f, pin[b], n, path, "tensor data");
            CLLM_HIP(hipMemcpyAsync(static_cast<char*>(base_) + off, pin[b], n, hipMemcpyHostToDevice, s));
            CLLM_HIP(hipEventRecord(done[b], s));
        }
        CLLM_HIP(hipStreamSynchronize(s));
    } catch (...) {
        cleanup();
        (void)hipFree(base_);
        base_ = nullptr;
        throw;
    }
    cleanup();

    size_t k = 0;
    auto at = [&](size_t i) -> const void* {
        return static_cast<const char*>(base_) + (pf.table[i].offset - pf.data_begin);
    };
    const bool quant = cfg_.wt != WType::BF16;
    auto linear = [&](int rows, int cols) {
        Linear L;
        L.w = at(k++);
        L.scales = quant ? at(k++) : nullptr;
        L.rows = rows;
        L.cols = cols;
        L.wt = cfg_.wt;
        return L;
    };
    const int H = cfg_.hidden, I = cfg_.inter, QKV = (cfg_.n_heads + 2 * cfg_.n_kv_heads) * cfg_.head_dim;
    inv_freq = static_cast<const float*>(at(k++));
    tok_embeddings = linear(cfg_.vocab, H);
    final_norm = static_cast<const float*>(at(k++));
    layers.resize(cfg_.n_layers);
    for (LayerWeights& L : layers) {
        L.attn_norm = static_cast<const float*>(at(k++));
        L.wqkv = linear(QKV, H);
        L.wo = linear(H, cfg_.n_heads * cfg_.head_dim);
        L.ffn_norm = static_cast<const float*>(at(k++));
        L.w_gate_up = linear(2 * I, H);
        L.w_down = linear(H, I);
    }
    CLLM_INTERNAL(k == pf.table.size(), "tensor pointer assignment");
}

Weights::~Weights() {
    if (base_) {
        const hipError_t e = hipFree(base_);
        if (e != hipSuccess) std::fprintf(stderr, "cudallm: hipFree in ~Weights: %s\n", hipGetErrorString(e));
    }
}

}  // namespace cllm
