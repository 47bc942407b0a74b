// .cudallm loader for the persistent decode engine.
//
// The file format is the reference's (src/model/cudallm_format.h:12-46, python/cudallm/format.py:22-147): a 256-byte
// header, a table of 80-byte entries in a fixed tensor order, 256-byte aligned tensor data.  Which tensors a file
// holds, in what order and with what shapes is the format's contract, restated here as data: a model schema (the
// global tensors and the tensors of one layer) and, per weight type, how one matrix is encoded (its weight dtype and
// its scales).  Validation is a table of header rules and a table of per-entry rules, so every violation reports the
// rule it broke.  After validation the data region is uploaded into ONE device allocation through two pinned 64 MiB
// buffers (the disk read of chunk i + 1 overlaps the copy of chunk i), and each consumer pointer is bound by tensor
// name.  Only Llama-3.2-1B dimensions are accepted (hidden 2048, inter 8192, 16 layers, 32/8 heads, head_dim 64,
// vocab 128256): the decode kernels are specialised for that shape, as the reference's are (weights.cpp:19-27).
#include "weights.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <unordered_map>

namespace cllm {

namespace {

// ---- the model the engine decodes ----

struct Geometry {
    uint32_t hidden = 2048, inter = 8192, layers = 16, heads = 32, kv_heads = 8, head_dim = 64, vocab = 128256;
    uint32_t int4_group = 128;
    uint32_t qkv_rows() const { return (heads + 2 * kv_heads) * head_dim; }
};
constexpr Geometry kModel{};
constexpr uint64_t kDataAlign = 256;
constexpr size_t kStageBytes = 64ull << 20;

// Storage width of each tensor dtype, in bits per element (I4X2 packs two 4-bit values per byte).
struct DTypeInfo {
    TDType dt;
    unsigned bits;
};
constexpr DTypeInfo kDTypes[] = {{TDType::F32, 32}, {TDType::BF16, 16}, {TDType::F16, 16}, {TDType::I8, 8},
                                 {TDType::I4X2, 4}};

bool known_dtype(uint32_t code) {
    return std::any_of(std::begin(kDTypes), std::end(kDTypes), [&](const DTypeInfo& d) { return uint32_t(d.dt) == code; });
}
uint64_t storage_bytes(TDType dt, uint64_t rows, uint64_t cols) {
    for (const DTypeInfo& d : kDTypes)
        if (d.dt == dt) return rows * cols * d.bits / 8;
    throw FormatError("tensor dtype " + std::to_string(static_cast<uint32_t>(dt)) + " has no storage width");
}

// How one weight matrix [rows][cols] is stored for each weight type: the ".weight" tensor, and for quantised files a
// ".scales" tensor of rows x scale_cols(cols) values.
struct Encoding {
    WType wt;
    TDType weight;
    bool scaled;
    TDType scale;
    uint32_t scale_group;  // columns per scale (0: one scale per row)
    uint32_t n_tensors;    // the file's tensor count with this encoding
};
constexpr Encoding kEncodings[] = {
    {WType::BF16, TDType::BF16, false, TDType::F32, 0, 99},
    {WType::INT8, TDType::I8, true, TDType::F32, 0, 164},
    {WType::INT4, TDType::I4X2, true, TDType::F16, 128, 164},
};
const Encoding& encoding_of(WType wt) {
    for (const Encoding& e : kEncodings)
        if (e.wt == wt) return e;
    throw FormatError("no encoding for weight type " + std::to_string(static_cast<int>(wt)));
}

// The model schema: global tensors, then per layer; a matrix expands to its encoding's tensors.
enum class Kind { Vector, Matrix };
struct Part {
    const char* name;
    Kind kind;
    uint32_t rows, cols;
};
const Part kGlobalParts[] = {
    {"rope.inv_freq", Kind::Vector, kModel.head_dim / 2, 1},
    {"tok_embeddings", Kind::Matrix, kModel.vocab, kModel.hidden},
    {"norm.weight", Kind::Vector, kModel.hidden, 1},
};
const Part kLayerParts[] = {
    {"attn_norm.weight", Kind::Vector, kModel.hidden, 1},
    {"wqkv", Kind::Matrix, kModel.qkv_rows(), kModel.hidden},
    {"wo", Kind::Matrix, kModel.hidden, kModel.heads * kModel.head_dim},
    {"ffn_norm.weight", Kind::Vector, kModel.hidden, 1},
    {"w_gate_up", Kind::Matrix, 2 * kModel.inter, kModel.hidden},
    {"w_down", Kind::Matrix, kModel.hidden, kModel.inter},
};

struct Expected {
    std::string name;
    TDType dt;
    uint32_t rows, cols;
};

void expand(const Part& part, const std::string& prefix, const Encoding& enc, std::vector<Expected>& out) {
    const std::string base = prefix + part.name;
    if (part.kind == Kind::Vector) {
        out.push_back({base, TDType::F32, part.rows, part.cols});
        return;
    }
    out.push_back({base + ".weight", enc.weight, part.rows, part.cols});
    if (enc.scaled) out.push_back({base + ".scales", enc.scale, part.rows, enc.scale_group ? part.cols / enc.scale_group : 1});
}

// Every tensor a file of this encoding holds, in file order.
std::vector<Expected> schema(const Encoding& enc) {
    std::vector<Expected> out;
    for (const Part& p : kGlobalParts) expand(p, "", enc, out);
    for (uint32_t l = 0; l < kModel.layers; ++l)
        for (const Part& p : kLayerParts) expand(p, "layers." + std::to_string(l) + ".", enc, out);
    return out;
}

// ---- validation rules ----

// A rule over the header; it returns the reason the header breaks it, or an empty string.
struct HeaderRule {
    std::function<std::string(const FileHeader&, const Encoding&)> broken;
};
HeaderRule field_is(const char* field, std::function<uint64_t(const FileHeader&)> got,
                    std::function<uint64_t(const Encoding&)> need) {
    return {[=](const FileHeader& h, const Encoding& e) {
        const uint64_t g = got(h), n = need(e);
        return g == n ? std::string()
                      : std::string("header ") + field + " is " + std::to_string(g) + ", this engine needs " +
                            std::to_string(n);
    }};
}
const std::vector<HeaderRule>& header_rules() {
    static const std::vector<HeaderRule> rules = {
        field_is("version", [](const FileHeader& h) { return h.version; }, [](const Encoding&) { return 1u; }),
        field_is("hidden_size", [](const FileHeader& h) { return h.hidden; }, [](const Encoding&) { return kModel.hidden; }),
        field_is("intermediate_size", [](const FileHeader& h) { return h.inter; },
                 [](const Encoding&) { return kModel.inter; }),
        field_is("n_layers", [](const FileHeader& h) { return h.n_layers; }, [](const Encoding&) { return kModel.layers; }),
        field_is("n_heads", [](const FileHeader& h) { return h.n_heads; }, [](const Encoding&) { return kModel.heads; }),
        field_is("n_kv_heads", [](const FileHeader& h) { return h.n_kv_heads; },
                 [](const Encoding&) { return kModel.kv_heads; }),
        field_is("head_dim", [](const FileHeader& h) { return h.head_dim; }, [](const Encoding&) { return kModel.head_dim; }),
        field_is("vocab_size", [](const FileHeader& h) { return h.vocab; }, [](const Encoding&) { return kModel.vocab; }),
        {[](const FileHeader& h, const Encoding&) {
            return h.max_seq_len > 0 && h.max_seq_len % 128 == 0 ? std::string()
                                                                  : "header max_seq_len must be a positive multiple of 128";
        }},
        field_is("n_tensors", [](const FileHeader& h) { return h.n_tensors; }, [](const Encoding& e) { return e.n_tensors; }),
        field_is("table_offset", [](const FileHeader& h) { return h.table_offset; }, [](const Encoding&) { return 256u; }),
        field_is("group_size", [](const FileHeader& h) { return h.group_size; },
                 [](const Encoding& e) { return e.scale_group; }),
    };
    return rules;
}

// A rule over one table entry against the tensor the schema expects there; `end` is where the previous tensor's data
// ended.  It returns the reason the entry breaks it, or an empty string.
struct EntryRule {
    std::function<std::string(const FileEntry&, const Expected&, uint64_t end)> broken;
};
const std::vector<EntryRule>& entry_rules() {
    static const std::vector<EntryRule> rules = {
        {[](const FileEntry& e, const Expected& x, uint64_t) {
            return e.dtype == static_cast<uint32_t>(x.dt) && e.rows == x.rows && e.cols == x.cols
                       ? std::string()
                       : "dtype or shape does not match the format (want dtype " + std::to_string(uint32_t(x.dt)) + ", " +
                             std::to_string(x.rows) + " x " + std::to_string(x.cols) + ")";
        }},
        {[](const FileEntry& e, const Expected&, uint64_t) {
            return e.offset % kDataAlign == 0 ? std::string() : "offset is not 256-byte aligned";
        }},
        {[](const FileEntry& e, const Expected&, uint64_t end) {
            return e.offset >= end ? std::string() : "overlaps the data before it";
        }},
        {[](const FileEntry& e, const Expected& x, uint64_t) {
            return e.nbytes == storage_bytes(x.dt, x.rows, x.cols) ? std::string() : "wrong nbytes for its dtype and shape";
        }},
    };
    return rules;
}

std::string entry_name(const FileEntry& e) { return std::string(e.name, strnlen(e.name, sizeof(e.name))); }

// Reads exactly n bytes at the stream's position or reports which part of the file ended early.
void read_span(std::ifstream& f, void* dst, size_t n, const std::string& path, const char* part) {
    f.read(static_cast<char*>(dst), static_cast<std::streamsize>(n));
    if (static_cast<size_t>(f.gcount()) != n) throw IoError(path + ": the file ends inside its " + part);
}

}  // namespace

ParsedFile parse_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) throw IoError("cannot open " + path);
    const uint64_t size = static_cast<uint64_t>(f.tellg());
    f.seekg(0);

    ParsedFile pf;
    FileHeader& h = pf.header;
    if (size < sizeof(FileHeader)) throw FormatError(path + ": too small to hold the 256-byte header");
    read_span(f, &h, sizeof(h), path, "header");
    if (std::memcmp(h.magic, "CLLM", 4) != 0) throw FormatError(path + ": bad magic (not a .cudallm file)");
    const bool known_type = std::any_of(std::begin(kEncodings), std::end(kEncodings),
                                        [&](const Encoding& e) { return uint32_t(e.wt) == h.weight_dtype; });
    if (!known_type)
        throw FormatError("weight_dtype " + std::to_string(h.weight_dtype) + " is not 1 (bf16), 3 (int8) or 4 (int4)");
    const Encoding& enc = encoding_of(static_cast<WType>(h.weight_dtype));
    for (const HeaderRule& r : header_rules()) {
        const std::string why = r.broken(h, enc);
        if (!why.empty()) throw FormatError(why);
    }

    const std::vector<Expected> want = schema(enc);
    CLLM_INTERNAL(want.size() == enc.n_tensors, "the schema and the encoding disagree on the tensor count");
    const uint64_t table_end = h.table_offset + uint64_t(h.n_tensors) * sizeof(FileEntry);
    if (size < table_end) throw FormatError(path + ": too small to hold the tensor table");
    pf.table.resize(h.n_tensors);
    f.seekg(static_cast<std::streamoff>(h.table_offset));
    read_span(f, pf.table.data(), pf.table.size() * sizeof(FileEntry), path, "tensor table");

    uint64_t end = table_end;
    for (size_t i = 0; i < pf.table.size(); ++i) {
        const FileEntry& e = pf.table[i];
        const Expected& x = want[i];
        const std::string name = entry_name(e);
        if (name != x.name)
            throw FormatError("tensor #" + std::to_string(i) + " is '" + name + "', expected '" + x.name + "'");
        if (!known_dtype(e.dtype)) throw FormatError("tensor '" + name + "': unknown dtype " + std::to_string(e.dtype));
        for (const EntryRule& r : entry_rules()) {
            const std::string why = r.broken(e, x, end);
            if (!why.empty()) throw FormatError("tensor '" + name + "': " + why);
        }
        end = e.offset + e.nbytes;
        pf.weight_bytes += e.nbytes;
    }
    pf.data_begin = pf.table.front().offset;
    pf.data_end = end;
    if (size < pf.data_end) throw FormatError(path + ": truncated inside the tensor data");

    ModelConfig& c = pf.config;
    c.wt = enc.wt;
    c.hidden = static_cast<int>(kModel.hidden);
    c.inter = static_cast<int>(kModel.inter);
    c.n_layers = static_cast<int>(kModel.layers);
    c.n_heads = static_cast<int>(kModel.heads);
    c.n_kv_heads = static_cast<int>(kModel.kv_heads);
    c.head_dim = static_cast<int>(kModel.head_dim);
    c.vocab = static_cast<int>(kModel.vocab);
    c.max_seq_len = static_cast<int>(h.max_seq_len);
    c.group_size = static_cast<int>(h.group_size);
    c.rms_eps = h.rms_eps;
    return pf;
}

namespace {

// Streams the file's data region into `dst` (span bytes) through two pinned staging buffers, alternating: the read of
// the next chunk into one buffer overlaps the copy of the previous chunk out of the other.
void upload(const std::string& path, uint64_t begin, uint64_t span, void* dst) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw IoError("cannot open " + path);
    f.seekg(static_cast<std::streamoff>(begin));
    struct Stage {
        void* host = nullptr;
        hipEvent_t free = nullptr;  // recorded after the copy out of `host`
    } stage[2];
    hipStream_t s = nullptr;
    auto release = [&] {
        if (s) (void)hipStreamSynchronize(s);
        for (Stage& b : stage) {
            if (b.free) (void)hipEventDestroy(b.free);
            if (b.host) (void)hipHostFree(b.host);
        }
        if (s) (void)hipStreamDestroy(s);
    };
    try {
        CLLM_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        for (Stage& b : stage) {
            CLLM_HIP(hipHostMalloc(&b.host, kStageBytes, hipHostMallocDefault));
            CLLM_HIP(hipEventCreateWithFlags(&b.free, hipEventDisableTiming));
        }
        for (uint64_t off = 0, chunk = 0; off < span; off += kStageBytes, ++chunk) {
            Stage& b = stage[chunk % 2];
            const size_t n = static_cast<size_t>(std::min<uint64_t>(kStageBytes, span - off));
            CLLM_HIP(hipEventSynchronize(b.free));
            read_span(f, b.host, n, path, "tensor data");
            CLLM_HIP(hipMemcpyAsync(static_cast<char*>(dst) + off, b.host, n, hipMemcpyHostToDevice, s));
            CLLM_HIP(hipEventRecord(b.free, s));
        }
        CLLM_HIP(hipStreamSynchronize(s));
    } catch (...) {
        release();
        throw;
    }
    release();
}

}  // namespace

Weights::Weights(const std::string& path) {
    const ParsedFile pf = parse_file(path);
    cfg_ = pf.config;
    weight_bytes_ = pf.weight_bytes;
    CLLM_HIP(hipMalloc(&base_, pf.data_end - pf.data_begin));
    try {
        upload(path, pf.data_begin, pf.data_end - pf.data_begin, base_);
    } catch (...) {
        (void)hipFree(base_);
        base_ = nullptr;
        throw;
    }

    // Device address of every tensor, by name.
    std::unordered_map<std::string, const void*> at;
    for (const FileEntry& e : pf.table) at[entry_name(e)] = static_cast<const char*>(base_) + (e.offset - pf.data_begin);
    auto tensor = [&](const std::string& name) {
        const auto it = at.find(name);
        CLLM_INTERNAL(it != at.end(), "a validated file lacks a schema tensor");
        return it->second;
    };
    const Encoding& enc = encoding_of(cfg_.wt);
    auto matrix = [&](const std::string& name, uint32_t rows, uint32_t cols) {
        Linear m;
        m.w = tensor(name + ".weight");
        m.scales = enc.scaled ? tensor(name + ".scales") : nullptr;
        m.rows = static_cast<int>(rows);
        m.cols = static_cast<int>(cols);
        m.wt = cfg_.wt;
        return m;
    };
    auto vec = [&](const std::string& name) { return static_cast<const float*>(tensor(name)); };
    inv_freq = vec("rope.inv_freq");
    final_norm = vec("norm.weight");
    tok_embeddings = matrix("tok_embeddings", kModel.vocab, kModel.hidden);
    layers.resize(kModel.layers);
    for (uint32_t l = 0; l < kModel.layers; ++l) {
        const std::string p = "layers." + std::to_string(l) + ".";
        LayerWeights& L = layers[l];
        L.attn_norm = vec(p + "attn_norm.weight");
        L.ffn_norm = vec(p + "ffn_norm.weight");
        L.wqkv = matrix(p + "wqkv", kModel.qkv_rows(), kModel.hidden);
        L.wo = matrix(p + "wo", kModel.hidden, kModel.heads * kModel.head_dim);
        L.w_gate_up = matrix(p + "w_gate_up", 2 * kModel.inter, kModel.hidden);
        L.w_down = matrix(p + "w_down", kModel.hidden, kModel.inter);
    }
}

Weights::~Weights() {
    if (base_) {
        const hipError_t e = hipFree(base_);
        if (e != hipSuccess) std::fprintf(stderr, "cudallm: hipFree in ~Weights: %s\n", hipGetErrorString(e));
    }
}

}  // namespace cllm
