// The C ABI of include/cudallm/cudallm.h: names, signatures, struct layouts and error codes of the
// reference interface (include/cudallm/cudallm.h:8-56, src/capi/cudallm_capi.cpp:84-316).
//
// Structure of this file:
//  * abi_entry() runs an entry point's body; a C++ exception never crosses the ABI, it becomes one of
//    the CUDALLM_* codes (chosen by the exception's type) and a thread-local message that names the
//    entry point.
//  * Test hooks stage their host operands through one device allocation per call (HookStaging), run
//    the kernel on the null stream, synchronise, and copy the outputs back.
#include "cudallm/cudallm.h"

#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "engine.h"

struct cudallm_engine {
    std::unique_ptr<cllm::Engine> impl;
};

namespace cllm {

[[noreturn]] void throw_hip(hipError_t err, const char* expr, const char* file, int line) {
    throw DeviceError(std::string(hipGetErrorString(err)) + " (" + expr + " at " + file + ":" + std::to_string(line) + ")");
}

const char* wtype_name(WType w) {
    switch (w) {
        case WType::BF16: return "bf16";
        case WType::INT8: return "int8";
        case WType::INT4: return "int4";
    }
    return "unknown";
}

}  // namespace cllm

namespace {

thread_local std::string t_message;

int record(int code, const char* entry, const char* what) {
    t_message = std::string(entry) + ": " + what;
    return code;
}

template <typename Body>
int abi_entry(const char* entry, Body&& body) noexcept {
    try {
        body();
        return CUDALLM_OK;
    } catch (const cllm::ArgError& e) {
        return record(CUDALLM_ERR_INVALID_ARG, entry, e.what());
    } catch (const cllm::IoError& e) {
        return record(CUDALLM_ERR_IO, entry, e.what());
    } catch (const cllm::FormatError& e) {
        return record(CUDALLM_ERR_FORMAT, entry, e.what());
    } catch (const cllm::DeviceError& e) {
        return record(CUDALLM_ERR_CUDA, entry, e.what());
    } catch (const cllm::StateError& e) {
        return record(CUDALLM_ERR_STATE, entry, e.what());
    } catch (const std::exception& e) {  // SequenceFull and logic errors: INTERNAL, as the reference reports them
        return record(CUDALLM_ERR_INTERNAL, entry, e.what());
    } catch (...) {
        return record(CUDALLM_ERR_INTERNAL, entry, "unrecognised exception");
    }
}

cllm::Engine& engine_of(cudallm_engine* e) {
    if (!e || !e->impl) throw cllm::ArgError("null engine handle");
    return *e->impl;
}

void need(bool ok, const char* why) {
    if (!ok) throw cllm::ArgError(why);
}

cllm::WType weight_type(int code) {
    need(code == 1 || code == 3 || code == 4, "weight_dtype must be 1 (bf16), 3 (int8) or 4 (int4)");
    return static_cast<cllm::WType>(code);
}

// Device memory for one hook call: operands are declared first (host source or sink and size), then
// one allocation is made and the inputs are uploaded; finish() waits for the kernels and copies the
// outputs back.  Freed when the call returns, on every path.
class HookStaging {
public:
    enum Dir { In, Out, InOut, Scratch };
    int add(const void* host, size_t bytes, Dir dir) {
        slots_.push_back({const_cast<void*>(host), bytes, dir, total_});
        total_ += (bytes + 255) / 256 * 256;
        return static_cast<int>(slots_.size()) - 1;
    }
    void upload() {
        if (total_) CLLM_HIP(hipMalloc(&dev_, total_));
        for (const Slot& s : slots_)
            if ((s.dir == In || s.dir == InOut) && s.bytes)
                CLLM_HIP(hipMemcpy(at(s), s.host, s.bytes, hipMemcpyHostToDevice));
    }
    template <typename T>
    T* dev(int slot) const {
        return slots_[slot].bytes ? static_cast<T*>(at(slots_[slot])) : nullptr;
    }
    void finish() {
        CLLM_HIP(hipGetLastError());
        CLLM_HIP(hipDeviceSynchronize());
        for (const Slot& s : slots_)
            if ((s.dir == Out || s.dir == InOut) && s.bytes)
                CLLM_HIP(hipMemcpy(s.host, at(s), s.bytes, hipMemcpyDeviceToHost));
    }
    ~HookStaging() {
        if (dev_) (void)hipFree(dev_);
    }

private:
    struct Slot {
        void* host;
        size_t bytes;
        Dir dir;
        size_t offset;
    };
    void* at(const Slot& s) const { return static_cast<char*>(dev_) + s.offset; }
    std::vector<Slot> slots_;
    size_t total_ = 0;
    void* dev_ = nullptr;
};

// The opt matvec on device pointers: shared by the plain and the timed launch entry points.
void enqueue_matvec(int weight_dtype, int epilogue, int rpb, const void* w, const void* scales, const float* x,
                    const float* norm_w, float eps, float* y, int rows, int cols, void* stream) {
    const cllm::WType wt = weight_type(weight_dtype);
    need(epilogue == 0 || epilogue == 1 || epilogue == 2, "epilogue must be 0, 1 or 2");
    need(rpb == 0 || rpb == 1 || rpb == 2 || rpb == 4 || rpb == 8, "rpb must be 0, 1, 2, 4 or 8");
    need(wt != cllm::WType::INT4 || cols % 128 == 0, "int4 weights need cols to be a multiple of 128");
    const cllm::MatvecArgs a{w, scales, x, norm_w, eps, y, rows, cols};
    const auto ep = static_cast<cllm::Epilogue>(epilogue);
    cllm::launch_matvec(wt, ep, a, rpb ? rpb : cllm::default_rpb(wt, ep, rows, cols), static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" {

const char* cudallm_last_error(void) { return t_message.c_str(); }

void cudallm_default_options(cudallm_options* out) {
    if (out) *out = cudallm_options{1, 1, 1, 1, 0, 0};  // opt, opt, fused, graph, file max_seq_len, default rpb
}

int cudallm_create(const char* path, const cudallm_options* opts, cudallm_engine** out) {
    if (out) *out = nullptr;
    return abi_entry("cudallm_create", [&] {
        need(path && opts && out, "path, options and output handle are required");
        need(opts->matvec_impl == 0 || opts->matvec_impl == 1, "matvec_impl must be 0 or 1");
        need(opts->attn_impl == 0 || opts->attn_impl == 1, "attn_impl must be 0 or 1");
        cllm::EngineOptions o;
        o.matvec = opts->matvec_impl;
        o.attn = opts->attn_impl;
        o.fuse = opts->fuse != 0;
        o.graph = opts->cuda_graph != 0;
        o.max_seq_len = opts->max_seq_len;
        o.matvec_rpb = opts->matvec_rpb;
        auto handle = std::make_unique<cudallm_engine>();
        handle->impl = std::make_unique<cllm::Engine>(path, o);
        *out = handle.release();
    });
}

void cudallm_destroy(cudallm_engine* e) { delete e; }

int cudallm_get_config(cudallm_engine* e, cudallm_config_info* out) {
    return abi_entry("cudallm_get_config", [&] {
        cllm::Engine& eng = engine_of(e);
        need(out, "output struct is required");
        const cllm::ModelConfig& c = eng.config();
        cudallm_config_info info{};
        info.weight_dtype = static_cast<int>(c.wt);
        info.hidden = c.hidden;
        info.inter = c.inter;
        info.n_layers = c.n_layers;
        info.n_heads = c.n_heads;
        info.n_kv_heads = c.n_kv_heads;
        info.head_dim = c.head_dim;
        info.vocab = c.vocab;
        info.max_seq_len = eng.max_seq();  // the engine's (option) value, not necessarily the file's
        info.group_size = c.group_size;
        info.rms_eps = c.rms_eps;
        info.weight_bytes = eng.weight_bytes();
        *out = info;
    });
}

int cudallm_reset(cudallm_engine* e) {
    return abi_entry("cudallm_reset", [&] { engine_of(e).reset(); });
}

int cudallm_pos(cudallm_engine* e) {
    if (!e || !e->impl) {
        record(CUDALLM_ERR_INVALID_ARG, "cudallm_pos", "null engine handle");
        return -1;
    }
    return e->impl->pos();
}

int cudallm_step(cudallm_engine* e, int token, float* logits_out, int* next_token_out) {
    return abi_entry("cudallm_step", [&] { engine_of(e).step(token, logits_out, next_token_out); });
}

int cudallm_step_debug(cudallm_engine* e, int token, float* residuals_out, float* logits_out, int* next_token_out) {
    return abi_entry("cudallm_step_debug",
                     [&] { engine_of(e).step_debug(token, residuals_out, logits_out, next_token_out); });
}

int cudallm_step_profile(cudallm_engine* e, int token, unsigned long long* stamps_out, long long capacity,
                         int* grid_out) {
    return abi_entry("cudallm_step_profile", [&] {
        cllm::Engine& eng = engine_of(e);
        need(grid_out, "grid_out is required");
        *grid_out = eng.step_profile(token, stamps_out, static_cast<long>(capacity));
    });
}

int cudallm_step_trace(cudallm_engine* e, int token, float* trace_out, long long capacity, float* logits_out,
                       int* next_token_out) {
    return abi_entry("cudallm_step_trace", [&] {
        engine_of(e).step_trace(token, trace_out, static_cast<long>(capacity), logits_out, next_token_out);
    });
}

int cudallm_get_stream(cudallm_engine* e, void** stream_out) {
    if (stream_out) *stream_out = nullptr;
    return abi_entry("cudallm_get_stream", [&] {
        cllm::Engine& eng = engine_of(e);
        need(stream_out, "stream_out is required");
        *stream_out = eng.stream();
    });
}

int cudallm_get_step_kind(cudallm_engine* e, int* kind_out, int* grid_out) {
    if (kind_out) *kind_out = -1;
    if (grid_out) *grid_out = 0;
    return abi_entry("cudallm_get_step_kind", [&] {
        cllm::Engine& eng = engine_of(e);
        need(kind_out && grid_out, "kind_out and grid_out are required");
        *kind_out = eng.persistent() ? 1 : 0;
        *grid_out = eng.persistent() ? eng.grid() : 0;
    });
}

int cudallm_kernel_matvec(int impl, int weight_dtype, int epilogue, int fuse_norm, int rpb, const void* w,
                          unsigned long long w_bytes, const void* scales, unsigned long long scales_bytes,
                          const float* x, const float* norm_w, float eps, float* y, int rows, int cols) {
    return abi_entry("cudallm_kernel_matvec", [&] {
        const cllm::WType wt = weight_type(weight_dtype);
        need(impl == 0 || impl == 1, "impl must be 0 (naive) or 1 (opt)");
        need(epilogue == 0 || epilogue == 1 || epilogue == 2, "epilogue must be 0 (STORE), 1 (ADD) or 2 (SWIGLU)");
        need(rows > 0 && cols > 0, "rows and cols must be positive");
        need(w && x && y, "w, x and y are required");
        need(rpb == 0 || rpb == 1 || rpb == 2 || rpb == 4 || rpb == 8, "rpb must be 0, 1, 2, 4 or 8");
        const auto ep = static_cast<cllm::Epilogue>(epilogue);
        need(impl == 1 || (wt == cllm::WType::BF16 && ep == cllm::Epilogue::STORE && !fuse_norm),
             "the naive kernel takes bf16 weights, the STORE epilogue and no fused norm only");
        need(!fuse_norm || norm_w, "fuse_norm is set but norm_w is null");
        const uint64_t n = static_cast<uint64_t>(rows) * static_cast<uint64_t>(cols);
        // What the shape needs of each buffer; the kernels never read past what the caller passed.
        uint64_t w_need = 2 * n, s_need = 0;
        if (wt == cllm::WType::INT8) w_need = n, s_need = 4ull * rows;
        if (wt == cllm::WType::INT4) {
            need(cols % 128 == 0, "int4 weights need cols to be a multiple of 128");
            w_need = n / 2, s_need = 2ull * rows * (cols / 128);
        }
        need(w_bytes >= w_need, "w_bytes does not cover rows x cols");
        need(s_need == 0 || (scales && scales_bytes >= s_need),
             "quantised weights need scales (scales_bytes covering every row or group)");
        const int y_rows = ep == cllm::Epilogue::SWIGLU ? rows / 2 : rows;

        HookStaging st;
        const int sw = st.add(w, w_bytes, HookStaging::In);
        const int ss = st.add(scales, scales ? scales_bytes : 0, HookStaging::In);
        const int sx = st.add(x, sizeof(float) * cols, HookStaging::In);
        const int sn = st.add(norm_w, fuse_norm ? sizeof(float) * cols : 0, HookStaging::In);
        const int sy = st.add(y, sizeof(float) * y_rows, HookStaging::InOut);  // ADD reads y
        st.upload();
        const cllm::MatvecArgs a{st.dev<void>(sw), st.dev<void>(ss), st.dev<float>(sx), st.dev<float>(sn), eps,
                                 st.dev<float>(sy), rows, cols};
        if (impl == 0)
            cllm::launch_matvec_naive(a, nullptr);
        else
            cllm::launch_matvec(wt, ep, a, rpb ? rpb : cllm::default_rpb(wt, ep, rows, cols), nullptr);
        st.finish();
    });
}

int cudallm_kernel_rmsnorm(const float* x, const float* w, float eps, float* y, int n) {
    return abi_entry("cudallm_kernel_rmsnorm", [&] {
        need(x && w && y && n > 0, "x, w and y are required and n must be positive");
        HookStaging st;
        const size_t b = sizeof(float) * n;
        const int sx = st.add(x, b, HookStaging::In), sw = st.add(w, b, HookStaging::In), sy = st.add(y, b, HookStaging::Out);
        st.upload();
        cllm::launch_rmsnorm(st.dev<float>(sx), st.dev<float>(sw), eps, st.dev<float>(sy), n, nullptr);
        st.finish();
    });
}

int cudallm_kernel_rope_kv(int fused, float* qkv, const float* inv_freq, int pos, unsigned short* k_cache,
                           unsigned short* v_cache, int nh, int nkv, int hd, int max_seq) {
    return abi_entry("cudallm_kernel_rope_kv", [&] {
        need(qkv && inv_freq && k_cache && v_cache, "qkv, inv_freq and both caches are required");
        need(nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && max_seq > 0, "head counts, an even head_dim and max_seq must be positive");
        need(pos >= 0 && pos < max_seq, "pos must lie in [0, max_seq)");
        const size_t cache = sizeof(uint16_t) * static_cast<size_t>(nkv) * max_seq * hd;
        HookStaging st;
        const int sq = st.add(qkv, sizeof(float) * (nh + 2 * nkv) * hd, HookStaging::InOut);
        const int si = st.add(inv_freq, sizeof(float) * (hd / 2), HookStaging::In);
        const int sk = st.add(k_cache, cache, HookStaging::InOut), sv = st.add(v_cache, cache, HookStaging::InOut);
        const int sp = st.add(&pos, sizeof(int), HookStaging::In);
        st.upload();
        float* q = st.dev<float>(sq);
        uint16_t *kc = st.dev<uint16_t>(sk), *vc = st.dev<uint16_t>(sv);
        const int* dpos = st.dev<int>(sp);
        if (fused) {
            cllm::launch_rope_kv_fused(q, st.dev<float>(si), kc, vc, dpos, nh, nkv, hd, max_seq, nullptr);
        } else {
            cllm::launch_rope_inplace(q, st.dev<float>(si), dpos, nh, nkv, hd, nullptr);
            cllm::launch_kv_write(q, kc, vc, dpos, nh, nkv, hd, max_seq, nullptr);
        }
        st.finish();
    });
}

int cudallm_kernel_attention(int impl, const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                             int ctx, float* out, int nh, int nkv, int hd, int max_seq) {
    return abi_entry("cudallm_kernel_attention", [&] {
        need(impl == 0 || impl == 1, "impl must be 0 (naive) or 1 (split-K)");
        need(q && k_cache && v_cache && out, "q, both caches and out are required");
        need(nh > 0 && nkv > 0 && hd > 0 && max_seq > 0, "head counts, head_dim and max_seq must be positive");
        need(ctx >= 1 && ctx <= max_seq, "ctx must lie in [1, max_seq]");
        const size_t cache = sizeof(uint16_t) * static_cast<size_t>(nkv) * max_seq * hd;
        const size_t splits = (static_cast<size_t>(max_seq) + cllm::kAttnChunk - 1) / cllm::kAttnChunk;
        const int pos = ctx - 1;
        HookStaging st;
        const int sq = st.add(q, sizeof(float) * nh * hd, HookStaging::In);
        const int sk = st.add(k_cache, cache, HookStaging::In), sv = st.add(v_cache, cache, HookStaging::In);
        const int sp = st.add(&pos, sizeof(int), HookStaging::In);
        const int so = st.add(out, sizeof(float) * nh * hd, HookStaging::Out);
        const int spo = st.add(nullptr, impl ? sizeof(float) * nh * splits * hd : 0, HookStaging::Scratch);
        const int spm = st.add(nullptr, impl ? sizeof(float) * nh * splits * 2 : 0, HookStaging::Scratch);
        st.upload();
        if (impl == 0)
            cllm::launch_attention_naive(st.dev<float>(sq), st.dev<uint16_t>(sk), st.dev<uint16_t>(sv), st.dev<int>(sp),
                                         st.dev<float>(so), nh, nkv, hd, max_seq, nullptr);
        else
            cllm::launch_attention_splitk(st.dev<float>(sq), st.dev<uint16_t>(sk), st.dev<uint16_t>(sv), st.dev<int>(sp),
                                          st.dev<float>(spo), st.dev<float>(spm), st.dev<float>(so), nh, nkv, hd,
                                          max_seq, nullptr);
        st.finish();
    });
}

int cudallm_kernel_silu_mul(const float* gu, float* act, int inter) {
    return abi_entry("cudallm_kernel_silu_mul", [&] {
        need(gu && act && inter > 0, "gu and act are required and inter must be positive");
        HookStaging st;
        const int sg = st.add(gu, sizeof(float) * 2 * inter, HookStaging::In);
        const int sa = st.add(act, sizeof(float) * inter, HookStaging::Out);
        st.upload();
        cllm::launch_silu_mul(st.dev<float>(sg), st.dev<float>(sa), inter, nullptr);
        st.finish();
    });
}

int cudallm_kernel_argmax(const float* logits, int n, int* out_idx) {
    return abi_entry("cudallm_kernel_argmax", [&] {
        need(logits && out_idx && n > 0, "logits and out_idx are required and n must be positive");
        const int zero[2] = {0, 0};  // token and position the kernel writes and advances
        HookStaging st;
        const int sl = st.add(logits, sizeof(float) * n, HookStaging::In);
        const int sv = st.add(nullptr, sizeof(float) * cllm::kArgmaxParts, HookStaging::Scratch);
        const int si = st.add(nullptr, sizeof(int) * cllm::kArgmaxParts, HookStaging::Scratch);
        const int stp = st.add(zero, sizeof(zero), HookStaging::In);
        st.upload();
        int* tp = st.dev<int>(stp);
        cllm::launch_argmax(st.dev<float>(sl), n, st.dev<float>(sv), st.dev<int>(si), tp, tp + 1, nullptr);
        st.finish();
        CLLM_HIP(hipMemcpy(out_idx, tp, sizeof(int), hipMemcpyDeviceToHost));
    });
}

int cudallm_launch_matvec(int weight_dtype, int epilogue, int rpb, const void* w, const void* scales, const float* x,
                          const float* norm_w, float eps, float* y, int rows, int cols, void* stream) {
    return abi_entry("cudallm_launch_matvec", [&] {
        enqueue_matvec(weight_dtype, epilogue, rpb, w, scales, x, norm_w, eps, y, rows, cols, stream);
    });
}

int cudallm_launch_matvec_timed(int weight_dtype, int epilogue, int rpb, const void* w, const void* scales,
                                const float* x, const float* norm_w, float eps, float* y, int rows, int cols,
                                void* stream, void* start_event, void* stop_event) {
    return abi_entry("cudallm_launch_matvec_timed", [&] {
        need(start_event && stop_event, "start_event and stop_event are required");
        struct Disarm {  // the events never stay armed for a later launch, also when this one is refused
            ~Disarm() { cllm::take_kernel_events(); }
        } disarm;
        cllm::arm_kernel_events(static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
        enqueue_matvec(weight_dtype, epilogue, rpb, w, scales, x, norm_w, eps, y, rows, cols, stream);
    });
}

int cudallm_launch_stream_read_timed(const void* src, unsigned long long bytes, int blocks_per_cu, unsigned* sink,
                                     unsigned long long sink_words, void* stream, void* start_event, void* stop_event) {
    return abi_entry("cudallm_launch_stream_read_timed", [&] {
        need(src && sink, "src and sink are required");
        need(start_event && stop_event, "start_event and stop_event are required");
        need(bytes >= (1ull << 20) && bytes % 16 == 0, "bytes must be >= 1 MiB and a multiple of 16");
        need(blocks_per_cu == 4 || blocks_per_cu == 8 || blocks_per_cu == 16, "blocks_per_cu must be 4, 8 or 16");
        struct Disarm {
            ~Disarm() { cllm::take_kernel_events(); }
        } disarm;
        cllm::arm_kernel_events(static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
        cllm::launch_stream_read(src, bytes, blocks_per_cu, sink, sink_words, static_cast<hipStream_t>(stream));
    });
}

int cudallm_launch_attention(const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                             const int* d_pos, float* part_o, float* part_ml, float* out, int nh, int nkv, int hd,
                             int max_seq, void* stream) {
    return abi_entry("cudallm_launch_attention", [&] {
        cllm::launch_attention_splitk(q, k_cache, v_cache, d_pos, part_o, part_ml, out, nh, nkv, hd, max_seq,
                                      static_cast<hipStream_t>(stream));
    });
}

int cudallm_launch_attention_static(const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                                    const int* d_pos, float* out, int nh, int nkv, int hd, int max_seq, void* stream) {
    return abi_entry("cudallm_launch_attention_static", [&] {
        cllm::launch_attention_splitk_static(q, k_cache, v_cache, d_pos, out, nh, nkv, hd, max_seq,
                                             static_cast<hipStream_t>(stream));
    });
}

int cudallm_measure_read_bandwidth(unsigned long long bytes, int reps, double* best_gbps, double* median_gbps) {
    return abi_entry("cudallm_measure_read_bandwidth", [&] {
        need(best_gbps && median_gbps, "best_gbps and median_gbps are required");
        const cllm::ReadBandwidth r = cllm::measure_read_bandwidth(bytes, reps);
        *best_gbps = r.best_gbps;
        *median_gbps = r.median_gbps;
    });
}

int cudallm_quantize_int8_rows(const float* w, int rows, int cols, signed char* q_out, float* scales_out) {
    return abi_entry("cudallm_quantize_int8_rows", [&] {
        need(w && q_out && scales_out && rows > 0 && cols > 0, "w, q_out and scales_out are required; shape positive");
        const size_t n = static_cast<size_t>(rows) * cols;
        HookStaging st;
        const int sw = st.add(w, 4 * n, HookStaging::In);
        const int sq = st.add(q_out, n, HookStaging::Out), ss = st.add(scales_out, 4ull * rows, HookStaging::Out);
        st.upload();
        cllm::launch_quantize_int8_rows(st.dev<float>(sw), rows, cols, st.dev<int8_t>(sq), st.dev<float>(ss), nullptr);
        st.finish();
    });
}

int cudallm_quantize_int4_groups(const float* w, int rows, int cols, int group, unsigned char* packed_out,
                                 unsigned short* scales_out) {
    return abi_entry("cudallm_quantize_int4_groups", [&] {
        need(w && packed_out && scales_out && rows > 0 && cols > 0, "w, packed_out and scales_out are required; shape positive");
        need(group == 128, "group must be 128");
        need(cols % 128 == 0, "cols must be a multiple of 128");
        const size_t n = static_cast<size_t>(rows) * cols;
        HookStaging st;
        const int sw = st.add(w, 4 * n, HookStaging::In);
        const int sp = st.add(packed_out, n / 2, HookStaging::Out);
        const int ss = st.add(scales_out, 2 * static_cast<size_t>(rows) * (cols / 128), HookStaging::Out);
        st.upload();
        cllm::launch_quantize_int4_groups(st.dev<float>(sw), rows, cols, st.dev<uint8_t>(sp), st.dev<uint16_t>(ss),
                                          nullptr);
        st.finish();
    });
}

int cudallm_unpack_int4(const unsigned char* packed, int rows, int cols, signed char* q_out) {
    return abi_entry("cudallm_unpack_int4", [&] {
        need(packed && q_out && rows > 0 && cols > 0 && cols % 2 == 0, "packed and q_out are required; cols even and positive");
        const size_t n = static_cast<size_t>(rows) * cols;
        HookStaging st;
        const int sp = st.add(packed, n / 2, HookStaging::In), sq = st.add(q_out, n, HookStaging::Out);
        st.upload();
        cllm::launch_unpack_int4(st.dev<uint8_t>(sp), rows, cols, st.dev<int8_t>(sq), nullptr);
        st.finish();
    });
}

}  // extern "C"
