// The C ABI (include/cudallm/cudallm.h).  Behaviour of each entry point follows reference
// src/capi/cudallm_capi.cpp:84-316: every call is guarded, exceptions become error codes plus a
// thread-local message, test hooks are synchronous and allocate per call.
#include "cudallm/cudallm.h"

#include <cstring>
#include <string>

#include "engine.h"

struct cudallm_engine {
    cllm::Engine* impl;
};

namespace cllm {

[[noreturn]] void throw_hip(hipError_t err, const char* expr, const char* file, int line) {
    throw DeviceError(std::string("HIP error at ") + file + ":" + std::to_string(line) + ": " + expr + ": " +
                      hipGetErrorString(err));
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

thread_local std::string g_last_error;

int code_of(const std::exception& e) {
    if (dynamic_cast<const cllm::ArgError*>(&e)) return CUDALLM_ERR_INVALID_ARG;
    if (dynamic_cast<const cllm::FormatError*>(&e)) return CUDALLM_ERR_FORMAT;
    if (dynamic_cast<const cllm::IoError*>(&e)) return CUDALLM_ERR_IO;
    if (dynamic_cast<const cllm::DeviceError*>(&e)) return CUDALLM_ERR_CUDA;
    if (dynamic_cast<const cllm::StateError*>(&e)) return CUDALLM_ERR_STATE;
    return CUDALLM_ERR_INTERNAL;
}

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return CUDALLM_OK;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return code_of(e);
    } catch (...) {
        g_last_error = "unknown exception";
        return CUDALLM_ERR_INTERNAL;
    }
}

// Device buffer owned by one test-hook call.
class DevBuf {
public:
    explicit DevBuf(size_t bytes) : n_(bytes) {
        if (bytes) CLLM_HIP(hipMalloc(&p_, bytes));
    }
    ~DevBuf() {
        if (p_) (void)hipFree(p_);
    }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    template <typename T>
    T* as() const {
        return static_cast<T*>(p_);
    }
    void put(const void* src) {
        if (n_) CLLM_HIP(hipMemcpy(p_, src, n_, hipMemcpyHostToDevice));
    }
    void get(void* dst) const {
        if (n_) CLLM_HIP(hipMemcpy(dst, p_, n_, hipMemcpyDeviceToHost));
    }

private:
    void* p_ = nullptr;
    size_t n_;
};

void finish() {
    CLLM_HIP(hipGetLastError());
    CLLM_HIP(hipDeviceSynchronize());
}

cllm::WType weight_type(int code) {
    CLLM_REQUIRE(code == 1 || code == 3 || code == 4, "weight_dtype must be 1 (bf16), 3 (int8) or 4 (int4)");
    return static_cast<cllm::WType>(code);
}

}  // namespace

extern "C" {

const char* cudallm_last_error(void) { return g_last_error.c_str(); }

void cudallm_default_options(cudallm_options* out) {
    if (!out) return;
    out->matvec_impl = 1;
    out->attn_impl = 1;
    out->fuse = 1;
    out->cuda_graph = 1;
    out->max_seq_len = 0;
    out->matvec_rpb = 0;
}

int cudallm_create(const char* path, const cudallm_options* opts, cudallm_engine** out) {
    return guarded([&] {
        CLLM_REQUIRE(path && opts && out, "cudallm_create: null argument");
        *out = nullptr;
        CLLM_REQUIRE(opts->matvec_impl == 0 || opts->matvec_impl == 1, "matvec_impl must be 0 or 1");
        CLLM_REQUIRE(opts->attn_impl == 0 || opts->attn_impl == 1, "attn_impl must be 0 or 1");
        cllm::EngineOptions o;
        o.matvec = opts->matvec_impl;
        o.attn = opts->attn_impl;
        o.fuse = opts->fuse != 0;
        o.graph = opts->cuda_graph != 0;
        o.max_seq_len = opts->max_seq_len;
        o.matvec_rpb = opts->matvec_rpb;
        auto* e = new cudallm_engine{nullptr};
        try {
            e->impl = new cllm::Engine(path, o);
        } catch (...) {
            delete e;
            throw;
        }
        *out = e;
    });
}

void cudallm_destroy(cudallm_engine* e) {
    if (!e) return;
    delete e->impl;
    delete e;
}

int cudallm_get_config(cudallm_engine* e, cudallm_config_info* out) {
    return guarded([&] {
        CLLM_REQUIRE(e && e->impl && out, "cudallm_get_config: null argument");
        const cllm::ModelConfig& c = e->impl->config();
        out->weight_dtype = static_cast<int>(c.wt);
        out->hidden = c.hidden;
        out->inter = c.inter;
        out->n_layers = c.n_layers;
        out->n_heads = c.n_heads;
        out->n_kv_heads = c.n_kv_heads;
        out->head_dim = c.head_dim;
        out->vocab = c.vocab;
        out->max_seq_len = e->impl->max_seq();
        out->group_size = c.group_size;
        out->rms_eps = c.rms_eps;
        out->weight_bytes = e->impl->weight_bytes();
    });
}

int cudallm_reset(cudallm_engine* e) {
    return guarded([&] {
        CLLM_REQUIRE(e && e->impl, "cudallm_reset: null engine");
        e->impl->reset();
    });
}

int cudallm_pos(cudallm_engine* e) {
    if (!e || !e->impl) {
        g_last_error = "cudallm_pos: null engine";
        return -1;
    }
    return e->impl->pos();
}

int cudallm_step(cudallm_engine* e, int token, float* logits_out, int* next_token_out) {
    return guarded([&] {
        CLLM_REQUIRE(e && e->impl, "cudallm_step: null engine");
        CLLM_REQUIRE(token >= -1, "cudallm_step: token must be >= -1");
        e->impl->step(token, logits_out, next_token_out);
    });
}

int cudallm_step_debug(cudallm_engine* e, int token, float* residuals_out, float* logits_out, int* next_token_out) {
    return guarded([&] {
        CLLM_REQUIRE(e && e->impl, "cudallm_step_debug: null engine");
        CLLM_REQUIRE(token >= -1, "cudallm_step_debug: token must be >= -1");
        CLLM_REQUIRE(residuals_out, "cudallm_step_debug: residuals_out is null");
        e->impl->step_debug(token, residuals_out, logits_out, next_token_out);
    });
}

int cudallm_step_profile(cudallm_engine* e, int token, unsigned long long* stamps_out, long long capacity,
                         int* grid_out) {
    return guarded([&] {
        CLLM_REQUIRE(e && e->impl && grid_out, "cudallm_step_profile: null argument");
        CLLM_REQUIRE(token >= -1, "cudallm_step_profile: token must be >= -1");
        *grid_out = e->impl->step_profile(token, stamps_out, static_cast<long>(capacity));
    });
}

int cudallm_get_stream(cudallm_engine* e, void** stream_out) {
    return guarded([&] {
        CLLM_REQUIRE(e && e->impl && stream_out, "cudallm_get_stream: null argument");
        *stream_out = e->impl->stream();
    });
}

int cudallm_kernel_matvec(int impl, int weight_dtype, int epilogue, int fuse_norm, int rpb, const void* w,
                          unsigned long long w_bytes, const void* scales, unsigned long long scales_bytes,
                          const float* x, const float* norm_w, float eps, float* y, int rows, int cols) {
    return guarded([&] {
        CLLM_REQUIRE(w && x && y && w_bytes > 0, "cudallm_kernel_matvec: null argument");
        CLLM_REQUIRE(rows > 0 && cols > 0, "cudallm_kernel_matvec: bad shape");
        CLLM_REQUIRE(impl == 0 || impl == 1, "cudallm_kernel_matvec: impl must be 0 or 1");
        CLLM_REQUIRE(epilogue >= 0 && epilogue <= 2, "cudallm_kernel_matvec: bad epilogue");
        const cllm::WType wt = weight_type(weight_dtype);
        const auto ep = static_cast<cllm::Epilogue>(epilogue);
        if (impl == 0)
            CLLM_REQUIRE(wt == cllm::WType::BF16 && ep == cllm::Epilogue::STORE && !fuse_norm,
                         "cudallm_kernel_matvec: naive requires bf16, STORE and no fused norm");
        if (fuse_norm) CLLM_REQUIRE(norm_w, "cudallm_kernel_matvec: fuse_norm needs norm_w");
        if (wt != cllm::WType::BF16)
            CLLM_REQUIRE(scales && scales_bytes > 0, "cudallm_kernel_matvec: quantized weights need scales");
        CLLM_REQUIRE(rpb == 0 || rpb == 1 || rpb == 2 || rpb == 4 || rpb == 8,
                     "cudallm_kernel_matvec: rpb must be 0, 1, 2, 4 or 8");
        // Buffer sizes must cover the shape: the kernels never read past what the caller passed.
        const uint64_t n = static_cast<uint64_t>(rows) * cols;
        const uint64_t need_w = wt == cllm::WType::BF16 ? 2 * n : wt == cllm::WType::INT8 ? n : n / 2;
        CLLM_REQUIRE(w_bytes >= need_w, "cudallm_kernel_matvec: w_bytes is smaller than rows x cols needs");
        if (wt == cllm::WType::INT8)
            CLLM_REQUIRE(scales_bytes >= 4ull * rows, "cudallm_kernel_matvec: scales_bytes too small");
        if (wt == cllm::WType::INT4) {
            CLLM_REQUIRE(cols % 128 == 0, "cudallm_kernel_matvec: int4 needs cols % 128 == 0");
            CLLM_REQUIRE(scales_bytes >= 2ull * rows * (cols / 128), "cudallm_kernel_matvec: scales_bytes too small");
        }
        const int out_rows = ep == cllm::Epilogue::SWIGLU ? rows / 2 : rows;

        DevBuf dw(w_bytes), ds(scales ? scales_bytes : 0), dx(sizeof(float) * cols),
            dn(fuse_norm ? sizeof(float) * cols : 0), dy(sizeof(float) * out_rows);
        dw.put(w);
        if (scales) ds.put(scales);
        dx.put(x);
        if (fuse_norm) dn.put(norm_w);
        dy.put(y);
        cllm::MatvecArgs a{dw.as<void>(), scales ? ds.as<void>() : nullptr, dx.as<float>(),
                           fuse_norm ? dn.as<float>() : nullptr, eps, dy.as<float>(), rows, cols};
        if (impl == 0)
            cllm::launch_matvec_naive(a, nullptr);
        else
            cllm::launch_matvec(wt, ep, a, rpb ? rpb : cllm::default_rpb(wt), nullptr);
        finish();
        dy.get(y);
    });
}

int cudallm_kernel_rmsnorm(const float* x, const float* w, float eps, float* y, int n) {
    return guarded([&] {
        CLLM_REQUIRE(x && w && y && n > 0, "cudallm_kernel_rmsnorm: bad argument");
        const size_t bytes = sizeof(float) * n;
        DevBuf dx(bytes), dw(bytes), dy(bytes);
        dx.put(x);
        dw.put(w);
        cllm::launch_rmsnorm(dx.as<float>(), dw.as<float>(), eps, dy.as<float>(), n, nullptr);
        finish();
        dy.get(y);
    });
}

int cudallm_kernel_rope_kv(int fused, float* qkv, const float* inv_freq, int pos, unsigned short* k_cache,
                           unsigned short* v_cache, int nh, int nkv, int hd, int max_seq) {
    return guarded([&] {
        CLLM_REQUIRE(qkv && inv_freq && k_cache && v_cache, "cudallm_kernel_rope_kv: null argument");
        CLLM_REQUIRE(nh > 0 && nkv > 0 && hd > 0 && hd % 2 == 0 && max_seq > 0 && pos >= 0 && pos < max_seq,
                     "cudallm_kernel_rope_kv: bad dimensions");
        const size_t qkv_bytes = sizeof(float) * (nh + 2 * nkv) * hd;
        const size_t cache_bytes = sizeof(uint16_t) * static_cast<size_t>(nkv) * max_seq * hd;
        DevBuf dq(qkv_bytes), dinv(sizeof(float) * (hd / 2)), dk(cache_bytes), dv(cache_bytes), dpos(sizeof(int));
        dq.put(qkv);
        dinv.put(inv_freq);
        dk.put(k_cache);
        dv.put(v_cache);
        dpos.put(&pos);
        if (fused) {
            cllm::launch_rope_kv_fused(dq.as<float>(), dinv.as<float>(), dk.as<uint16_t>(), dv.as<uint16_t>(),
                                       dpos.as<int>(), nh, nkv, hd, max_seq, nullptr);
        } else {
            cllm::launch_rope_inplace(dq.as<float>(), dinv.as<float>(), dpos.as<int>(), nh, nkv, hd, nullptr);
            cllm::launch_kv_write(dq.as<float>(), dk.as<uint16_t>(), dv.as<uint16_t>(), dpos.as<int>(), nh, nkv, hd,
                                  max_seq, nullptr);
        }
        finish();
        dq.get(qkv);
        dk.get(k_cache);
        dv.get(v_cache);
    });
}

int cudallm_kernel_attention(int impl, const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                             int ctx, float* out, int nh, int nkv, int hd, int max_seq) {
    return guarded([&] {
        CLLM_REQUIRE(q && k_cache && v_cache && out, "cudallm_kernel_attention: null argument");
        CLLM_REQUIRE(impl == 0 || impl == 1, "cudallm_kernel_attention: impl must be 0 or 1");
        CLLM_REQUIRE(nh > 0 && nkv > 0 && hd > 0 && max_seq > 0 && ctx >= 1 && ctx <= max_seq,
                     "cudallm_kernel_attention: bad dimensions");
        const size_t q_bytes = sizeof(float) * nh * hd;
        const size_t cache_bytes = sizeof(uint16_t) * static_cast<size_t>(nkv) * max_seq * hd;
        const int pos = ctx - 1;
        const size_t n_split = (max_seq + cllm::kAttnChunk - 1) / cllm::kAttnChunk;
        DevBuf dq(q_bytes), dk(cache_bytes), dv(cache_bytes), dpos(sizeof(int)), dout(q_bytes),
            dpo(impl == 1 ? sizeof(float) * nh * n_split * hd : 0), dpml(impl == 1 ? sizeof(float) * nh * n_split * 2 : 0);
        dq.put(q);
        dk.put(k_cache);
        dv.put(v_cache);
        dpos.put(&pos);
        if (impl == 0)
            cllm::launch_attention_naive(dq.as<float>(), dk.as<uint16_t>(), dv.as<uint16_t>(), dpos.as<int>(),
                                         dout.as<float>(), nh, nkv, hd, max_seq, nullptr);
        else
            cllm::launch_attention_splitk(dq.as<float>(), dk.as<uint16_t>(), dv.as<uint16_t>(), dpos.as<int>(),
                                          dpo.as<float>(), dpml.as<float>(), dout.as<float>(), nh, nkv, hd, max_seq,
                                          nullptr);
        finish();
        dout.get(out);
    });
}

int cudallm_kernel_silu_mul(const float* gu, float* act, int inter) {
    return guarded([&] {
        CLLM_REQUIRE(gu && act && inter > 0, "cudallm_kernel_silu_mul: bad argument");
        DevBuf dgu(sizeof(float) * 2 * inter), dact(sizeof(float) * inter);
        dgu.put(gu);
        cllm::launch_silu_mul(dgu.as<float>(), dact.as<float>(), inter, nullptr);
        finish();
        dact.get(act);
    });
}

int cudallm_kernel_argmax(const float* logits, int n, int* out_idx) {
    return guarded([&] {
        CLLM_REQUIRE(logits && out_idx && n > 0, "cudallm_kernel_argmax: bad argument");
        DevBuf dl(sizeof(float) * n), dpv(sizeof(float) * cllm::kArgmaxParts), dpi(sizeof(int) * cllm::kArgmaxParts),
            dtok(sizeof(int)), dpos(sizeof(int));
        const int zero = 0;
        dl.put(logits);
        dtok.put(&zero);
        dpos.put(&zero);
        cllm::launch_argmax(dl.as<float>(), n, dpv.as<float>(), dpi.as<int>(), dtok.as<int>(), dpos.as<int>(), nullptr);
        finish();
        dtok.get(out_idx);
    });
}

int cudallm_launch_matvec(int weight_dtype, int epilogue, int rpb, const void* w, const void* scales, const float* x,
                          const float* norm_w, float eps, float* y, int rows, int cols, void* stream) {
    return guarded([&] {
        CLLM_REQUIRE(epilogue >= 0 && epilogue <= 2, "cudallm_launch_matvec: bad epilogue");
        CLLM_REQUIRE(rpb == 0 || rpb == 1 || rpb == 2 || rpb == 4 || rpb == 8, "cudallm_launch_matvec: bad rpb");
        const cllm::WType wt = weight_type(weight_dtype);
        if (wt == cllm::WType::INT4) CLLM_REQUIRE(cols % 128 == 0, "cudallm_launch_matvec: int4 needs cols % 128 == 0");
        cllm::MatvecArgs a{w, scales, x, norm_w, eps, y, rows, cols};
        cllm::launch_matvec(wt, static_cast<cllm::Epilogue>(epilogue), a, rpb ? rpb : cllm::default_rpb(wt),
                            static_cast<hipStream_t>(stream));
    });
}

int cudallm_launch_attention(const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                             const int* d_pos, float* part_o, float* part_ml, float* out, int nh, int nkv, int hd,
                             int max_seq, void* stream) {
    return guarded([&] {
        cllm::launch_attention_splitk(q, k_cache, v_cache, d_pos, part_o, part_ml, out, nh, nkv, hd, max_seq,
                                      static_cast<hipStream_t>(stream));
    });
}

int cudallm_quantize_int8_rows(const float* w, int rows, int cols, signed char* q_out, float* scales_out) {
    return guarded([&] {
        CLLM_REQUIRE(w && q_out && scales_out && rows > 0 && cols > 0, "cudallm_quantize_int8_rows: bad argument");
        const size_t n = static_cast<size_t>(rows) * cols;
        DevBuf dw(4 * n), dq(n), ds(4ull * rows);
        dw.put(w);
        cllm::launch_quantize_int8_rows(dw.as<float>(), rows, cols, dq.as<int8_t>(), ds.as<float>(), nullptr);
        finish();
        dq.get(q_out);
        ds.get(scales_out);
    });
}

int cudallm_quantize_int4_groups(const float* w, int rows, int cols, int group, unsigned char* packed_out,
                                 unsigned short* scales_out) {
    return guarded([&] {
        CLLM_REQUIRE(w && packed_out && scales_out && rows > 0 && cols > 0, "cudallm_quantize_int4_groups: bad argument");
        CLLM_REQUIRE(group == 128, "cudallm_quantize_int4_groups: group must be 128");
        CLLM_REQUIRE(cols % 128 == 0, "cudallm_quantize_int4_groups: cols must be a multiple of 128");
        const size_t n = static_cast<size_t>(rows) * cols;
        DevBuf dw(4 * n), dp(n / 2), ds(2 * static_cast<size_t>(rows) * (cols / 128));
        dw.put(w);
        cllm::launch_quantize_int4_groups(dw.as<float>(), rows, cols, dp.as<uint8_t>(), ds.as<uint16_t>(), nullptr);
        finish();
        dp.get(packed_out);
        ds.get(scales_out);
    });
}

int cudallm_unpack_int4(const unsigned char* packed, int rows, int cols, signed char* q_out) {
    return guarded([&] {
        CLLM_REQUIRE(packed && q_out && rows > 0 && cols > 0 && cols % 2 == 0, "cudallm_unpack_int4: bad argument");
        const size_t n = static_cast<size_t>(rows) * cols;
        DevBuf dp(n / 2), dq(n);
        dp.put(packed);
        cllm::launch_unpack_int4(dp.as<uint8_t>(), rows, cols, dq.as<int8_t>(), nullptr);
        finish();
        dq.get(q_out);
    });
}

}  // extern "C"
