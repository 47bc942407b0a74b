// Decode engine.  Op order and step semantics follow reference src/engine/engine.cpp:117-237:
//
//   fused:   embedding; per layer { qkv (+attn_norm) ; rope_kv ; attention ; wo (+=x) ;
//                                   gate_up (+ffn_norm, SwiGLU) ; down (+=x) } ; lm_head (+final_norm) ; argmax
//   unfused: the same with standalone rmsnorm / add / silu_mul kernels and rope_inplace + kv_write.
//
// The token and position live in device memory (argmax writes the token and advances the
// position), so one captured hipGraph replays every step; the host only launches it.
#include "engine.h"

#include <cstdio>

namespace cllm {

void validate_options(const EngineOptions& o, const ModelConfig& c) {
    CLLM_REQUIRE(o.matvec == 0 || o.matvec == 1, "matvec_impl must be 0 or 1");
    CLLM_REQUIRE(o.attn == 0 || o.attn == 1, "attn_impl must be 0 or 1");
    if (o.matvec == 0) {
        CLLM_REQUIRE(c.wt == WType::BF16, "the naive matvec needs bf16 weights");
        CLLM_REQUIRE(!o.fuse, "the naive matvec needs fuse = 0");
    }
    CLLM_REQUIRE(o.matvec_rpb == 0 || o.matvec_rpb == 1 || o.matvec_rpb == 2 || o.matvec_rpb == 4 || o.matvec_rpb == 8,
                 "matvec_rpb must be 0, 1, 2, 4 or 8");
    CLLM_REQUIRE(o.max_seq_len >= 0 && o.max_seq_len % 128 == 0, "max_seq_len must be 0 or a positive multiple of 128");
    CLLM_REQUIRE(o.max_seq_len <= c.max_seq_len, "max_seq_len exceeds the file's max_seq_len");
}

namespace {

// Bump allocation inside one arena, 256-byte aligned slots.
struct Carver {
    size_t off = 0;
    template <typename T>
    size_t take(size_t count) {
        const size_t at = off;
        off = (off + count * sizeof(T) + 255) & ~size_t(255);
        return at;
    }
};

}  // namespace

Engine::Engine(const std::string& path, const EngineOptions& opts) : opts_(opts) {
    {
        // Validate file and options before any device work.
        const ParsedFile pf = parse_file(path);
        validate_options(opts_, pf.config);
    }
    weights_ = std::make_unique<Weights>(path);
    const ModelConfig& c = weights_->config();
    max_seq_ = opts_.max_seq_len ? opts_.max_seq_len : c.max_seq_len;
    rpb_ = opts_.matvec_rpb ? opts_.matvec_rpb : default_rpb(c.wt);
    try {
        CLLM_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
        const size_t H = c.hidden, I = c.inter, V = c.vocab, S = max_seq_, KV = c.n_kv_heads, D = c.head_dim,
                     NH = c.n_heads, L = c.n_layers, NS = S / kAttnChunk;
        Carver cv;
        const size_t o_x = cv.take<float>(H), o_xb = cv.take<float>(H), o_qkv = cv.take<float>((NH + 2 * KV) * D),
                     o_att = cv.take<float>(NH * D), o_tmp = cv.take<float>(H), o_gu = cv.take<float>(2 * I),
                     o_act = cv.take<float>(I), o_log = cv.take<float>(V), o_po = cv.take<float>(NH * NS * D),
                     o_pml = cv.take<float>(NH * NS * 2), o_av = cv.take<float>(kArgmaxParts),
                     o_ai = cv.take<int>(kArgmaxParts), o_tok = cv.take<int>(1), o_pos = cv.take<int>(1),
                     o_k = cv.take<uint16_t>(L * KV * S * D), o_v = cv.take<uint16_t>(L * KV * S * D);
        CLLM_HIP(hipMalloc(&arena_, cv.off));
        CLLM_HIP(hipMemset(arena_, 0, cv.off));
        char* b = static_cast<char*>(arena_);
        x_ = reinterpret_cast<float*>(b + o_x);
        xb_ = reinterpret_cast<float*>(b + o_xb);
        qkv_ = reinterpret_cast<float*>(b + o_qkv);
        att_ = reinterpret_cast<float*>(b + o_att);
        tmp_ = reinterpret_cast<float*>(b + o_tmp);
        gu_ = reinterpret_cast<float*>(b + o_gu);
        act_ = reinterpret_cast<float*>(b + o_act);
        logits_ = reinterpret_cast<float*>(b + o_log);
        part_o_ = reinterpret_cast<float*>(b + o_po);
        part_ml_ = reinterpret_cast<float*>(b + o_pml);
        arg_v_ = reinterpret_cast<float*>(b + o_av);
        arg_i_ = reinterpret_cast<int*>(b + o_ai);
        d_token_ = reinterpret_cast<int*>(b + o_tok);
        d_pos_ = reinterpret_cast<int*>(b + o_pos);
        k_cache_ = reinterpret_cast<uint16_t*>(b + o_k);
        v_cache_ = reinterpret_cast<uint16_t*>(b + o_v);
        CLLM_HIP(hipDeviceSynchronize());
    } catch (...) {
        release();
        throw;
    }
}

void Engine::release() noexcept {
    auto report = [](hipError_t e, const char* what) {
        if (e != hipSuccess) std::fprintf(stderr, "cudallm: %s in ~Engine: %s\n", what, hipGetErrorString(e));
    };
    if (exec_) report(hipGraphExecDestroy(exec_), "hipGraphExecDestroy");
    if (graph_) report(hipGraphDestroy(graph_), "hipGraphDestroy");
    exec_ = nullptr;
    graph_ = nullptr;
    if (arena_) report(hipFree(arena_), "hipFree");
    arena_ = nullptr;
    if (stream_) report(hipStreamDestroy(stream_), "hipStreamDestroy");
    stream_ = nullptr;
}

Engine::~Engine() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    release();
}

void Engine::reset() {
    CLLM_HIP(hipStreamSynchronize(stream_));
    launch_set_token(d_pos_, 0, stream_);  // a kernel, not a memset
    CLLM_HIP(hipStreamSynchronize(stream_));
    host_pos_ = 0;
}

void Engine::step(int token, float* logits_out, int* next_token_out) {
    if (host_pos_ >= max_seq_) throw StateError("step: the sequence is full (pos == max_seq_len); call reset()");
    CLLM_REQUIRE(token >= -1 && token < config().vocab, "step: token out of range");
    if (token >= 0) launch_set_token(d_token_, token, stream_);
    if (opts_.graph) {
        if (!exec_) {
            CLLM_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
            try {
                enqueue_forward(nullptr);
            } catch (...) {
                hipGraph_t broken = nullptr;
                (void)hipStreamEndCapture(stream_, &broken);
                if (broken) (void)hipGraphDestroy(broken);
                throw;
            }
            CLLM_HIP(hipStreamEndCapture(stream_, &graph_));
            CLLM_HIP(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0));
        }
        CLLM_HIP(hipGraphLaunch(exec_, stream_));
    } else {
        enqueue_forward(nullptr);
    }
    host_pos_ += 1;
    if (logits_out || next_token_out) {
        CLLM_HIP(hipStreamSynchronize(stream_));
        if (logits_out)
            CLLM_HIP(hipMemcpy(logits_out, logits_, sizeof(float) * config().vocab, hipMemcpyDeviceToHost));
        if (next_token_out) CLLM_HIP(hipMemcpy(next_token_out, d_token_, sizeof(int), hipMemcpyDeviceToHost));
    }
}

void Engine::step_debug(int token, float* residuals_out, float* logits_out, int* next_token_out) {
    if (host_pos_ >= max_seq_) throw StateError("step_debug: the sequence is full (pos == max_seq_len); call reset()");
    CLLM_REQUIRE(token >= -1 && token < config().vocab, "step_debug: token out of range");
    CLLM_REQUIRE(residuals_out, "step_debug: residuals_out is null");
    if (token >= 0) launch_set_token(d_token_, token, stream_);
    enqueue_forward(residuals_out);
    host_pos_ += 1;
    CLLM_HIP(hipStreamSynchronize(stream_));
    if (logits_out) CLLM_HIP(hipMemcpy(logits_out, logits_, sizeof(float) * config().vocab, hipMemcpyDeviceToHost));
    if (next_token_out) CLLM_HIP(hipMemcpy(next_token_out, d_token_, sizeof(int), hipMemcpyDeviceToHost));
}

void Engine::linear(const Linear& L, const float* x, float* y, Epilogue ep, const float* norm_w) {
    MatvecArgs a{L.w, L.scales, x, norm_w, config().rms_eps, y, L.rows, L.cols};
    if (opts_.matvec == 0) {
        CLLM_INTERNAL(ep == Epilogue::STORE && !norm_w, "naive matvec: STORE only");
        launch_matvec_naive(a, stream_);
    } else {
        launch_matvec(L.wt, ep, a, rpb_, stream_);
    }
}

void Engine::enqueue_forward(float* residuals_out) {
    const ModelConfig& c = config();
    const Weights& W = *weights_;
    const int H = c.hidden, NH = c.n_heads, KV = c.n_kv_heads, D = c.head_dim;
    const size_t layer_cache = static_cast<size_t>(KV) * max_seq_ * D;
    auto snapshot = [&](int k) {
        if (!residuals_out) return;
        CLLM_HIP(hipStreamSynchronize(stream_));
        CLLM_HIP(hipMemcpy(residuals_out + static_cast<size_t>(k) * H, x_, sizeof(float) * H, hipMemcpyDeviceToHost));
    };
    const Linear& E = W.tok_embeddings;
    launch_embedding(E.wt, E.w, E.scales, d_token_, x_, H, c.vocab, c.group_size, stream_);
    snapshot(0);
    for (int l = 0; l < c.n_layers; ++l) {
        const LayerWeights& L = W.layers[l];
        uint16_t* kl = k_cache_ + l * layer_cache;
        uint16_t* vl = v_cache_ + l * layer_cache;
        if (opts_.fuse) {
            linear(L.wqkv, x_, qkv_, Epilogue::STORE, L.attn_norm);
            launch_rope_kv_fused(qkv_, W.inv_freq, kl, vl, d_pos_, NH, KV, D, max_seq_, stream_);
        } else {
            launch_rmsnorm(x_, L.attn_norm, c.rms_eps, xb_, H, stream_);
            linear(L.wqkv, xb_, qkv_, Epilogue::STORE, nullptr);
            launch_rope_inplace(qkv_, W.inv_freq, d_pos_, NH, KV, D, stream_);
            launch_kv_write(qkv_, kl, vl, d_pos_, NH, KV, D, max_seq_, stream_);
        }
        if (opts_.attn == 0)
            launch_attention_naive(qkv_, kl, vl, d_pos_, att_, NH, KV, D, max_seq_, stream_);
        else
            launch_attention_splitk(qkv_, kl, vl, d_pos_, part_o_, part_ml_, att_, NH, KV, D, max_seq_, stream_);
        if (opts_.fuse) {
            linear(L.wo, att_, x_, Epilogue::ADD, nullptr);
            linear(L.w_gate_up, x_, act_, Epilogue::SWIGLU, L.ffn_norm);
            linear(L.w_down, act_, x_, Epilogue::ADD, nullptr);
        } else {
            linear(L.wo, att_, tmp_, Epilogue::STORE, nullptr);
            launch_add_inplace(x_, tmp_, H, stream_);
            launch_rmsnorm(x_, L.ffn_norm, c.rms_eps, xb_, H, stream_);
            linear(L.w_gate_up, xb_, gu_, Epilogue::STORE, nullptr);
            launch_silu_mul(gu_, act_, c.inter, stream_);
            linear(L.w_down, act_, tmp_, Epilogue::STORE, nullptr);
            launch_add_inplace(x_, tmp_, H, stream_);
        }
        snapshot(l + 1);
    }
    if (opts_.fuse) {
        linear(E, x_, logits_, Epilogue::STORE, W.final_norm);
    } else {
        launch_rmsnorm(x_, W.final_norm, c.rms_eps, xb_, H, stream_);
        linear(E, xb_, logits_, Epilogue::STORE, nullptr);
    }
    launch_argmax(logits_, c.vocab, arg_v_, arg_i_, d_token_, d_pos_, stream_);
}

}  // namespace cllm
