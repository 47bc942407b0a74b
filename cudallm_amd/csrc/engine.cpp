// Decode engine.  Op order and step semantics follow reference src/engine/engine.cpp:117-237:
//
//   fused:   embedding; per layer { qkv (+attn_norm) ; rope_kv ; attention ; wo (+=x) ;
//                                   gate_up (+ffn_norm, SwiGLU) ; down (+=x) } ; lm_head (+final_norm) ; argmax
//   unfused: the same with standalone rmsnorm / add / silu_mul kernels and rope_inplace + kv_write.
//
// The token and position live in device memory (argmax writes the token and advances the
// position), so every step is the same launch: the persistent kernel, or one captured hipGraph of the
// multi-kernel step; the host only enqueues it.
#include "engine.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

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
        // Persistent decode kernel: fused + opt options, contexts up to 8192 (one split per lane
        // in the LSE merge), and one co-resident workgroup per CU (64 to 4096 CUs).  CUDALLM_PERSISTENT=0 selects
        // the kernel-per-op graph instead (for comparisons).
        const char* env = std::getenv("CUDALLM_PERSISTENT");
        const bool want = opts_.fuse && opts_.matvec == 1 && opts_.attn == 1 && S <= 8192 && !(env && !std::strcmp(env, "0"));
        grid_ = device_cu_count();
        persistent_ = want && grid_ >= kDecodeMinGrid && grid_ <= kDecodeMaxGrid && decode_max_grid(c.wt) >= grid_;
        const size_t QKV = (NH + 2 * KV) * D;
        const size_t o_tx = cv.take<uint64_t>((L + 1) * H), o_txa = cv.take<uint64_t>(L * H),
                     o_tqkv = cv.take<uint64_t>(L * QKV), o_tatt = cv.take<uint64_t>(L * NH * D),
                     o_tpart = cv.take<uint64_t>(persistent_ ? L * NH * NS * (D + 2) : 1),
                     o_tact = cv.take<uint64_t>(L * I), o_targ = cv.take<uint64_t>(2 * 4096),
                     o_res = cv.take<float>((L + 1) * H), o_layers = cv.take<DecodeLayer>(L),
                     o_step = cv.take<unsigned>(1), o_err = cv.take<unsigned>(1),
                     o_stamps = cv.take<unsigned long long>(static_cast<size_t>(grid_) * kStampSlots);
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
        d_res_ = reinterpret_cast<float*>(b + o_res);
        d_err_ = reinterpret_cast<unsigned*>(b + o_err);
        d_stamps_ = reinterpret_cast<unsigned long long*>(b + o_stamps);
        const Weights& W = *weights_;
        std::vector<DecodeLayer> table(L);
        for (size_t l = 0; l < L; ++l) {
            const LayerWeights& lw = W.layers[l];
            table[l] = {lw.attn_norm, lw.wqkv.w, lw.wqkv.scales, lw.wo.w, lw.wo.scales,
                        lw.ffn_norm, lw.w_gate_up.w, lw.w_gate_up.scales, lw.w_down.w, lw.w_down.scales};
        }
        auto* d_layers = reinterpret_cast<DecodeLayer*>(b + o_layers);
        CLLM_HIP(hipMemcpy(d_layers, table.data(), sizeof(DecodeLayer) * L, hipMemcpyHostToDevice));
        const unsigned one = 1;  // tags of step 0 would equal the zero-filled buffers
        CLLM_HIP(hipMemcpy(b + o_step, &one, sizeof(one), hipMemcpyHostToDevice));
        dp_.layers = d_layers;
        dp_.emb = W.tok_embeddings.w;
        dp_.emb_s = W.tok_embeddings.scales;
        dp_.inv_freq = W.inv_freq;
        dp_.final_norm = W.final_norm;
        dp_.k_cache = k_cache_;
        dp_.v_cache = v_cache_;
        dp_.max_seq = max_seq_;
        dp_.tx = reinterpret_cast<uint64_t*>(b + o_tx);
        dp_.txa = reinterpret_cast<uint64_t*>(b + o_txa);
        dp_.tqkv = reinterpret_cast<uint64_t*>(b + o_tqkv);
        dp_.tatt = reinterpret_cast<uint64_t*>(b + o_tatt);
        dp_.tpart = reinterpret_cast<uint64_t*>(b + o_tpart);
        dp_.tact = reinterpret_cast<uint64_t*>(b + o_tact);
        dp_.targ = reinterpret_cast<uint64_t*>(b + o_targ);
        dp_.logits = logits_;
        dp_.d_token = d_token_;
        dp_.d_pos = d_pos_;
        dp_.d_step = reinterpret_cast<unsigned*>(b + o_step);
        dp_.d_err = d_err_;
        dp_.residuals = nullptr;
        dp_.stamps = nullptr;
        dp_.eps = c.rms_eps;
        const char* stall = std::getenv("CUDALLM_STALL");  // timing perturbation for tests only
        dp_.stall = stall ? static_cast<unsigned>(std::strtoul(stall, nullptr, 0)) : 0u;
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

void Engine::check_device_error() {
    unsigned e = 0;
    CLLM_HIP(hipMemcpy(&e, d_err_, sizeof(e), hipMemcpyDeviceToHost));
    if (e) {
        throw DeviceError(
            "persistent decode kernel: a cross-workgroup wait exceeded its bound (were all workgroups "
            "co-resident? another process may be sharing the GPU); the results of this sequence are invalid");
    }
}

void Engine::reset() {
    CLLM_HIP(hipStreamSynchronize(stream_));
    if (persistent_) check_device_error();
    launch_set_token(d_pos_, 0, stream_);  // a kernel, not a memset
    CLLM_HIP(hipStreamSynchronize(stream_));
    host_pos_ = 0;
}

void Engine::step(int token, float* logits_out, int* next_token_out) {
    if (host_pos_ >= max_seq_) throw SequenceFull("step: the sequence is full (pos == max_seq_len); call reset()");
    CLLM_REQUIRE(token >= -1 && token < config().vocab, "step: token out of range");
    if (token >= 0) launch_set_token(d_token_, token, stream_);
    // The persistent step is one kernel, launched directly with or without cuda_graph: replaying it as a one-node
    // graph left 8.8 us between consecutive kernels on MI355X against 4.1 us for a plain launch.  The
    // multi-kernel step is captured once and replayed.
    if (opts_.graph && !persistent_) {
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
    } else if (persistent_) {
        launch_decode(config().wt, dp_, grid_, stream_);
    } else {
        enqueue_forward(nullptr);
    }
    host_pos_ += 1;
    if (logits_out || next_token_out) {
        CLLM_HIP(hipStreamSynchronize(stream_));
        if (persistent_) check_device_error();
        if (logits_out)
            CLLM_HIP(hipMemcpy(logits_out, logits_, sizeof(float) * config().vocab, hipMemcpyDeviceToHost));
        if (next_token_out) CLLM_HIP(hipMemcpy(next_token_out, d_token_, sizeof(int), hipMemcpyDeviceToHost));
    }
}

void Engine::step_debug(int token, float* residuals_out, float* logits_out, int* next_token_out) {
    if (host_pos_ >= max_seq_) throw SequenceFull("step_debug: the sequence is full (pos == max_seq_len); call reset()");
    CLLM_REQUIRE(token >= -1 && token < config().vocab, "step_debug: token out of range");
    CLLM_REQUIRE(residuals_out, "step_debug: residuals_out is null");
    if (token >= 0) launch_set_token(d_token_, token, stream_);
    if (persistent_) {
        DecodeParams p = dp_;
        p.residuals = d_res_;
        launch_decode(config().wt, p, grid_, stream_);
    } else {
        enqueue_forward(residuals_out);
    }
    host_pos_ += 1;
    CLLM_HIP(hipStreamSynchronize(stream_));
    if (persistent_) {
        check_device_error();
        const ModelConfig& c = config();
        CLLM_HIP(hipMemcpy(residuals_out, d_res_, sizeof(float) * (c.n_layers + 1) * c.hidden, hipMemcpyDeviceToHost));
    }
    if (logits_out) CLLM_HIP(hipMemcpy(logits_out, logits_, sizeof(float) * config().vocab, hipMemcpyDeviceToHost));
    if (next_token_out) CLLM_HIP(hipMemcpy(next_token_out, d_token_, sizeof(int), hipMemcpyDeviceToHost));
}

int Engine::step_profile(int token, unsigned long long* stamps_out, long capacity) {
    if (!persistent_) throw StateError("step_profile: this engine does not use the persistent decode kernel");
    if (host_pos_ >= max_seq_) throw SequenceFull("step_profile: the sequence is full (pos == max_seq_len); call reset()");
    CLLM_REQUIRE(token >= -1 && token < config().vocab, "step_profile: token out of range");
    CLLM_REQUIRE(stamps_out && capacity >= static_cast<long>(grid_) * kStampSlots,
                 "step_profile: stamps_out must hold grid * 128 values");
    if (token >= 0) launch_set_token(d_token_, token, stream_);
    CLLM_HIP(hipMemsetAsync(d_stamps_, 0, sizeof(unsigned long long) * grid_ * kStampSlots, stream_));
    DecodeParams p = dp_;
    p.stamps = d_stamps_;
    launch_decode(config().wt, p, grid_, stream_);
    host_pos_ += 1;
    CLLM_HIP(hipStreamSynchronize(stream_));
    check_device_error();
    CLLM_HIP(hipMemcpy(stamps_out, d_stamps_, sizeof(unsigned long long) * grid_ * kStampSlots, hipMemcpyDeviceToHost));
    return grid_;
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
