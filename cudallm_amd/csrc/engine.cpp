// Decode engine.  What a step computes is the op order of reference src/engine/engine.cpp:181-237; how
// it is run is this file's own:
//
//  * Default options: the persistent decode kernel, one launch per token (its workgroups' co-residency is
//    verified once, at construction, by a probe launch).  Its
//    cross-workgroup handoffs are tagged words (decode.h) whose epochs the host restarts before the
//    32-bit tags could repeat.
//  * Ablation options: a step program, the list of kernel launches of one step in op order, built
//    once at construction.  With cuda_graph the program is captured into a hipGraph on first use and
//    replayed; step_debug runs it directly with its debug-only entries, device copies of the residual
//    stream into a snapshot buffer that the host reads once at the end.
//
// The token and position live in device memory (argmax writes the token and advances the position),
// so consecutive steps need no host round trip.
#include "engine.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <vector>

namespace cllm {

void validate_options(const EngineOptions& o, const ModelConfig& c) {
    const int r = o.matvec_rpb;
    const struct {
        bool ok;
        const char* why;
    } rules[] = {
        {o.matvec == 0 || o.matvec == 1, "options: matvec_impl is neither 0 (naive) nor 1 (opt)"},
        {o.attn == 0 || o.attn == 1, "options: attn_impl is neither 0 (naive) nor 1 (split-K)"},
        {o.matvec == 1 || c.wt == WType::BF16, "options: the naive matvec only reads bf16 weights"},
        {o.matvec == 1 || !o.fuse, "options: the naive matvec has no fused epilogues, so it needs fuse = 0"},
        {r == 0 || r == 1 || r == 2 || r == 4 || r == 8, "options: matvec_rpb takes 0, 1, 2, 4 or 8"},
        {o.max_seq_len >= 0 && o.max_seq_len % 128 == 0, "options: max_seq_len is neither 0 nor a positive multiple of 128"},
        {o.max_seq_len <= c.max_seq_len, "options: max_seq_len exceeds the context the file was written for"},
    };
    for (const auto& rule : rules)
        if (!rule.ok) throw ArgError(rule.why);
}

TraceLayout TraceLayout::of(const ModelConfig& c) {
    const size_t L = c.n_layers, H = c.hidden, QKV = static_cast<size_t>(c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
    TraceLayout t{};
    t.residuals = 0;
    t.qkv = (L + 1) * H;
    t.att = t.qkv + L * QKV;
    t.xa = t.att + L * static_cast<size_t>(c.n_heads) * c.head_dim;
    t.act = t.xa + L * H;
    t.total = t.act + L * static_cast<size_t>(c.inter);
    return t;
}

namespace {

// Sub-allocations of one arena, each 256-byte aligned.
class ArenaPlan {
public:
    template <typename T>
    size_t reserve(size_t count) {
        const size_t at = size_;
        size_ = (size_ + count * sizeof(T) + 255) / 256 * 256;
        return at;
    }
    size_t size() const { return size_; }

private:
    size_t size_ = 0;
};

// Records everything `record` enqueues on `s` into an executable graph.  The capture is ended on every
// path, so a failure inside `record` never leaves the stream capturing.
void capture_graph(hipStream_t s, const std::function<void()>& record, hipGraph_t* graph, hipGraphExec_t* exec) {
    CLLM_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    std::exception_ptr failed;
    try {
        record();
    } catch (...) {
        failed = std::current_exception();
    }
    hipGraph_t g = nullptr;
    const hipError_t ended = hipStreamEndCapture(s, &g);
    if (failed || ended != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        if (failed) std::rethrow_exception(failed);
        CLLM_HIP(ended);
    }
    const hipError_t made = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
    if (made != hipSuccess) {
        (void)hipGraphDestroy(g);
        CLLM_HIP(made);
    }
    *graph = g;
}

unsigned env_step_limit() {
    // Test hook: a smaller epoch limit makes the tag restart happen within a short sequence.
    const char* v = std::getenv("CUDALLM_EPOCH_LIMIT");
    if (!v) return kDecodeStepLimit;
    const unsigned long n = std::strtoul(v, nullptr, 0);
    return n >= 1 && n < kDecodeStepLimit ? static_cast<unsigned>(n) : kDecodeStepLimit;
}

}  // namespace

Engine::Engine(const std::string& path, const EngineOptions& opts) : opts_(opts) {
    // The file and the options are checked before any device work.
    validate_options(opts_, parse_file(path).config);
    weights_ = std::make_unique<Weights>(path);
    const ModelConfig& c = weights_->config();
    max_seq_ = opts_.max_seq_len ? opts_.max_seq_len : c.max_seq_len;
    rpb_ = opts_.matvec_rpb;  // 0: the library's per-shape choice (default_rpb)
    step_limit_ = env_step_limit();
    try {
        CLLM_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
        const size_t H = c.hidden, I = c.inter, V = c.vocab, S = max_seq_, KV = c.n_kv_heads, D = c.head_dim,
                     NH = c.n_heads, L = c.n_layers, NS = S / kAttnChunk, QKV = (NH + 2 * KV) * D;

        // The persistent kernel needs: the default options, one workgroup per CU with the grid a multiple of 8,
        // all of them resident at once (checked below with a probe launch), and a context it supports.
        // CUDALLM_PERSISTENT=0 selects the multi-kernel step instead (for comparisons).
        const char* env = std::getenv("CUDALLM_PERSISTENT");
        const bool wanted = opts_.fuse && opts_.matvec == 1 && opts_.attn == 1 && !(env && !std::strcmp(env, "0"));
        // CUDALLM_DECODE_GRID overrides the grid (a multiple of 8, at most the CU count) for grid-size sweeps.
        grid_ = device_cu_count();
        if (const char* g = std::getenv("CUDALLM_DECODE_GRID")) {
            const int want = std::atoi(g);
            CLLM_REQUIRE(want >= kDecodeMinGrid && want <= grid_ && want % 8 == 0,
                         "CUDALLM_DECODE_GRID: a multiple of 8, at least 64 and at most the CU count");
            grid_ = want;
        }
        persistent_ = wanted && S <= static_cast<size_t>(kDecodeMaxSeq) && grid_ % 8 == 0 &&
                      grid_ >= kDecodeMinGrid && grid_ <= kDecodeMaxGrid && decode_max_grid(c.wt) >= grid_;

        ArenaPlan ap;
        const size_t at_x = ap.reserve<float>(H), at_xb = ap.reserve<float>(H), at_qkv = ap.reserve<float>(QKV),
                     at_att = ap.reserve<float>(NH * D), at_tmp = ap.reserve<float>(H), at_gu = ap.reserve<float>(2 * I),
                     at_act = ap.reserve<float>(I), at_logits = ap.reserve<float>(V),
                     at_po = ap.reserve<float>(NH * NS * D), at_pml = ap.reserve<float>(NH * NS * 2),
                     at_av = ap.reserve<float>(kArgmaxParts), at_ai = ap.reserve<int>(kArgmaxParts),
                     at_tok = ap.reserve<int>(1), at_pos = ap.reserve<int>(1),
                     at_k = ap.reserve<uint16_t>(L * KV * S * D), at_v = ap.reserve<uint16_t>(L * KV * S * D),
                     at_res = ap.reserve<float>((L + 1) * H);
        // Tagged buffers of the persistent kernel, contiguous so that one clear covers them all.
        const size_t n_part = persistent_ ? L * NH * NS * (D + 2) : 1;
        const size_t at_tx = ap.reserve<uint64_t>((L + 1) * H), at_txa = ap.reserve<uint64_t>(L * H),
                     at_tqkv = ap.reserve<uint64_t>(L * QKV), at_tatt = ap.reserve<uint64_t>(L * NH * D),
                     at_tpart = ap.reserve<uint64_t>(n_part), at_tact = ap.reserve<uint64_t>(L * I),
                     at_targ = ap.reserve<uint64_t>(2 * kDecodeMaxGrid);
        const size_t at_tags_end = ap.size();
        const size_t at_layers = ap.reserve<DecodeLayer>(L), at_step = ap.reserve<unsigned>(1),
                     at_err = ap.reserve<unsigned>(1), at_probe = ap.reserve<unsigned>(2),
                     at_stamps = ap.reserve<unsigned long long>(static_cast<size_t>(grid_) * kStampSlots);
        CLLM_HIP(hipMalloc(&arena_, ap.size()));
        CLLM_HIP(hipMemset(arena_, 0, ap.size()));
        char* base = static_cast<char*>(arena_);
        auto at = [base](size_t off) { return static_cast<void*>(base + off); };
        x_ = static_cast<float*>(at(at_x));
        xb_ = static_cast<float*>(at(at_xb));
        qkv_ = static_cast<float*>(at(at_qkv));
        att_ = static_cast<float*>(at(at_att));
        tmp_ = static_cast<float*>(at(at_tmp));
        gu_ = static_cast<float*>(at(at_gu));
        act_ = static_cast<float*>(at(at_act));
        logits_ = static_cast<float*>(at(at_logits));
        part_o_ = static_cast<float*>(at(at_po));
        part_ml_ = static_cast<float*>(at(at_pml));
        arg_v_ = static_cast<float*>(at(at_av));
        arg_i_ = static_cast<int*>(at(at_ai));
        d_token_ = static_cast<int*>(at(at_tok));
        d_pos_ = static_cast<int*>(at(at_pos));
        k_cache_ = static_cast<uint16_t*>(at(at_k));
        v_cache_ = static_cast<uint16_t*>(at(at_v));
        d_res_ = static_cast<float*>(at(at_res));
        tags_begin_ = at(at_tx);
        tags_bytes_ = at_tags_end - at_tx;
        d_stamps_ = static_cast<unsigned long long*>(at(at_stamps));

        const Weights& W = *weights_;
        std::vector<DecodeLayer> table;
        table.reserve(L);
        for (const LayerWeights& lw : W.layers)
            table.push_back({lw.attn_norm, lw.wqkv.w, lw.wqkv.scales, lw.wo.w, lw.wo.scales, lw.ffn_norm,
                             lw.w_gate_up.w, lw.w_gate_up.scales, lw.w_down.w, lw.w_down.scales});
        auto* d_layers = static_cast<DecodeLayer*>(at(at_layers));
        CLLM_HIP(hipMemcpy(d_layers, table.data(), sizeof(DecodeLayer) * L, hipMemcpyHostToDevice));
        // The first launch uses step 1: tags of step 0 could only be confused with never-written words if the
        // counter started at -1, but starting at 1 keeps every live tag away from the zero-filled arena.
        const unsigned first_step = 1;
        CLLM_HIP(hipMemcpy(at(at_step), &first_step, sizeof(first_step), hipMemcpyHostToDevice));

        dp_ = DecodeParams{};
        dp_.layers = d_layers;
        dp_.emb = W.tok_embeddings.w;
        dp_.emb_s = W.tok_embeddings.scales;
        dp_.inv_freq = W.inv_freq;
        dp_.final_norm = W.final_norm;
        dp_.k_cache = k_cache_;
        dp_.v_cache = v_cache_;
        dp_.max_seq = max_seq_;
        dp_.tx = static_cast<uint64_t*>(at(at_tx));
        dp_.txa = static_cast<uint64_t*>(at(at_txa));
        dp_.tqkv = static_cast<uint64_t*>(at(at_tqkv));
        dp_.tatt = static_cast<uint64_t*>(at(at_tatt));
        dp_.tpart = static_cast<uint64_t*>(at(at_tpart));
        dp_.tact = static_cast<uint64_t*>(at(at_tact));
        dp_.targ = static_cast<uint64_t*>(at(at_targ));
        dp_.logits = logits_;
        dp_.d_token = d_token_;
        dp_.d_pos = d_pos_;
        dp_.d_step = static_cast<unsigned*>(at(at_step));
        dp_.d_err = static_cast<unsigned*>(at(at_err));
        dp_.eps = c.rms_eps;
        const char* stall = std::getenv("CUDALLM_STALL");  // timing perturbation, tests only
        dp_.stall = stall ? static_cast<unsigned>(std::strtoul(stall, nullptr, 0)) : 0u;

        CLLM_HIP(hipDeviceSynchronize());
        // Every workgroup of the persistent grid must be resident at once (their waits on each other would
        // otherwise only end at their bounds).  One probe launch checks it for this device and kernel; if it
        // fails (another process holding CUs, say), this engine runs the multi-kernel step instead.
        if (persistent_ && !decode_grid_is_resident(c.wt, dp_, grid_, static_cast<unsigned*>(at(at_probe)), stream_)) {
            std::fprintf(stderr, "cudallm: the %d workgroups of the persistent decode kernel were not all resident at "
                                 "once; using the multi-kernel step\n", grid_);
            persistent_ = false;
        }
        if (!persistent_) build_program();
        CLLM_HIP(hipDeviceSynchronize());
    } catch (...) {
        release();
        throw;
    }
}

void Engine::release() noexcept {
    auto check = [](hipError_t e, const char* what) {
        if (e != hipSuccess) std::fprintf(stderr, "cudallm: %s while destroying an engine: %s\n", what, hipGetErrorString(e));
    };
    if (graph_exec_) check(hipGraphExecDestroy(graph_exec_), "hipGraphExecDestroy");
    if (graph_) check(hipGraphDestroy(graph_), "hipGraphDestroy");
    graph_exec_ = nullptr;
    graph_ = nullptr;
    if (arena_) check(hipFree(arena_), "hipFree");
    arena_ = nullptr;
    if (stream_) check(hipStreamDestroy(stream_), "hipStreamDestroy");
    stream_ = nullptr;
}

Engine::~Engine() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    release();
}

// ---- the multi-kernel step ------------------------------------------------------------------

void Engine::build_program() {
    const ModelConfig& c = config();
    const Weights& W = *weights_;
    const int H = c.hidden, NH = c.n_heads, KV = c.n_kv_heads, D = c.head_dim, I = c.inter, ms = max_seq_;
    const float eps = c.rms_eps;
    const size_t cache_stride = static_cast<size_t>(KV) * max_seq_ * D;
    const bool naive_mv = opts_.matvec == 0, naive_attn = opts_.attn == 0;
    const int rpb = rpb_;
    auto emit = [this](std::function<void(hipStream_t)> f) { program_.push_back({false, std::move(f)}); };
    auto snapshot = [this, H](int k) {
        float* dst = d_res_ + static_cast<size_t>(k) * H;
        const float* src = x_;
        program_.push_back({true, [dst, src, H](hipStream_t s) {
                                CLLM_HIP(hipMemcpyAsync(dst, src, sizeof(float) * H, hipMemcpyDeviceToDevice, s));
                            }});
    };
    auto matvec = [&](const Linear& L, const float* in, float* out, Epilogue ep, const float* norm_w) {
        const MatvecArgs a{L.w, L.scales, in, norm_w, eps, out, L.rows, L.cols};
        const WType wt = L.wt;
        if (naive_mv) {
            CLLM_INTERNAL(ep == Epilogue::STORE && !norm_w, "naive matvec: STORE without a fused norm only");
            emit([a](hipStream_t s) { launch_matvec_naive(a, s); });
        } else {
            const int r = rpb ? rpb : default_rpb(wt, ep, a.rows, a.cols);
            emit([a, wt, ep, r](hipStream_t s) { launch_matvec(wt, ep, a, r, s); });
        }
    };
    float *x = x_, *xb = xb_, *qkv = qkv_, *att = att_, *tmp = tmp_, *gu = gu_, *act = act_;
    const int* pos = d_pos_;
    auto attention = [&](const uint16_t* kl, const uint16_t* vl) {
        if (naive_attn) {
            emit([=](hipStream_t s) { launch_attention_naive(qkv, kl, vl, pos, att, NH, KV, D, ms, s); });
        } else {
            float *po = part_o_, *pml = part_ml_;
            emit([=](hipStream_t s) { launch_attention_splitk(qkv, kl, vl, pos, po, pml, att, NH, KV, D, ms, s); });
        }
    };

    {
        const Linear E = W.tok_embeddings;
        const int* tok = d_token_;
        const int V = c.vocab, g = c.group_size;
        emit([=](hipStream_t s) { launch_embedding(E.wt, E.w, E.scales, tok, x, H, V, g, s); });
    }
    snapshot(0);
    for (int l = 0; l < c.n_layers; ++l) {
        const LayerWeights& lw = W.layers[l];
        uint16_t* kl = k_cache_ + l * cache_stride;
        uint16_t* vl = v_cache_ + l * cache_stride;
        const float* inv_freq = W.inv_freq;
        if (opts_.fuse) {
            matvec(lw.wqkv, x, qkv, Epilogue::STORE, lw.attn_norm);
            emit([=](hipStream_t s) { launch_rope_kv_fused(qkv, inv_freq, kl, vl, pos, NH, KV, D, ms, s); });
            attention(kl, vl);
            matvec(lw.wo, att, x, Epilogue::ADD, nullptr);
            matvec(lw.w_gate_up, x, act, Epilogue::SWIGLU, lw.ffn_norm);
            matvec(lw.w_down, act, x, Epilogue::ADD, nullptr);
        } else {
            const float *an = lw.attn_norm, *fn = lw.ffn_norm;
            emit([=](hipStream_t s) { launch_rmsnorm(x, an, eps, xb, H, s); });
            matvec(lw.wqkv, xb, qkv, Epilogue::STORE, nullptr);
            emit([=](hipStream_t s) { launch_rope_inplace(qkv, inv_freq, pos, NH, KV, D, s); });
            emit([=](hipStream_t s) { launch_kv_write(qkv, kl, vl, pos, NH, KV, D, ms, s); });
            attention(kl, vl);
            matvec(lw.wo, att, tmp, Epilogue::STORE, nullptr);
            emit([=](hipStream_t s) { launch_add_inplace(x, tmp, H, s); });
            emit([=](hipStream_t s) { launch_rmsnorm(x, fn, eps, xb, H, s); });
            matvec(lw.w_gate_up, xb, gu, Epilogue::STORE, nullptr);
            emit([=](hipStream_t s) { launch_silu_mul(gu, act, I, s); });
            matvec(lw.w_down, act, tmp, Epilogue::STORE, nullptr);
            emit([=](hipStream_t s) { launch_add_inplace(x, tmp, H, s); });
        }
        snapshot(l + 1);
    }
    if (opts_.fuse) {
        matvec(W.tok_embeddings, x, logits_, Epilogue::STORE, W.final_norm);
    } else {
        const float* fn = W.final_norm;
        emit([=](hipStream_t s) { launch_rmsnorm(x, fn, eps, xb, H, s); });
        matvec(W.tok_embeddings, xb, logits_, Epilogue::STORE, nullptr);
    }
    float *lg = logits_, *av = arg_v_;
    int *ai = arg_i_, *tok = d_token_, *dpos = d_pos_;
    const int V = c.vocab;
    emit([=](hipStream_t s) { launch_argmax(lg, V, av, ai, tok, dpos, s); });
}

void Engine::run_program(bool debug) {
    for (const Op& op : program_)
        if (debug || !op.debug_only) op.enqueue(stream_);
}

// ---- the persistent step --------------------------------------------------------------------

void Engine::launch_persistent(const DecodeParams& p) {
    if (launches_ >= step_limit_) {
        // Restart the epochs before the 32-bit tags could repeat: with every tagged word zero and the step
        // counter back at 0, no word written under the old numbering can carry a tag of the new one.
        CLLM_HIP(hipMemsetAsync(tags_begin_, 0, tags_bytes_, stream_));
        CLLM_HIP(hipMemsetAsync(dp_.d_step, 0, sizeof(unsigned), stream_));
        launches_ = 0;
    }
    launch_decode(config().wt, p, grid_, stream_);
    ++launches_;
}

void Engine::raise_if_kernel_failed() {
    if (!persistent_) return;
    unsigned flag = 0;
    CLLM_HIP(hipMemcpy(&flag, dp_.d_err, sizeof(flag), hipMemcpyDeviceToHost));
    if (flag)
        throw DeviceError(
            "persistent decode kernel: a wait on another workgroup ran past its bound, so this sequence's results are "
            "invalid; reset() starts a new sequence");
}

// ---- steps ----------------------------------------------------------------------------------

void Engine::reset() {
    CLLM_HIP(hipStreamSynchronize(stream_));
    unsigned flag = 0;
    if (persistent_) {
        CLLM_HIP(hipMemcpy(&flag, dp_.d_err, sizeof(flag), hipMemcpyDeviceToHost));
        if (flag) CLLM_HIP(hipMemsetAsync(dp_.d_err, 0, sizeof(unsigned), stream_));
    }
    launch_set_token(d_pos_, 0, stream_);  // position 0 (a kernel, not a memset)
    CLLM_HIP(hipStreamSynchronize(stream_));
    host_pos_ = 0;
    if (flag)
        throw DeviceError(
            "persistent decode kernel: the previous sequence had a wait that ran past its bound (its results were "
            "invalid); the engine is reset and usable");
}

void Engine::begin_step(const char* who, int token) {
    if (host_pos_ >= max_seq_)
        throw SequenceFull(std::string(who) + ": sequence full at max_seq_len positions; reset() starts a new one");
    if (token < -1 || token >= config().vocab)
        throw ArgError(std::string(who) + ": token must be -1 or a vocabulary index");
    if (token >= 0) launch_set_token(d_token_, token, stream_);
}

void Engine::read_outputs(float* logits_out, int* next_token_out) {
    if (logits_out) CLLM_HIP(hipMemcpy(logits_out, logits_, sizeof(float) * config().vocab, hipMemcpyDeviceToHost));
    if (next_token_out) CLLM_HIP(hipMemcpy(next_token_out, d_token_, sizeof(int), hipMemcpyDeviceToHost));
}

void Engine::step(int token, float* logits_out, int* next_token_out) {
    begin_step("step", token);
    // The persistent step is one kernel launched directly whether or not cuda_graph is set (replaying a one-node
    // graph of it only adds launch latency).  The multi-kernel program is captured on first use and replayed.
    if (persistent_) {
        launch_persistent(dp_);
    } else if (opts_.graph) {
        if (!graph_exec_) capture_graph(stream_, [this] { run_program(false); }, &graph_, &graph_exec_);
        CLLM_HIP(hipGraphLaunch(graph_exec_, stream_));
    } else {
        run_program(false);
    }
    host_pos_ += 1;
    if (!logits_out && !next_token_out) return;  // fully asynchronous
    CLLM_HIP(hipStreamSynchronize(stream_));
    raise_if_kernel_failed();
    read_outputs(logits_out, next_token_out);
}

void Engine::step_debug(int token, float* residuals_out, float* logits_out, int* next_token_out) {
    CLLM_REQUIRE(residuals_out, "step_debug: residuals_out is required");
    begin_step("step_debug", token);
    if (persistent_) {
        DecodeParams p = dp_;
        p.residuals = d_res_;
        launch_persistent(p);
    } else {
        run_program(true);
    }
    host_pos_ += 1;
    CLLM_HIP(hipStreamSynchronize(stream_));
    raise_if_kernel_failed();
    const ModelConfig& c = config();
    CLLM_HIP(hipMemcpy(residuals_out, d_res_, sizeof(float) * (c.n_layers + 1) * c.hidden, hipMemcpyDeviceToHost));
    read_outputs(logits_out, next_token_out);
}

int Engine::step_profile(int token, unsigned long long* stamps_out, long capacity) {
    if (!persistent_) throw StateError("step_profile: this engine's options do not select the persistent decode kernel");
    CLLM_REQUIRE(stamps_out && capacity >= static_cast<long>(grid_) * kStampSlots,
                 "step_profile: stamps_out must hold grid * 128 values");
    begin_step("step_profile", token);
    const size_t bytes = sizeof(unsigned long long) * grid_ * kStampSlots;
    CLLM_HIP(hipMemsetAsync(d_stamps_, 0, bytes, stream_));
    DecodeParams p = dp_;
    p.stamps = d_stamps_;
    launch_persistent(p);
    host_pos_ += 1;
    CLLM_HIP(hipStreamSynchronize(stream_));
    raise_if_kernel_failed();
    CLLM_HIP(hipMemcpy(stamps_out, d_stamps_, bytes, hipMemcpyDeviceToHost));
    return grid_;
}

void Engine::step_trace(int token, float* trace_out, long capacity, float* logits_out, int* next_token_out) {
    if (!persistent_) throw StateError("step_trace: this engine's options do not select the persistent decode kernel");
    const ModelConfig& c = config();
    const TraceLayout t = TraceLayout::of(c);
    CLLM_REQUIRE(trace_out && capacity >= static_cast<long>(t.total), "step_trace: trace_out is too small");
    begin_step("step_trace", token);
    DecodeParams p = dp_;
    p.residuals = d_res_;
    launch_persistent(p);
    host_pos_ += 1;
    CLLM_HIP(hipStreamSynchronize(stream_));
    raise_if_kernel_failed();
    CLLM_HIP(hipMemcpy(trace_out + t.residuals, d_res_, sizeof(float) * (c.n_layers + 1) * c.hidden,
                       hipMemcpyDeviceToHost));
    // Each tagged word holds its fp32 value in the low half.
    auto unpack = [&](const uint64_t* src, size_t n, float* dst) {
        std::vector<uint64_t> words(n);
        CLLM_HIP(hipMemcpy(words.data(), src, sizeof(uint64_t) * n, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < n; ++i) {
            const uint32_t bits = static_cast<uint32_t>(words[i]);
            std::memcpy(dst + i, &bits, sizeof(bits));
        }
    };
    unpack(dp_.tqkv, t.att - t.qkv, trace_out + t.qkv);
    unpack(dp_.tatt, t.xa - t.att, trace_out + t.att);
    unpack(dp_.txa, t.act - t.xa, trace_out + t.xa);
    unpack(dp_.tact, t.total - t.act, trace_out + t.act);
    read_outputs(logits_out, next_token_out);
}

}  // namespace cllm
