/*
 * cudallm C ABI — MI355X (gfx950) implementation.
 *
 * Every declaration below keeps the name, signature, struct layout and error code of the
 * reference interface it replaces (wasiqnauman/cudallm, include/cudallm/cudallm.h:8-56,
 * implemented there in src/capi/cudallm_capi.cpp:84-316), so a ctypes / C caller built for
 * the reference binds this libcudallm.so unchanged.  Entry points with no counterpart in the
 * reference are marked "no reference counterpart" and say who they are for.
 *
 * Conventions (reference src/capi/cudallm_capi.cpp:19-44):
 *  - every int-returning call returns one of the CUDALLM_* codes below, never throws;
 *  - on failure cudallm_last_error() returns a thread-local message;
 *  - all host buffers are owned by the caller; the engine handle is opaque;
 *  - an engine is single-threaded (one HIP stream), calls on one engine must not overlap.
 */
#ifndef CUDALLM_CUDALLM_H
#define CUDALLM_CUDALLM_H

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes: reference include/cudallm/cudallm.h:8-14.  Code 4 keeps its reference name;
 * here it reports a HIP runtime / device error. */
#define CUDALLM_OK 0
#define CUDALLM_ERR_INVALID_ARG 1
#define CUDALLM_ERR_IO 2
#define CUDALLM_ERR_FORMAT 3
#define CUDALLM_ERR_CUDA 4
#define CUDALLM_ERR_STATE 5
#define CUDALLM_ERR_INTERNAL 6

typedef struct cudallm_engine cudallm_engine;

/* Reference include/cudallm/cudallm.h:18-25 (6 x int). */
typedef struct {
    int matvec_impl;   /* 0 naive, 1 opt */
    int attn_impl;     /* 0 naive, 1 opt (split-K GQA) */
    int fuse;          /* 0/1: fused RMSNorm / residual / SwiGLU / RoPE+KV-write op order */
    int cuda_graph;    /* 0/1: capture the decode step once as a hipGraph and replay it */
    int max_seq_len;   /* 0 = from file, else a positive multiple of 128 <= the file's value */
    int matvec_rpb;    /* 0 = the library's per-shape choice; else 1, 2, 4 or 8 rows per wave per iteration (the
                          grid's workgroups per CU stay the library's per-shape choice either way) */
} cudallm_options;

/* Reference include/cudallm/cudallm.h:27-32 (10 x int, float, u64 at offset 48). */
typedef struct {
    int weight_dtype;  /* 1 bf16, 3 int8, 4 int4 */
    int hidden, inter, n_layers, n_heads, n_kv_heads, head_dim, vocab, max_seq_len, group_size;
    float rms_eps;
    unsigned long long weight_bytes;
} cudallm_config_info;

/* Reference cudallm.h:34 / cudallm_capi.cpp:86. */
const char* cudallm_last_error(void);
/* Reference cudallm.h:35 / cudallm_capi.cpp:88-96: opt, opt, 1, 1, 0, 0. */
void cudallm_default_options(cudallm_options* out);
/* Reference cudallm.h:36 / cudallm_capi.cpp:98-120.  *out = NULL on failure. */
int  cudallm_create(const char* path, const cudallm_options* opts, cudallm_engine** out);
/* Reference cudallm.h:37 / cudallm_capi.cpp:122-126.  NULL-safe. */
void cudallm_destroy(cudallm_engine* e);
/* Reference cudallm.h:38 / cudallm_capi.cpp:128-145. */
int  cudallm_get_config(cudallm_engine* e, cudallm_config_info* out);
/* Reference cudallm.h:39 / cudallm_capi.cpp:147-152: position back to 0. */
int  cudallm_reset(cudallm_engine* e);
/* Reference cudallm.h:40 / cudallm_capi.cpp:154-160: -1 for a NULL engine. */
int  cudallm_pos(cudallm_engine* e);
/* Reference cudallm.h:41 / cudallm_capi.cpp:162-168.  token -1 = previous device argmax;
 * logits_out (vocab floats) and next_token_out may be NULL; if both are NULL no sync. */
int  cudallm_step(cudallm_engine* e, int token, float* logits_out, int* next_token_out);
/* Reference cudallm.h:42 / cudallm_capi.cpp:170-177.  Never uses the graph; residuals_out
 * receives (n_layers+1)*hidden floats: after the embedding and after each layer. */
int  cudallm_step_debug(cudallm_engine* e, int token, float* residuals_out, float* logits_out, int* next_token_out);

/* One decode step (like cudallm_step with no outputs, but synchronous and never from the graph)
 * that also records when each workgroup of the persistent decode kernel finished each phase.
 * No reference counterpart: the reference profiled from outside with nsys.  stamps_out receives
 * grid x 128 values of the GPU's 100 MHz real-time clock, per workgroup: [0] start,
 * [1 + 6*layer + k] end of phase k (0 qkv, 1 attention, 2 split merge, 3 wo, 4 gate_up, 5 down),
 * [97] lm_head end, [98] argmax end (workgroup 0); for layer 1 only, [100 + 2k] when phase k's input had
 * arrived and [101 + 2k] when its prologue was done; capacity >= grid * 128.  CUDALLM_ERR_STATE if the
 * engine's options do not select the persistent kernel. */
int  cudallm_step_profile(cudallm_engine* e, int token, unsigned long long* stamps_out, long long capacity,
                          int* grid_out);

/* One decode step of the persistent kernel (synchronous, like cudallm_step_debug) that also returns
 * every vector its phases exchanged.  No reference counterpart: the reference's test hooks check each
 * kernel alone (tests/test_kernels.py); this lets a test check each phase of the fused kernel the same
 * way, from that phase's own inputs.  trace_out receives, in floats:
 *   [0, (L+1)*H)            the residual stream entering each layer, then after the last layer;
 *   then L * (nh+2*nkv)*hd  per layer q and k after RoPE, then v (the qkv phase's output);
 *   then L * nh*hd          per layer the attention output (after the split merge);
 *   then L * H              per layer the residual after attention (x + Wo att);
 *   then L * inter          per layer the SwiGLU output silu(gate) * up;
 * capacity >= that total.  logits_out / next_token_out as for cudallm_step.  CUDALLM_ERR_STATE if the
 * engine's options do not select the persistent kernel. */
int  cudallm_step_trace(cudallm_engine* e, int token, float* trace_out, long long capacity, float* logits_out,
                        int* next_token_out);

/* The HIP stream (a hipStream_t) on which the engine enqueues every step.  No reference
 * counterpart (the reference's stream is private to its Engine, src/engine/engine.cpp:40): it lets
 * a caller order its own device work after the engine's, or time steps with HIP events recorded
 * on this stream.  The stream belongs to the engine and dies with it. */
int  cudallm_get_stream(cudallm_engine* e, void** stream_out);

/* How this engine runs a step: *kind_out = 1 for the persistent decode kernel (one launch per token), 0 for the
 * multi-kernel program (the reference's ablation options, or a device where the persistent grid was not resident
 * at once); *grid_out = the persistent kernel's workgroups (0 for the program).  No reference counterpart (the
 * reference has one step path): benchmarks use it to refuse a run that did not time the kernel they name. */
int  cudallm_get_step_kind(cudallm_engine* e, int* kind_out, int* grid_out);

/* ---- single-kernel test hooks: host pointers in/out; allocate, copy, run, copy back, free ----
 * Reference cudallm.h:44-56 / cudallm_capi.cpp:179-316. */

/* weight_dtype 1 bf16 (u16 bits [rows][cols]), 3 int8 ([rows][cols] + fp32 scale per row),
 * 4 int4 (u8 [rows][cols/2], low nibble = even column, stored q+8; fp16 scale per 128 columns).
 * epilogue 0 STORE y=d, 1 ADD y+=d, 2 SWIGLU y[r]=silu(d_r)*d_{r+rows/2} (rows/2 outputs). */
int cudallm_kernel_matvec(int impl, int weight_dtype, int epilogue, int fuse_norm, int rpb,
                          const void* w, unsigned long long w_bytes, const void* scales, unsigned long long scales_bytes,
                          const float* x, const float* norm_w, float eps,
                          float* y /* in/out (ADD reads it) */, int rows, int cols);
int cudallm_kernel_rmsnorm(const float* x, const float* w, float eps, float* y, int n);
int cudallm_kernel_rope_kv(int fused, float* qkv /* in/out */, const float* inv_freq, int pos,
                           unsigned short* k_cache, unsigned short* v_cache /* in/out, fp16 bits, [nkv][max_seq][hd] */,
                           int nh, int nkv, int hd, int max_seq);
int cudallm_kernel_attention(int impl, const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                             int ctx, float* out, int nh, int nkv, int hd, int max_seq);
int cudallm_kernel_silu_mul(const float* gu, float* act, int inter);
int cudallm_kernel_argmax(const float* logits, int n, int* out_idx);

/* ---- device-pointer launches on a caller's HIP stream (no reference counterpart in C) ----
 * They expose the engine's kernels the way the reference's C++ tools reach them
 * (src/kernels/kernels.h:31,36 launch_matvec_opt / launch_attention_opt, used by
 * src/tools/cudallm_kernelbench.cpp), for kernel benchmarks and for integrators that own their
 * device memory.  All pointers are device pointers; `stream` is a hipStream_t (NULL = default
 * stream); the call only enqueues work.  Shapes are validated; buffer extents are the caller's
 * contract, exactly as for a kernel launch. */

/* Same operands and epilogues as cudallm_kernel_matvec (opt kernel); norm_w != NULL fuses RMSNorm. */
int cudallm_launch_matvec(int weight_dtype, int epilogue, int rpb, const void* w, const void* scales,
                          const float* x, const float* norm_w, float eps, float* y, int rows, int cols, void* stream);
/* cudallm_launch_attention without the scratch arguments, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No reference counterpart.  The
 * split partials live in a static device array of 8192 slots (about 2.1 MiB per GPU, held until the process ends),
 * so nh * max_seq / 128 must be at most 8192 (e.g. 32 heads up to max_seq 32768), else CUDALLM_ERR_INVALID_ARG.
 * The call allocates nothing.  Calls that overlap on one GPU share that array and race; serialise them (one stream,
 * or events). */
int cudallm_launch_attention_static(const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                                    const int* d_pos, float* out, int nh, int nkv, int hd, int max_seq, void* stream);
/* cudallm_launch_matvec whose kernel records start_event / stop_event (hipEvent_t, created by the caller) at its
 * own start and end (hipExtLaunchKernel), so hipEventElapsedTime gives the kernel's duration without the launch
 * gap: what a profiler's kernel trace reports.  For kernel benchmarks. */
int cudallm_launch_matvec_timed(int weight_dtype, int epilogue, int rpb, const void* w, const void* scales,
                                const float* x, const float* norm_w, float eps, float* y, int rows, int cols,
                                void* stream, void* start_event, void* stop_event);
/* Split-K GQA attention over ctx = *d_pos + 1 tokens; part_o holds nh*(max_seq/128)*hd floats and
 * part_ml nh*(max_seq/128)*2 floats of scratch. */
int cudallm_launch_attention(const float* q, const unsigned short* k_cache, const unsigned short* v_cache,
                             const int* d_pos, float* part_o, float* part_ml, float* out, int nh, int nkv, int hd,
                             int max_seq, void* stream);

/* Measured stream-read bandwidth of device memory (GB/s = 1e9 B/s): a `bytes` buffer (>= 64 MiB; use more than
 * the 256 MB Infinity Cache, e.g. 4 GiB) read `reps` times after warm-up for each of a few launch shapes; the best
 * and the median of the best shape.  No reference counterpart in C: the reference measures the same quantity with
 * its tool src/tools/cudallm_bandwidth.cpp:19-68 ("read_gbps_best", the peak its roofline fractions use). */
int cudallm_measure_read_bandwidth(unsigned long long bytes, int reps, double* best_gbps, double* median_gbps);
/* One read of `bytes` (>= 1 MiB, a multiple of 16) at device pointer `src` by the kernel above, with
 * blocks_per_cu (4, 8 or 16) x CUs workgroups; its dispatch records start_event / stop_event at the kernel's start
 * and end, as cudallm_launch_matvec_timed does.  `sink` is device memory of sink_words >= blocks_per_cu x CUs words
 * that the kernel writes only if the data XOR-folds to one fixed word.  For kernel benchmarks: the read time of a
 * matvec's own bytes, on the same copies, bounds what the matvec can reach.  No reference counterpart. */
int cudallm_launch_stream_read_timed(const void* src, unsigned long long bytes, int blocks_per_cu, unsigned* sink,
                                     unsigned long long sink_words, void* stream, void* start_event, void* stop_event);

/* ---- weight quantisers on the GPU (no reference counterpart in C) ----
 * They replace the reference's offline numpy quantisers, python/cudallm/quantize.py:5-38, with
 * bit-identical results; for exporters and synthetic-model writers.  Host pointers in/out. */

/* q[r][c] = clip(rint(w/s_r), -127, 127), s_r = max|w[r]|/127 (1 for a zero row). */
int cudallm_quantize_int8_rows(const float* w, int rows, int cols, signed char* q_out, float* scales_out);
/* s = fp16(max|group|/7) (1 for a zero group), q = clip(rint(w/fp32(s)), -8, 7), packed two per
 * byte as (q+8) with the even column in the low nibble.  group must be 128; cols % 128 == 0. */
int cudallm_quantize_int4_groups(const float* w, int rows, int cols, int group, unsigned char* packed_out,
                                 unsigned short* scales_out /* fp16 bits [rows][cols/group] */);
/* Inverse of the nibble packing: q_out[r][c] in [-8, 7] (python/cudallm/quantize.py:32-38). */
int cudallm_unpack_int4(const unsigned char* packed, int rows, int cols, signed char* q_out);

#ifdef __cplusplus
}
#endif

#endif /* CUDALLM_CUDALLM_H */
