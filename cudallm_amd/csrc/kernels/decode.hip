// Persistent batch-1 decode step for gfx950: one launch computes one token.
//
// What is computed is the fused op order of reference src/engine/engine.cpp:181-237 (embedding;
// per layer qkv with RMSNorm prologue, RoPE + fp16 KV write, split-K GQA attention with an LSE
// merge, wo + residual, gate_up with RMSNorm prologue and SwiGLU, down + residual; lm_head with
// the final RMSNorm; argmax that writes the token and advances the position).  How it is
// scheduled is this file's own:
//
//  * One workgroup of 8 waves per CU, every workgroup running every phase.  Waves 0-3 compute;
//    wave 4 + w is the loader of compute wave w.  Matvec rows are dealt to compute waves
//    round-robin, attention splits to workgroups.
//  * The rows a compute wave will multiply are fixed by its index alone, so its loader walks that
//    whole schedule (every phase of every layer, then lm_head) from the first instruction of the
//    step and streams the rows as 1 KiB lines (64 lanes x 16 B) into the compute wave's LDS ring,
//    running ahead across phase boundaries; it only ever waits for ring space.  HBM therefore
//    keeps streaming while compute waves wait for the inputs of their next phase.  The loader
//    keeps RingCfg::NB lines in flight with ordinary 128-bit loads and copies each landed line into the
//    ring; quantised lines carry one 32-bit side value per lane (row scale or group scale).
//  * Phases exchange vectors through tagged 64-bit words (see decode.h).  A consumer loads the
//    vector it needs with relaxed agent-scope atomics and re-loads only entries whose tag is not
//    yet the current phase's.  Compute waves issue no weight loads, so these polls are never
//    queued behind a weight stream.  No grid barriers, no RMW atomics and no cache flushes on the
//    data path: the dependency chain costs one store->load hop per phase.
//  * The four compute waves synchronise among themselves with an LDS epoch barrier (the loaders
//    run their own schedule and never join a workgroup barrier).
//  * Every wait is bounded.  On overrun the wave sets the sticky d_err flag and continues with
//    whatever it read; other waits notice the flag and stop waiting, so the grid always drains.
//    Indices never depend on activation values and the token is clamped, so no access can leave
//    its buffer even then.  The host reports the flag as a device error.
#include "../decode.h"
#include "../decode_walk.h"
#include "../kernels.h"
#include "device.h"
#include "digits.h"
#include "dot.h"

namespace cllm {
namespace dk {

using mv::Fmt;
using mv::chunk_dot;
using mv::kBias;
using mv::row_bytes;

constexpr int kCW = 4;                  // compute waves per workgroup (loaders are waves kCW..2kCW-1)
constexpr int kThreads = kDecodeThreads;
constexpr int kCT = kCW * kWave;        // compute threads
static_assert(kThreads == 2 * kCT, "one loader wave per compute wave");
constexpr int H = 2048, INTER = 8192, NH = 32, NKV = 8, HD = 64, QKV = (NH + 2 * NKV) * HD, VOCAB = 128256, NL = 16;
constexpr int kTagStride = 8;            // tag slots per layer
constexpr unsigned kEpochStride = 256;   // tag slots per step
constexpr unsigned kSpinCap = 1u << 20;     // bounded waits on other workgroups (~1 s of polling)
constexpr unsigned kLdsSpinCap = 1u << 26;  // bounded waits inside the workgroup (a few seconds)
constexpr int kPartStride = HD + 2;      // o[64], m, l
constexpr int kMergeOneWave = 16;        // split merges up to this many splits take one wave per head
constexpr int kPairs = QKV / 2;          // RoPE pairs (i, i+32) of every q/k/v head
// Tuning knobs of the decode kernel, overridable at build time (cudallm_amd/sweep_decode.py sweeps them): lines in
// flight per loader wave, ring slots per compute wave and lm_head rows per unit (each for bf16 / quantised).
#ifndef CLLM_LOADER_LINES
#define CLLM_LOADER_LINES 16
#endif
#ifndef CLLM_RING_SLOTS_BF16
// 30 bf16 slots fit, but 24 measured 4.6 us per step faster on MI355X (against 30: 26 -1.9, 22 +12.6; against 24:
// 25 +2.7, 23 +10.4; three alternating pairs each).
#define CLLM_RING_SLOTS_BF16 24
#endif
#ifndef CLLM_RING_SLOTS_QUANT
#define CLLM_RING_SLOTS_QUANT 22
#endif
#ifndef CLLM_LM_ROWS_BF16
#define CLLM_LM_ROWS_BF16 2
#endif
#ifndef CLLM_LM_ROWS_QUANT
#define CLLM_LM_ROWS_QUANT 8
#endif
// Per-type overrides of the quantised knobs.  int4 keeps 20 ring slots (-1.1 us per step against 22, three
// alternating pairs on MI355X); 4-row int8 lm_head units measured +0.4 us, so int8 keeps the shared value.
#ifndef CLLM_RING_SLOTS_INT4
#define CLLM_RING_SLOTS_INT4 20
#endif
#ifndef CLLM_LM_ROWS_INT8
#define CLLM_LM_ROWS_INT8 CLLM_LM_ROWS_QUANT
#endif
template <WType WT>
constexpr int kLmR = WT == WType::BF16 ? CLLM_LM_ROWS_BF16 : WT == WType::INT8 ? CLLM_LM_ROWS_INT8 : CLLM_LM_ROWS_QUANT;  // lm_head rows per unit
static_assert(walk::kH == H && walk::kInter == INTER && walk::kVocab == VOCAB && walk::kPairs == kPairs,
              "the weight walk and the kernel agree on the shapes");
static_assert(VOCAB % kLmR<WType::BF16> == 0 && VOCAB % kLmR<WType::INT8> == 0 && VOCAB % kLmR<WType::INT4> == 0,
              "lm_head units");

enum : unsigned { T_QKV = 0, T_ATT_PART = 1, T_ATT = 2, T_XA = 3, T_ACT = 4, T_X = 5 };
constexpr unsigned T_ARG = NL * kTagStride;

// Attention tiles in Smem::big (floats): K as fp16 pairs [128][kKs] (16-byte aligned rows whose
// 128-bit reads by 16 consecutive lanes hit distinct banks), V [128][8] x 16 B, scores [4][128], q [4][64].
constexpr int kKs = 36;
constexpr int kAttnV = kAttnChunk * kKs, kAttnP = kAttnV + kAttnChunk * HD / 2, kAttnQ = kAttnP + 4 * kAttnChunk;
// The digit table of the integer dot products sits after the down-projection input: a wave can be
// fetching that input (next phase) while another still reads the table.
constexpr int kDigOff = INTER, kDigWordsMax = 3 * 512;
constexpr int kBig = kAttnQ + 4 * HD > kDigOff + kDigWordsMax ? kAttnQ + 4 * HD : kDigOff + kDigWordsMax;
static_assert(kBig >= INTER, "big holds the down-projection input");
// Phase inputs live in big too, which leaves the LDS to the rings.  bf16 (whose swizzled down input spans
// all 8192 floats) puts every input at big + 0, each overwrite behind a barrier or a carrive/cwait pair.
// The quantised weights have room to spare: the layer input (qkv; lm_head's final-norm input) gets a
// region of its own past the digit table and gate_up's input sits at big + H beside wo's, so none of
// those fetches waits for another wave.
template <WType WT>
constexpr int kXin = WT == WType::BF16 ? 0 : kBig;
template <WType WT>
constexpr int kXgu = WT == WType::BF16 ? 0 : H;
template <WType WT>
constexpr int kBigOf = WT == WType::BF16 ? kBig : kBig + H;
// Rows of wo and down per compute wave (r = gw, gw + NW, ...) at the smallest grid the kernel takes: the
// residual inputs at those rows are all a wave keeps of the layer input and of the residual after attention.
constexpr int kRPW = 8;
static_assert(kDecodeMinGrid * kCW * kRPW >= H, "residual rows per wave");

// Ring geometry per weight type.
template <WType WT>
struct RingCfg {
    static constexpr bool kQuant = WT != WType::BF16;
    static constexpr int S = WT == WType::INT4 ? CLLM_RING_SLOTS_INT4 : kQuant ? CLLM_RING_SLOTS_QUANT : CLLM_RING_SLOTS_BF16;  // 1 KiB slots per compute wave
    static constexpr int SS = kQuant ? S : 1;                  // side-value slots
    static constexpr int LPR2 = Fmt<WT>::CPL;                  // lines per 2048-wide row
    static constexpr int LPR8 = INTER / Fmt<WT>::CPC / kWave;  // lines per 8192-wide row
    // Lines in flight per loader wave (16 measured best on MI355X: deeper queues also delay the small polling loads of
    // the phase handoffs behind them).
    static constexpr int NB = CLLM_LOADER_LINES;
};

// A compute wave waits for every line of a unit (two 2048-wide rows; an lm_head unit of kLmR rows) before it
// releases any, so a unit must fit its ring: otherwise the loader can never publish the unit's last lines and the
// wait for them runs out (an error, not a result).
template <WType WT>
constexpr bool kUnitsFitRing = 2 * RingCfg<WT>::LPR2 <= RingCfg<WT>::S && kLmR<WT> * RingCfg<WT>::LPR2 <= RingCfg<WT>::S;
static_assert(kUnitsFitRing<WType::BF16> && kUnitsFitRing<WType::INT8> && kUnitsFitRing<WType::INT4>,
              "a unit's lines fit the ring");

template <WType WT>
struct Smem {
    u32x4 ring[kCW][RingCfg<WT>::S][kWave];
    float side[kCW][RingCfg<WT>::SS][kWave];
    float big[kBigOf<WT>];  // phase inputs | attention tiles | SwiGLU output | digit tables
    float xres[kCW * kRPW];  // layer input at the wave's wo rows
    float ares[kCW * kRPW];  // residual after attention at the wave's down rows (the same rows)
    float rope_c[HD / 2], rope_s[HD / 2];
    float part[kCW];
    float pmax[kCW];  // per-wave max |x g| of the last fetch with MXG
    float red_v[kCW];
    int red_i[kCW];
    unsigned bar[kCW];
    int full[kCW];  // lines the loader has published, per compute wave
    int done[kCW];  // lines the compute wave has released
};

// ---- cross-workgroup tagged words ------------------------------------------------------------

// Every device pointer in DecodeParams is global memory; saying so keeps the accesses off the
// flat path (which would also count against the LDS counter).
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* glob(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}

// The layer's weight pointers (field by field: a struct copy cannot read another address space).
__device__ __forceinline__ DecodeLayer load_layer(const DecodeLayer* t, int l) {
    const __attribute__((address_space(1))) DecodeLayer* g = glob(t + l);
    DecodeLayer L;
    L.attn_norm = g->attn_norm;
    L.wqkv = g->wqkv;
    L.sqkv = g->sqkv;
    L.wo = g->wo;
    L.so = g->so;
    L.ffn_norm = g->ffn_norm;
    L.wgu = g->wgu;
    L.sgu = g->sgu;
    L.wd = g->wd;
    L.sd = g->sd;
    return L;
}

__device__ __forceinline__ uint64_t tload(const uint64_t* a) {
    return __hip_atomic_load(glob(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(uint64_t* a, float v, unsigned tag) {
    __hip_atomic_store(glob(a), (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tagged(uint64_t v, unsigned tag) { return static_cast<unsigned>(v >> 32) == tag; }
__device__ __forceinline__ float tvalue(uint64_t v) { return __builtin_bit_cast(float, static_cast<uint32_t>(v)); }
__device__ __forceinline__ bool failed(unsigned* err) {
    return __hip_atomic_load(glob(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void fail(unsigned* err) {
    __hip_atomic_fetch_or(glob(err), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// True when a wait must stop: it ran out of polls, or another wave already failed.  Polls are not
// spaced by s_sleep: each already takes a memory round trip, and without the sleep int4 measured
// 3.8 us per step faster on MI355X (bf16 and int8 within 1.5 us).
__device__ __forceinline__ bool give_up(unsigned& spins, unsigned* err) {
    if (++spins >= kSpinCap || ((spins & 255u) == 0 && failed(err))) {
        fail(err);
        return true;
    }
    return false;
}

// Wait for two tagged values (per lane) with both loads in flight: one round trip, not two.
__device__ __forceinline__ void wait2(const uint64_t* a, const uint64_t* b, unsigned tag, unsigned* err, float& va,
                                      float& vb) {
    uint64_t x = tload(a), y = tload(b);
    unsigned spins = 0;
    while (!(tagged(x, tag) && tagged(y, tag)) && !give_up(spins, err)) {
        if (!tagged(x, tag)) x = tload(a);
        if (!tagged(y, tag)) y = tload(b);
    }
    va = tvalue(x);
    vb = tvalue(y);
}

// Test hook: sleep about 13 us when the stall mask selects `bit` (and this workgroup, with kStallOdd).
// The mask is a kernel argument, so the test is a scalar branch that normal runs never take.
__device__ __forceinline__ void stall_at(const DecodeParams& p, unsigned bit) {
    if ((p.stall & bit) && (!(p.stall & kStallOdd) || (blockIdx.x & 1)) &&
        (!(p.stall & kStallWave0) || threadIdx.x < kWave)) {
#pragma unroll 1
        for (int i = 0; i < 4; ++i) __builtin_amdgcn_s_sleep(127);
    }
}

// ---- workgroup-local synchronisation (LDS) ---------------------------------------------------

// The flags below only order LDS accesses, and the LDS executes a wave's accesses in issue order,
// so a relaxed access behind a compiler barrier is enough.  A release/acquire atomic would also wait
// for the wave's outstanding global stores (one counter covers loads and stores on this GPU): a full
// memory round trip per ring slot or barrier.
__device__ __forceinline__ int lds_load(int* a) {
    const int v = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    asm volatile("" ::: "memory");  // later LDS reads stay after this one
    return v;
}
__device__ __forceinline__ void lds_store(int* a, int v) {
    asm volatile("" ::: "memory");  // earlier LDS accesses stay before this one
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// One step of a bounded wait on a partner in this workgroup.  No global access on this path (it
// would make every wait end with a full drain of the wave's memory counter); an overrun is kept
// in `lbad` and reported once, when the wave finishes.  No s_sleep between polls: an LDS poll
// costs the SIMD little, and without the sleep int8 measured 7 us per step faster on MI355X.
__device__ __forceinline__ bool lds_give_up(unsigned& spins, bool& lbad) {
    if (++spins >= kLdsSpinCap) {
        lbad = true;
        return true;
    }
    return false;
}

// Barrier of the kCW compute waves: each publishes its epoch, then waits for all.  Orders the
// LDS writes made before it against the reads made after it.
__device__ __forceinline__ void cbar(unsigned* bar, unsigned& ep, int wave, int lane, bool& lbad) {
    ++ep;
    asm volatile("" ::: "memory");
    if (lane == 0) __hip_atomic_store(bar + wave, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    unsigned spins = 0;
    for (;;) {
        unsigned lo = ~0u;
#pragma unroll
        for (int w = 0; w < kCW; ++w) lo = min(lo, __hip_atomic_load(bar + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (lo >= ep || lds_give_up(spins, lbad)) break;
    }
    asm volatile("" ::: "memory");
}

// cbar in two halves: carrive() publishes the wave's next epoch (it has finished reading what the
// barrier protects) and returns it; cwait(e) waits until every compute wave has published e.  Waves
// announce early and wait only where they are about to overwrite.
__device__ __forceinline__ unsigned carrive(unsigned* bar, unsigned& ep, int wave, int lane) {
    ++ep;
    asm volatile("" ::: "memory");
    if (lane == 0) __hip_atomic_store(bar + wave, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return ep;
}
__device__ __forceinline__ void cwait(unsigned* bar, unsigned e, bool& lbad) {
    unsigned spins = 0;
    for (;;) {
        unsigned lo = ~0u;
#pragma unroll
        for (int w = 0; w < kCW; ++w) lo = min(lo, __hip_atomic_load(bar + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (lo >= e || lds_give_up(spins, lbad)) break;
    }
    asm volatile("" ::: "memory");
}

// Wait until the loader has published `need` lines of this wave's ring.
__device__ __forceinline__ void ring_wait(int need, int& cfull, int* full, bool& lbad) {
    if (cfull >= need) return;
    unsigned spins = 0;
    for (;;) {
        cfull = lds_load(full);
        if (cfull >= need || lds_give_up(spins, lbad)) break;
    }
}

// ---- the loader ------------------------------------------------------------------------------

// Walks a compute wave's weight rows in the order the compute code multiplies them: per layer the
// segments qkv (RoPE pairs: rows r and r+32), wo, gate_up (gate row u, up row u+inter), down
// (8192-wide rows); then lm_head (kLmR consecutive rows per unit).  Unit u of a segment belongs to
// compute wave gw when u = gw (mod NW).  With NW a multiple of 32 the rows of consecutive units
// of a wave are a fixed stride apart in every segment, so a line advance is pointer arithmetic.
// All state is wave-uniform.
template <WType WT>
struct Stream {
    const DecodeParams* p;
    int gw, NW;
    int l = 0, seg = 0;
    bool end = false;
    walk::Walker<const char*> w;  // the segment's lines (decode_walk.h)

    __device__ void set_seg() {
        const char* mat;
        const char* sc;
        if (seg == 4) {
            mat = static_cast<const char*>(p->emb);
            sc = static_cast<const char*>(p->emb_s);
        } else {
            const DecodeLayer L = load_layer(p->layers, l);
            mat = static_cast<const char*>(seg == 0 ? L.wqkv : seg == 1 ? L.wo : seg == 2 ? L.wgu : L.wd);
            sc = static_cast<const char*>(seg == 0 ? L.sqkv : seg == 1 ? L.so : seg == 2 ? L.sgu : L.sd);
        }
        w.start(walk::seg_of(WT, seg, gw, NW, kLmR<WT>), mat, sc);
    }
    // Next segment (each wave has units in every segment when NW <= kPairs).
    __device__ void next_seg() {
        if (seg == 4) {
            end = true;
            return;
        }
        if (seg == 3) {
            if (l + 1 < NL) {
                ++l;
                seg = 0;
            } else {
                seg = 4;
            }
        } else {
            ++seg;
        }
        set_seg();
    }
    __device__ void init(const DecodeParams* pp, int gw_, int nw) {
        p = pp, gw = gw_, NW = nw, l = 0, seg = 0, end = false;
        set_seg();
    }
};

template <WType WT>
__device__ __forceinline__ float side_value(uint32_t raw) {
    if constexpr (WT == WType::INT4) return half_bits_to_float(static_cast<uint16_t>(raw));
    return __builtin_bit_cast(float, raw);
}

// Loader wave for compute wave `wave`: RingCfg::NB lines in flight.  Every slot always holds a load (a
// repeat of the last line where the stream has none, at a segment switch or past the end), so the
// in-order completion count the compiler waits on is exact; each landed line is copied into the
// ring and published through full[wave].  The segment switch runs once per round of NB slots.
// loader() and fetch() are force-inlined: with the inliner's own choice (which also inlined them) the
// step measured 19-24 us slower on MI355X for every weight type.
template <WType WT>
__device__ __forceinline__ void loader(const DecodeParams& p, Smem<WT>& sm, int wave, int lane) {
    using C = RingCfg<WT>;
    unsigned* err = p.d_err;
    const int gw = blockIdx.x * kCW + wave, NW = gridDim.x * kCW;
    Stream<WT> st;
    st.init(&p, gw, NW);
    const int loff = lane * 16;
    const int soff = WT == WType::INT4 ? (lane / 4) * 2 : 0;
    u32x4 buf[C::NB];
    uint32_t sd[C::NB];
    bool v[C::NB];
    const char* last = st.w.cur;
    const char* slast = st.w.scur;
    auto issue = [&](int s) {
        v[s] = st.w.have;
        if (st.w.have) {
            last = st.w.cur;
            slast = st.w.scur;
        }
        buf[s] = load_stream(last + loff);
        if constexpr (WT == WType::INT8) sd[s] = gload(reinterpret_cast<const uint32_t*>(slast));
        if constexpr (WT == WType::INT4) sd[s] = gload(reinterpret_cast<const uint16_t*>(slast + soff));
        if (st.w.have) st.w.advance();
    };
#pragma unroll
    for (int s = 0; s < C::NB; ++s) issue(s);
    int k = 0, cdone = 0, slot = 0;  // slot = k mod S, kept as a counter
    bool lbad = false;
    for (;;) {
        bool any = false;
#pragma unroll
        for (int s = 0; s < C::NB; ++s) {
            if (v[s]) {
                any = true;
                if (k - cdone >= C::S) {
                    unsigned spins = 0;
                    for (;;) {
                        cdone = lds_load(&sm.done[wave]);
                        if (k - cdone < C::S || lds_give_up(spins, lbad)) break;
                    }
                }
                sm.ring[wave][slot][lane] = buf[s];
                if constexpr (C::kQuant) sm.side[wave][slot][lane] = side_value<WT>(sd[s]);
                ++k;
                slot = slot + 1 == C::S ? 0 : slot + 1;
                if (lane == 0) lds_store(&sm.full[wave], k);
            }
            issue(s);
            // bf16 also switches segment half-way through a round, so the next segment's first lines go out up to
            // 8 slots sooner: -2 to -4 us per bf16 step.  The quantised kernels keep one switch per round: the earlier
            // switch streams more during the handoffs and slows their polls (int8 +1.5, int4 +7 us).
            if constexpr (WT == WType::BF16) {
                if (s == C::NB / 2 - 1 && !st.w.have && !st.end) {
                    stall_at(p, kStallLoader);
                    st.next_seg();
                }
            }
        }
        if (!st.w.have && !st.end) {
            stall_at(p, kStallLoader);
            st.next_seg();
        }
        if (!any && st.end) break;
    }
    if (lbad) fail(err);
}

// ---- compute-wave helpers --------------------------------------------------------------------

// LDS position of element i of an 8192-wide input stored for the down projection: lane l of
// 16-byte chunk c needs elements (64 c + l) CPC .. + CPC - 1, kept as [chunk][quad][lane] float4s
// so the 64 lanes' 128-bit reads of one quad are consecutive (no bank conflicts).
template <int CPC>
__device__ __forceinline__ int swz(int i) {
    const int c = i / (kWave * CPC), l = (i / CPC) % kWave, q = (i % CPC) / 4, e = i % 4;
    return ((c * (CPC / 4) + q) * kWave + l) * 4 + e;
}

// The whole compute group copies N tagged floats into LDS once every tag equals `tag` (at swz<SWZ>
// positions when SWZ > 0); with SQ, each wave also leaves the sum of squares of the values it
// copied in part[wave].  Callers follow with cbar().
//
// With MX = 1, each wave also leaves max |x_i g_i| over the entries it copied in pmax[wave] (g: the
// norm weights, read while the wait runs), from which the fixed-point scale of the integer dot
// products is derived; with MX = 2, max |x_i|.
//
// With TWO, each thread first polls only its last entry and loads the others once that one is current: a wait
// that starts long before the producers finish then keeps 1/PT of the polls in flight, which leaves the memory
// path to the producers' stores.  Measured on MI355X for the wo input, which every workgroup starts polling while
// the few attention workgroups still compute: int4 -16, int8 -4 us per step, and bf16 -4.6 us once attention wrote
// whole lines (+3 before); for int8's gate_up input a further -9 us, and for int8's qkv input -2 us.  Polling one
// stage again (after the whole-line attention stores): int8 +6, int4 +16 us.
template <int N, bool SQ, int SWZ = 0, int MX = 0, bool TWO = false>
__device__ __forceinline__ void fetch(const uint64_t* src, unsigned tag, float* dst, float* part, unsigned* err, int tid,
                      const float* g = nullptr, float* pmax = nullptr) {
    constexpr int PT = N / kCT;
    constexpr bool MXG = MX == 1;
    static_assert(N % kCT == 0, "fetch size");
    unsigned spins = 0;
    float gv[MXG ? PT : 1];
    if constexpr (MXG)
#pragma unroll
        for (int k = 0; k < PT; ++k) gv[k] = gload(g + tid + k * kCT);
    if constexpr (TWO) {
        uint64_t f = tload(src + tid + (PT - 1) * kCT);
        while (!tagged(f, tag) && !give_up(spins, err)) f = tload(src + tid + (PT - 1) * kCT);
    }
    uint64_t v[PT];
#pragma unroll
    for (int k = 0; k < PT; ++k) v[k] = tload(src + tid + k * kCT);
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < PT; ++k) ok = ok && tagged(v[k], tag);
        if (ok || give_up(spins, err)) break;
#pragma unroll
        for (int k = 0; k < PT; ++k)
            if (!tagged(v[k], tag)) v[k] = tload(src + tid + k * kCT);
    }
    float ss = 0.f, mx = 0.f;
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const float x = tvalue(v[k]);
        const int i = tid + k * kCT;
        if constexpr (SWZ > 0) {
            dst[swz<SWZ>(i)] = x;
        } else {
            dst[i] = x;
        }
        ss += x * x;
        if constexpr (MX == 1) mx = fmaxf(mx, fabsf(x * gv[k]));
        if constexpr (MX == 2) mx = fmaxf(mx, fabsf(x));
    }
    if constexpr (SQ) {
        ss = wave_sum(ss);
        if ((tid & (kWave - 1)) == 0) part[tid / kWave] = ss;
    }
    if constexpr (MX != 0) {
        mx = wave_max(mx);
        if ((tid & (kWave - 1)) == 0) pmax[tid / kWave] = mx;
    }
}

// 1 / rms from the per-wave partial sums of squares (same partition and order in every workgroup).
__device__ __forceinline__ float rms_inv(const float* part, float eps) {
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < kCW; ++w) ss += part[w];
    return rsqrtf(ss / static_cast<float>(H) + eps);
}

typedef const __attribute__((address_space(1))) f32x4 global_f32x4;

// ---- integer dot products for the quantised weights (gate_up and lm_head) ----------------------
//
// The normalised input x^ = (x inv) g is written as a 22-bit fixed-point integer with one power-of-two
// scale per phase, xi = rint(x^ 2^e) (|xi| <= 2^22), and split into signed digits: three base-256
// digits (bytes) for int8 weights, six base-16 digits (nibbles) for int4 weights, packed in the
// weights' own layout so that v_dot4_i32_i8 / v_dot8_i32_i4 multiply raw weight words.  The integer
// partial sums are exact; the only new rounding is that of xi (at most 2^-23 of max |x^|), against
// fp32's 2^-24 of each |x^|.  Adding the offset C = (base/2) * (1 + base + base^2 ...) makes every digit
// of xi + C non-negative, and xor C then turns each of them into its signed two's-complement form.
template <WType WT>
struct Dig {
    static constexpr int ND = WT == WType::INT8 ? 3 : 6;      // digits
    static constexpr int WPD = 2048 / (WT == WType::INT8 ? 4 : 8);  // digit words per digit (2048 columns)
    static constexpr uint32_t C = WT == WType::INT8 ? 0x808080u : 0x888888u;
    uint32_t d[24];  // the lane's words: int8 [digit][chunk][word], int4 [digit][word]
};
static_assert(Dig<WType::INT8>::ND * Dig<WType::INT8>::WPD == Dig<WType::INT4>::ND * Dig<WType::INT4>::WPD,
              "digit tables share one size");
static_assert(Dig<WType::INT8>::ND * Dig<WType::INT8>::WPD == kDigWordsMax, "digit table size");

// The norm weights of columns 8 tid .. 8 tid + 7, loaded before the phase waits for its input so that the
// digit prologue after the wait does not start a memory round trip of its own.
struct Norm8 {
    f32x4 g0, g1;
};
__device__ __forceinline__ Norm8 load_norm8(const float* g, int tid) {
    return {*((global_f32x4*)g + 2 * tid), *((global_f32x4*)g + 2 * tid + 1)};
}

// Thread tid writes the digit words of columns 8 tid .. 8 tid + 7 (all 2048 by the compute group).
template <WType WT>
__device__ void make_digits(const float* x, const Norm8& gn, float inv, int e, uint32_t* tab, int tid) {
    using D = Dig<WT>;
    const f32x4 x0 = reinterpret_cast<const f32x4*>(x)[2 * tid], x1 = reinterpret_cast<const f32x4*>(x)[2 * tid + 1];
    const f32x4 g0 = gn.g0, g1 = gn.g1;
    const float scale = ldexpf(1.f, e);
    uint32_t u[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float xc = c < 4 ? x0[c] : x1[c - 4];
        const float gc = c < 4 ? g0[c] : g1[c - 4];
        u[c] = fixed_word(xc * inv * gc, scale, D::C);
    }
    if constexpr (WT == WType::INT8) {
        uint32_t P[2][3];
        byte_planes(u[0], u[1], u[2], u[3], P[0]);
        byte_planes(u[4], u[5], u[6], u[7], P[1]);
#pragma unroll
        for (int k = 0; k < 3; ++k)
#pragma unroll
            for (int h = 0; h < 2; ++h) tab[k * D::WPD + 2 * tid + h] = P[h][k] ^ 0x80808080u;
    } else {
        uint32_t w[6];
        nibble_words(u, w);
#pragma unroll
        for (int k = 0; k < 6; ++k) tab[k * D::WPD + tid] = w[k] ^ 0x88888888u;
    }
}

// The lane's digit words (same column mapping as its weight chunks).
template <WType WT>
__device__ __forceinline__ void load_digits(const uint32_t* tab, int lane, Dig<WT>& dg) {
    using D = Dig<WT>;
    if constexpr (WT == WType::INT8) {
#pragma unroll
        for (int k = 0; k < 3; ++k)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(tab + k * D::WPD + (c * kWave + lane) * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) dg.d[(k * 2 + c) * 4 + i] = v[i];
            }
    } else {
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(tab + k * D::WPD + lane * 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) dg.d[k * 4 + i] = v[i];
        }
    }
}

// After the fetch of a normalised phase input (and its barrier): the scale exponent from the waves'
// max |x g| and inv, and this thread's digit words into the table.  Returns 2^-e.  Callers follow
// with a barrier, then load_digits().
template <WType WT, typename SM>
__device__ __forceinline__ float digits_prologue(SM& sm, float inv, const Norm8& gn, int tid, const float* x = nullptr) {
    float m = 0.f;
#pragma unroll
    for (int w = 0; w < kCW; ++w) m = fmaxf(m, sm.pmax[w]);
    const int e = dig_exponent(m * inv);
    make_digits<WT>(x ? x : sm.big, gn, inv, e, reinterpret_cast<uint32_t*>(sm.big + kDigOff), tid);
    return ldexpf(1.f, -e);
}

// Norm weights of the lane's 32 columns of a 2048-wide row (same column mapping as the matvec).
template <WType WT>
struct NormW {
    f32x4 v[Fmt<WT>::CPL * Fmt<WT>::CPC / 4];
};
template <WType WT>
__device__ __forceinline__ void load_norm(const float* w, int lane, NormW<WT>& n) {
    using F = Fmt<WT>;
#pragma unroll
    for (int k = 0; k < F::CPL; ++k)
#pragma unroll
        for (int j = 0; j < F::CPC; j += 4) n.v[(k * F::CPC + j) / 4] = *((global_f32x4*)(w + (k * kWave + lane) * F::CPC + j));
}

// The lane's 32 inputs of a 2048-wide row, scaled by inv * norm_w when a norm is given.
template <WType WT, bool NORM>
__device__ __forceinline__ void lane_inputs(const float* x, const NormW<WT>* nw, float inv, float* xr, float& xsum,
                                            int lane) {
    using F = Fmt<WT>;
    xsum = 0.f;
#pragma unroll
    for (int k = 0; k < F::CPL; ++k) {
        const int c0 = (k * kWave + lane) * F::CPC;
#pragma unroll
        for (int j = 0; j < F::CPC; j += 4) {
            const f32x4 xv = *reinterpret_cast<const f32x4*>(x + c0 + j);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = xv[e];
                if constexpr (NORM) v = v * inv * nw->v[(k * F::CPC + j) / 4][e];
                xr[k * F::CPC + j + e] = v;
                xsum += v;
            }
        }
    }
}

// One 2048-wide row as this lane holds it: its 16-byte chunks and its side value.
template <WType WT>
struct Row {
    u32x4 w[Fmt<WT>::CPL];
    float s;
};

// Compute wave's view of its ring.  bf16 keeps the slot of line k (k mod S) as a counter and reads the lines of a
// row that does not wrap round the ring's end at fixed offsets from one address: the division was about 7 scalar
// instructions per line, and a wave issues one instruction of any kind per 4 cycles (bf16 -12 us per step on
// MI355X).  The quantised kernels keep the division: with the counter and the no-wrap branch int8 measured +7 and
// int4 +11 us, and with the counter alone int4 +4 us.
struct Cons {
    int k = 0;      // lines consumed
    int slot = 0;   // k mod S (bf16)
    int cfull = 0;  // published lines last seen
};

// Ring slot of line k + off (off < S).
template <WType WT>
__device__ __forceinline__ int ring_slot(const Cons& cs, int off) {
    if constexpr (WT != WType::BF16) return (cs.k + off) % RingCfg<WT>::S;
    const int s = cs.slot + off;
    return s >= RingCfg<WT>::S ? s - RingCfg<WT>::S : s;
}

// Lines k + off .. k + off + N - 1 of the wave's ring into w (with SIDE, their side values into sd).
template <WType WT, int N, bool SIDE = false>
__device__ __forceinline__ void ring_read(Smem<WT>& sm, const Cons& cs, int off, int wave, int lane, u32x4* w,
                                          float* sd = nullptr) {
    using C = RingCfg<WT>;
    static_assert(N <= C::S && (!SIDE || C::kQuant), "ring read");
    const int s0 = ring_slot<WT>(cs, off);
    if (WT == WType::BF16 && s0 <= C::S - N) {
        const u32x4* b = &sm.ring[wave][s0][lane];
#pragma unroll
        for (int c = 0; c < N; ++c) w[c] = b[c * kWave];
        if constexpr (SIDE) {
            const float* bs = &sm.side[wave][s0][lane];
#pragma unroll
            for (int c = 0; c < N; ++c) sd[c] = bs[c * kWave];
        }
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) {
            const int sl = s0 + c < C::S ? s0 + c : s0 + c - C::S;
            w[c] = sm.ring[wave][sl][lane];
            if constexpr (SIDE) sd[c] = sm.side[wave][sl][lane];
        }
    }
}
template <WType WT>
__device__ __forceinline__ float ring_side(Smem<WT>& sm, const Cons& cs, int off, int wave, int lane) {
    return sm.side[wave][ring_slot<WT>(cs, off)][lane];
}
template <WType WT>
__device__ __forceinline__ void ring_advance(Cons& cs, int n) {
    if constexpr (WT == WType::BF16) cs.slot = ring_slot<WT>(cs, n);
    cs.k += n;
}

template <WType WT>
__device__ __forceinline__ void take_row(Smem<WT>& sm, Cons& cs, int wave, int lane, bool& lbad, Row<WT>& r) {
    using C = RingCfg<WT>;
    ring_wait(cs.k + C::LPR2, cs.cfull, &sm.full[wave], lbad);
    ring_read<WT, C::LPR2>(sm, cs, 0, wave, lane, r.w);
    if constexpr (C::kQuant) r.s = ring_side<WT>(sm, cs, 0, wave, lane);
    ring_advance<WT>(cs, C::LPR2);
}
template <WType WT>
__device__ __forceinline__ void release(Smem<WT>& sm, const Cons& cs, int wave, int lane) {
    if (lane == 0) lds_store(&sm.done[wave], cs.k);
}
// Where the row loops release a unit's lines.  bf16 and int8 release them as soon as the rows are read into
// registers, so the loader refills the slots during the dot products (bf16 -5, int8 -2 us per step on MI355X);
// int4 releases them after the dot products (released early, +4 us).  Both are safe: the reads are issued before
// the release, LDS executes a wave's accesses in order, and the loader writes a slot only after it has seen the
// release.
template <WType WT>
__device__ __forceinline__ void release_early(Smem<WT>& sm, const Cons& cs, int wave, int lane) {
    if constexpr (WT != WType::INT4) release(sm, cs, wave, lane);
}
template <WType WT>
__device__ __forceinline__ void release_late(Smem<WT>& sm, const Cons& cs, int wave, int lane) {
    if constexpr (WT == WType::INT4) release(sm, cs, wave, lane);
}

// Complete dot of a 2048-wide row, uniform across the wave.
template <WType WT>
__device__ __forceinline__ float row_dot(const Row<WT>& r, const float* xr, float xsum) {
    using F = Fmt<WT>;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < F::CPL; ++k) s += chunk_dot<WT>(r.w[k], xr + k * F::CPC);
    if constexpr (WT == WType::INT8) s -= kBias<WT> * xsum;
    if constexpr (WT == WType::INT4) s = r.s * (s - kBias<WT> * xsum);
    s = wave_sum(s);
    if constexpr (WT == WType::INT8) s *= r.s;
    return s;
}

// A lane's share of the dot of a 2048-wide quantised row with the input digits, before any scale: int8:
// sum_k 256^k sum(q d_k); int4: sum_k 16^k sum(q d_k) (the stored nibble u = q + 8 becomes q by xor 8).
template <WType WT>
__device__ __forceinline__ float dig_part(const Row<WT>& r, const Dig<WT>& dg) {
    if constexpr (WT == WType::INT8) {
        int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int w = static_cast<int>(r.w[c][i]);
                a0 = __builtin_amdgcn_sdot4(w, static_cast<int>(dg.d[(0 * 2 + c) * 4 + i]), a0, false);
                a1 = __builtin_amdgcn_sdot4(w, static_cast<int>(dg.d[(1 * 2 + c) * 4 + i]), a1, false);
                a2 = __builtin_amdgcn_sdot4(w, static_cast<int>(dg.d[(2 * 2 + c) * 4 + i]), a2, false);
            }
        return fmaf(fmaf(static_cast<float>(a2), 256.f, static_cast<float>(a1)), 256.f, static_cast<float>(a0));
    } else {
        int a[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int w = static_cast<int>(r.w[0][i] ^ 0x88888888u);
#pragma unroll
            for (int k = 0; k < 6; ++k) a[k] = __builtin_amdgcn_sdot8(w, static_cast<int>(dg.d[k * 4 + i]), a[k], false);
        }
        const int p0 = a[0] + 16 * a[1], p1 = a[2] + 16 * a[3], p2 = a[4] + 16 * a[5];
        return fmaf(static_cast<float>(p2), 65536.f, static_cast<float>(p0 + 256 * p1));
    }
}

// Complete dot of a 2048-wide quantised row against the input digits, uniform across the wave; `sc` = 2^-e.
// int8 scales the wave's sum by the row scale, int4 each lane's share by its group scale.
template <WType WT>
__device__ __forceinline__ float row_dot_dig(const Row<WT>& r, const Dig<WT>& dg, float sc) {
    if constexpr (WT == WType::INT8) {
        return wave_sum(dig_part<WT>(r, dg)) * sc * r.s;
    } else {
        return wave_sum(dig_part<WT>(r, dg) * r.s) * sc;
    }
}

// A lane's share of row_dot_dig, scaled by the row's (int8) or the lane's group (int4) scale but not yet summed
// over the wave: lm_head sums its rows together with rows_sum.
template <WType WT>
__device__ __forceinline__ float row_part_dig(const Row<WT>& r, const Dig<WT>& dg) {
    return dig_part<WT>(r, dg) * r.s;
}

// ---- int4 down projection on digits ------------------------------------------------------------
//
// The 8192 SwiGLU outputs a get the same treatment as the normalised inputs of gate_up: one power-of-two
// scale from max |a|, ai = rint(a 2^e), six signed base-16 digits packed like the weights.  Digit word
// (k, m) holds digit k of columns 8m .. 8m + 7 at tab[k * 1024 + m]; a down row's line c gives lane l the
// columns 2048 c + 32 l .. + 31, i.e. words m = 256 c + 4 l + i.
constexpr int kDownWords = INTER / 8;  // digit words per digit

// Thread tid builds the digit words of column groups m = tid + kCT j (j < 4) from the natural-order inputs in
// LDS.  Callers read (this) before a barrier and write the table after it, over the same LDS.
__device__ __forceinline__ void down_digits(const float* a, int e, int tid, uint32_t (&dw)[4][6]) {
    static_assert(INTER / 8 / kCT == 4, "four column groups per thread");
    static_assert(6 * kDownWords <= kBig, "the digit table fits where the inputs were");
    constexpr uint32_t C = 0x888888u;
    const float scale = ldexpf(1.f, e);
#pragma unroll
    for (int j = 0; j < INTER / 8 / kCT; ++j) {
        const int m = tid + kCT * j;
        const f32x4 x0 = reinterpret_cast<const f32x4*>(a)[2 * m], x1 = reinterpret_cast<const f32x4*>(a)[2 * m + 1];
        uint32_t u[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) u[c] = fixed_word(c < 4 ? x0[c] : x1[c - 4], scale, C);
        nibble_words(u, dw[j]);
#pragma unroll
        for (int k = 0; k < 6; ++k) dw[j][k] ^= 0x88888888u;
    }
}

// One int4 down row (4 ring lines) against the digit table; `sc` = 2^-e.  Per line and lane: the six digit
// dot products recombined exactly, times the lane's group scale.
__device__ __forceinline__ float down_dot_dig4(Smem<WType::INT4>& sm, Cons& cs, const uint32_t* tab, float sc, int wave,
                                               int lane, bool& lbad) {
    using C = RingCfg<WType::INT4>;
    static_assert(C::LPR8 == 4, "int4 down rows are 4 lines");
    ring_wait(cs.k + 4, cs.cfull, &sm.full[wave], lbad);
    u32x4 w[4];
    float gs[4];
    ring_read<WType::INT4, 4, true>(sm, cs, 0, wave, lane, w, gs);
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint32_t* t = tab + (g * kWave + lane) * 4;
        u32x4 d[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) d[k] = *reinterpret_cast<const u32x4*>(t + k * kDownWords);
        int a[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int wq = static_cast<int>(w[g][i] ^ 0x88888888u);
#pragma unroll
            for (int k = 0; k < 6; ++k) a[k] = __builtin_amdgcn_sdot8(wq, static_cast<int>(d[k][i]), a[k], false);
        }
        const int p0 = a[0] + 16 * a[1], p1 = a[2] + 16 * a[3], p2 = a[4] + 16 * a[5];
        s = fmaf(fmaf(static_cast<float>(p2), 65536.f, static_cast<float>(p0 + 256 * p1)), gs[g], s);
    }
    ring_advance<WType::INT4>(cs, 4);
    release(sm, cs, wave, lane);
    return wave_sum(s) * sc;
}

// int8: three signed base-256 digits; digit word (k, m) holds digit k of columns 4m .. 4m + 3 at
// tab[k * 2048 + m], so a down row's line c gives lane l the words m = 256 c + 4 l + i.
__device__ __forceinline__ void down_digits8(const float* a, int e, int tid, uint32_t (&dw)[4][6]) {
    constexpr uint32_t C = 0x808080u;
    const float scale = ldexpf(1.f, e);
#pragma unroll
    for (int j = 0; j < INTER / 8 / kCT; ++j) {
        const int m = tid + kCT * j;
        const f32x4 x0 = reinterpret_cast<const f32x4*>(a)[2 * m], x1 = reinterpret_cast<const f32x4*>(a)[2 * m + 1];
        uint32_t u[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) u[c] = fixed_word(c < 4 ? x0[c] : x1[c - 4], scale, C);
        uint32_t P[2][3];
        byte_planes(u[0], u[1], u[2], u[3], P[0]);
        byte_planes(u[4], u[5], u[6], u[7], P[1]);
#pragma unroll
        for (int k = 0; k < 3; ++k)
#pragma unroll
            for (int h = 0; h < 2; ++h) dw[j][2 * k + h] = P[h][k] ^ 0x80808080u;
    }
}

// One int8 down row (8 ring lines, four at a time) against the digit table; `sc` = 2^-e.  The digit dot
// products stay integer over the whole row; the row scale is applied once.
__device__ __forceinline__ float down_dot_dig8(Smem<WType::INT8>& sm, Cons& cs, const uint32_t* tab, float sc, int wave,
                                               int lane, bool& lbad) {
    using C = RingCfg<WType::INT8>;
    static_assert(C::LPR8 == 8, "int8 down rows are 8 lines");
    int a0 = 0, a1 = 0, a2 = 0;
    float rs = 1.f;
#pragma unroll
    for (int c0 = 0; c0 < 8; c0 += 4) {
        ring_wait(cs.k + 4, cs.cfull, &sm.full[wave], lbad);
        u32x4 w[4];
        ring_read<WType::INT8, 4>(sm, cs, 0, wave, lane, w);
        rs = ring_side<WType::INT8>(sm, cs, 0, wave, lane);
        ring_advance<WType::INT8>(cs, 4);
        release(sm, cs, wave, lane);  // the lines are in registers
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t* t = tab + ((c0 + g) * kWave + lane) * 4;
            const u32x4 d0 = *reinterpret_cast<const u32x4*>(t), d1 = *reinterpret_cast<const u32x4*>(t + 2 * kDownWords),
                        d2 = *reinterpret_cast<const u32x4*>(t + 4 * kDownWords);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int wi = static_cast<int>(w[g][i]);
                a0 = __builtin_amdgcn_sdot4(wi, static_cast<int>(d0[i]), a0, false);
                a1 = __builtin_amdgcn_sdot4(wi, static_cast<int>(d1[i]), a1, false);
                a2 = __builtin_amdgcn_sdot4(wi, static_cast<int>(d2[i]), a2, false);
            }
        }
    }
    const float t = fmaf(fmaf(static_cast<float>(a2), 256.f, static_cast<float>(a1)), 256.f, static_cast<float>(a0));
    return wave_sum(t) * sc * rs;
}

// The wave's two down rows r and r + NW at once (ring lines k .. k + 4 LPR8 - 1 in row order): the digit words of
// each column group are read from the table once for both rows, which halves the phase's LDS reads (six digit
// words per weight word).  Same arithmetic per row as down_dot_dig4 / down_dot_dig8.
__device__ __forceinline__ void down_dot2_dig4(Smem<WType::INT4>& sm, Cons& cs, const uint32_t* tab, float sc, int wave,
                                               int lane, bool& lbad, float& d0, float& d1) {
    using C = RingCfg<WType::INT4>;
    static_assert(C::LPR8 == 4 && C::S >= 8, "two int4 down rows fit the ring");
    ring_wait(cs.k + 8, cs.cfull, &sm.full[wave], lbad);
    u32x4 w[8];  // row q's line g at 4 q + g
    float gs[8];
    ring_read<WType::INT4, 8, true>(sm, cs, 0, wave, lane, w, gs);
    float s[2] = {0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint32_t* t = tab + (g * kWave + lane) * 4;
        u32x4 d[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) d[k] = *reinterpret_cast<const u32x4*>(t + k * kDownWords);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            int a[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int wq = static_cast<int>(w[4 * q + g][i] ^ 0x88888888u);
#pragma unroll
                for (int k = 0; k < 6; ++k) a[k] = __builtin_amdgcn_sdot8(wq, static_cast<int>(d[k][i]), a[k], false);
            }
            const int p0 = a[0] + 16 * a[1], p1 = a[2] + 16 * a[3], p2 = a[4] + 16 * a[5];
            s[q] = fmaf(fmaf(static_cast<float>(p2), 65536.f, static_cast<float>(p0 + 256 * p1)), gs[4 * q + g], s[q]);
        }
    }
    ring_advance<WType::INT4>(cs, 8);
    release(sm, cs, wave, lane);
    d0 = wave_sum(s[0]) * sc;
    d1 = wave_sum(s[1]) * sc;
}

__device__ __forceinline__ void down_dot2_dig8(Smem<WType::INT8>& sm, Cons& cs, const uint32_t* tab, float sc, int wave,
                                               int lane, bool& lbad, float& d0, float& d1) {
    using C = RingCfg<WType::INT8>;
    constexpr int R = C::LPR8, HALF = R / 2;  // lines per row; each row is read in two halves of HALF lines
    static_assert(R == 8 && C::S >= 2 * R, "two int8 down rows fit the ring");
    ring_wait(cs.k + 2 * R, cs.cfull, &sm.full[wave], lbad);
    int a[2][3] = {{0, 0, 0}, {0, 0, 0}};
    const float rs0 = ring_side<WType::INT8>(sm, cs, 0, wave, lane), rs1 = ring_side<WType::INT8>(sm, cs, R, wave, lane);
#pragma unroll
    for (int c0 = 0; c0 < R; c0 += HALF) {
        u32x4 w[2][HALF];
#pragma unroll
        for (int q = 0; q < 2; ++q) ring_read<WType::INT8, HALF>(sm, cs, R * q + c0, wave, lane, w[q]);
        // Release what has been read.  The ring holds row 0's R lines, then row 1's: after the first half the lines
        // read form a prefix of HALF (row 1's first half does not extend it), after the second half all 2 R (int8
        // -2.7 us per step on MI355X).
        if (lane == 0) lds_store(&sm.done[wave], cs.k + (c0 == 0 ? HALF : 2 * R));
#pragma unroll
        for (int g = 0; g < HALF; ++g) {
            const uint32_t* t = tab + ((c0 + g) * kWave + lane) * 4;
            const u32x4 e0 = *reinterpret_cast<const u32x4*>(t), e1 = *reinterpret_cast<const u32x4*>(t + 2 * kDownWords),
                        e2 = *reinterpret_cast<const u32x4*>(t + 4 * kDownWords);
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int wi = static_cast<int>(w[q][g][i]);
                    a[q][0] = __builtin_amdgcn_sdot4(wi, static_cast<int>(e0[i]), a[q][0], false);
                    a[q][1] = __builtin_amdgcn_sdot4(wi, static_cast<int>(e1[i]), a[q][1], false);
                    a[q][2] = __builtin_amdgcn_sdot4(wi, static_cast<int>(e2[i]), a[q][2], false);
                }
        }
    }
    ring_advance<WType::INT8>(cs, 2 * R);
    const float t0 = fmaf(fmaf(static_cast<float>(a[0][2]), 256.f, static_cast<float>(a[0][1])), 256.f, static_cast<float>(a[0][0]));
    const float t1 = fmaf(fmaf(static_cast<float>(a[1][2]), 256.f, static_cast<float>(a[1][1])), 256.f, static_cast<float>(a[1][0]));
    d0 = wave_sum(t0) * sc * rs0;
    d1 = wave_sum(t1) * sc * rs1;
}

// Per-chunk sums of the lane's down-projection inputs (the bias correction of quantised chunks);
// the same for every row, so computed once per phase.  The quantised down rows now use the digit
// dots, so only bf16 (with nothing to sum) calls this; the unused variable stays in the quantised
// kernels because deleting it changed int4's schedule of the merge phase (3 us per step slower).
template <WType WT>
struct DownSums {
    float v[RingCfg<WT>::kQuant ? RingCfg<WT>::LPR8 : 1];
};
template <WType WT>
__device__ __forceinline__ void down_sums(const float* x, int lane, DownSums<WT>& ds) {
    using F = Fmt<WT>;
    if constexpr (RingCfg<WT>::kQuant) {
        const f32x4* xq = reinterpret_cast<const f32x4*>(x);
#pragma unroll
        for (int c = 0; c < RingCfg<WT>::LPR8; ++c) {
            float t = 0.f;
#pragma unroll
            for (int q = 0; q < F::CPC / 4; ++q) {
                const f32x4 t4 = xq[(c * (F::CPC / 4) + q) * kWave + lane];
                t += (t4[0] + t4[1]) + (t4[2] + t4[3]);
            }
            ds.v[c] = t;
        }
    }
}

// Dot of one 8192-wide row (down projection) taken from the ring four lines at a time, inputs from
// LDS in the swz layout.
template <WType WT>
__device__ __forceinline__ float down_dot(Smem<WT>& sm, Cons& cs, const float* x, const DownSums<WT>& ds, int wave,
                                          int lane, bool& lbad) {
    using F = Fmt<WT>;
    using C = RingCfg<WT>;
    constexpr int G = 4;
    static_assert(C::LPR8 % G == 0, "down lines");
    float s = 0.f, rs = 1.f;
#pragma unroll
    for (int c0 = 0; c0 < C::LPR8; c0 += G) {
        ring_wait(cs.k + G, cs.cfull, &sm.full[wave], lbad);
        u32x4 w[G];
        float sc[G];
        ring_read<WT, G, C::kQuant>(sm, cs, 0, wave, lane, w, sc);
        ring_advance<WT>(cs, G);
        release(sm, cs, wave, lane);  // the lines are in registers
        // Opaque per group, so the LDS reads of x are not hoisted out of the row loop (the same
        // inputs serve every row of the wave: hoisted, they would pin LPR8 * CPC registers).
        int xo = lane;
        asm volatile("" : "+v"(xo));
        const f32x4* xq = reinterpret_cast<const f32x4*>(x);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float xc[F::CPC];
#pragma unroll
            for (int q = 0; q < F::CPC / 4; ++q) {
                const f32x4 t4 = xq[((c0 + g) * (F::CPC / 4) + q) * kWave + xo];
#pragma unroll
                for (int e = 0; e < 4; ++e) xc[4 * q + e] = t4[e];
            }
            float t = chunk_dot<WT>(w[g], xc);
            if constexpr (C::kQuant) t -= kBias<WT> * ds.v[c0 + g];
            if constexpr (WT == WType::INT4) t *= sc[g];
            s += t;
        }
        if constexpr (WT == WType::INT8) rs = sc[0];
    }
    s = wave_sum(s);
    if constexpr (WT == WType::INT8) s *= rs;
    return s;
}

template <WType WT>
__device__ __forceinline__ float embed(const void* w, const void* s, int tok, int j) {
    const size_t t = static_cast<size_t>(tok);
    if constexpr (WT == WType::BF16) {
        return __builtin_bit_cast(float, static_cast<uint32_t>(gload(static_cast<const uint16_t*>(w) + t * H + j)) << 16);
    } else if constexpr (WT == WType::INT8) {
        return static_cast<float>(gload(static_cast<const int8_t*>(w) + t * H + j)) *
               gload(static_cast<const float*>(s) + t);
    } else {
        const uint8_t b = gload(static_cast<const uint8_t*>(w) + t * (H / 2) + j / 2);
        const int q = static_cast<int>((j & 1) ? (b >> 4) : (b & 0x0F)) - 8;
        return static_cast<float>(q) *
               half_bits_to_float(gload(static_cast<const uint16_t*>(s) + t * (H / 128) + j / 128));
    }
}

// Phase-end timestamp of this workgroup (thread 0), when stamping is enabled.
__device__ __forceinline__ void stamp(const DecodeParams& p, int slot) {
    if (p.stamps && threadIdx.x == 0) *glob(p.stamps + blockIdx.x * kStampSlots + slot) = __builtin_amdgcn_s_memrealtime();
}
// In-phase timestamp, recorded for layer 1 only (slots kInPhase + 2 * phase + {0: input arrived, 1: prologue done}).
constexpr int kInPhase = 100;
__device__ __forceinline__ void stamp_in(const DecodeParams& p, int l, int phase, int k) {
    if (l == 1) stamp(p, kInPhase + 2 * phase + k);
}
// Steps inside the first attention task of layer 1 (slots kAttnSteps + 0..5).
constexpr int kAttnSteps = 112;
__device__ __forceinline__ void stamp_attn(const DecodeParams& p, int l, bool first, int k) {
    if (l == 1 && first) stamp(p, kAttnSteps + k);
}

// SiLU g / (1 + e^-g) from the hardware base-2 exponential and reciprocal (each within about 1 ulp) instead
// of expf's range reduction and an IEEE divide: about a third of the instructions, with a relative error of a
// few 1e-7 for |g| < 20 and at most about 6e-6 where e^-g is a finite float.  Measured on MI355X against the
// exact form: bf16 -2.4, int4 -7.9, int8 -4 us per step (int8 was +10.8 before the layer inputs moved out of
// the LDS, when a shorter gate_up let more streaming overlap the next handoffs).
__device__ __forceinline__ float silu_hw(float g) {
    return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));  // log2(e)
}

// Drain this wave's outstanding global accesses before a row loop.  They are long complete by then
// (earlier phases' stores); without it the compiler, which cannot tell the loop's first iteration
// from the others, waits for them in every iteration before reusing their registers.
__device__ __forceinline__ void drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Argmax order: larger value first, then lower index (numpy's tie rule).  NaN never wins.
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int CTRL>
__device__ __forceinline__ void arg_dpp(float& v, int& i) {
    const float ov = dpp<CTRL>(v);
    const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xf, 0xf, true);
    if (arg_better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}

// Argmax over the 64 lanes of a wave; the result is uniform across the wave.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    arg_dpp<kDppXor1>(v, i);
    arg_dpp<kDppXor2>(v, i);
    arg_dpp<kDppHalfMirror>(v, i);
    arg_dpp<kDppMirror>(v, i);
    float bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float ov = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), r));
        const int oi = __builtin_amdgcn_readlane(i, r);
        if (arg_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    v = bv;
    i = bi;
}

constexpr int kDppRor8 = 0x128;  // row_ror:8: lane i reads lane (i + 8) mod 16 of its 16-lane row

// LSE merge for contexts past 64 splits (more than 8192 positions): one wave per head, the splits in blocks of 64
// (lane s holds split sb + s).  Pass 1 takes the maximum over every block; pass 2 adds up l e^(m - M) per block
// and the o values in split order.  Kept out of line: it is off the hot path, and inlined its state would
// compete for the main loop's registers.
__device__ __noinline__ void merge_long(const uint64_t* tpart, uint64_t* tatt, unsigned tg, int nsplit, int NS, int gw,
                                        int NW, int lane, unsigned* err) {
    const unsigned tag = tg + T_ATT_PART;
    for (int h = gw; h < NH; h += NW) {
        const uint64_t* pp = tpart + static_cast<size_t>(h) * NS * kPartStride;
        auto poll_ml = [&](int sb, float& ms, float& ls) {
            const bool in = sb + lane < nsplit;
            uint64_t vm = static_cast<uint64_t>(tag) << 32, vl = vm;
            if (in) {
                vm = tload(pp + (sb + lane) * kPartStride + HD);
                vl = tload(pp + (sb + lane) * kPartStride + HD + 1);
            }
            unsigned spins = 0;
            while (!(tagged(vm, tag) && tagged(vl, tag)) && !give_up(spins, err)) {
                if (!tagged(vm, tag)) vm = tload(pp + (sb + lane) * kPartStride + HD);
                if (!tagged(vl, tag)) vl = tload(pp + (sb + lane) * kPartStride + HD + 1);
            }
            ms = in ? tvalue(vm) : -INFINITY;
            ls = in ? tvalue(vl) : 0.f;
        };
        float M = -INFINITY;
        for (int sb = 0; sb < nsplit; sb += kWave) {
            float ms, ls;
            poll_ml(sb, ms, ls);
            M = fmaxf(M, wave_max(ms));
        }
        float Lsum = 0.f, acc = 0.f;
        for (int sb64 = 0; sb64 < nsplit; sb64 += kWave) {
            float ms, ls;
            poll_ml(sb64, ms, ls);
            const float e = sb64 + lane < nsplit ? expf(ms - M) : 0.f;
            Lsum += wave_sum(ls * e);
            const int end = min(nsplit, sb64 + kWave);
            for (int sb = sb64; sb < end; ++sb) {
                uint64_t v = tload(pp + sb * kPartStride + lane);
                unsigned spins = 0;
                while (!tagged(v, tag) && !give_up(spins, err)) v = tload(pp + sb * kPartStride + lane);
                acc = fmaf(tvalue(v), __shfl(e, sb - sb64), acc);
            }
        }
        tstore(tatt + h * HD + lane, acc / Lsum, tg + T_ATT);
    }
}

    // 17 to 64 splits: one workgroup per head, its splits spread over the 4 waves.  Head h goes to the
    // workgroup whose attention index (ab above) is G - 32 + h: tasks are dealt in ab order, so these 32 hold
    // the fewest (none up to 28 splits) and start polling first.  Wave w takes splits w Q .. w Q + Q - 1
    // (Q <= 16): every (m, l) and o value in flight at once, one round trip, where one wave per head needed
    // up to four (at 8000 positions, bf16 1361 -> 1547 tok/s on MI355X).  Each wave merges its splits in order
    // against its own maximum, then wave 0 adds the 4 partials in wave order, rescaled to the head's maximum:
    // out = sum_w e^(M_w - M) acc_w / sum_w e^(M_w - M) L_w.  Up to 16 splits the one-wave merge above is
    // faster (its single round has no barrier or LDS step: 7-12 us per step at 2-3 splits).
// Inlined: out of line, its call made the whole step 26-52 us slower on MI355X (the call constrains the caller's
// register allocation around it), where inlined it costs 1-6 us per step at short contexts, which never run it.
template <WType WT>
__device__ __forceinline__ void merge_par(Smem<WT>& sm, const uint64_t* tpart, uint64_t* tatt, unsigned tg, int nsplit, int NS,
                                       unsigned& ep, unsigned ep_in, bool& lbad, unsigned* err, int wave, int lane) {
    const int G = gridDim.x, h = (static_cast<int>(blockIdx.x) + G / 2) % G - (G - NH);
    if (h >= 0) {
        const int Q = (nsplit + kCW - 1) / kCW, s0 = wave * Q, cnt = max(0, min(Q, nsplit - s0));
        const uint64_t* pp = tpart + (static_cast<size_t>(h) * NS + s0) * kPartStride;
        const unsigned tag = tg + T_ATT_PART;
        uint64_t vm = static_cast<uint64_t>(tag) << 32, vl = vm;
        if (lane < cnt) {
            vm = tload(pp + lane * kPartStride + HD);
            vl = tload(pp + lane * kPartStride + HD + 1);
        }
        uint64_t v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            v[k] = k < cnt ? tload(pp + k * kPartStride + lane) : static_cast<uint64_t>(tag) << 32;
        unsigned spins = 0;
        for (;;) {
            bool ok = tagged(vm, tag) && tagged(vl, tag);
#pragma unroll
            for (int k = 0; k < 16; ++k) ok = ok && tagged(v[k], tag);
            if (ok || give_up(spins, err)) break;
            if (!tagged(vm, tag)) vm = tload(pp + lane * kPartStride + HD);
            if (!tagged(vl, tag)) vl = tload(pp + lane * kPartStride + HD + 1);
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (k < cnt && !tagged(v[k], tag)) v[k] = tload(pp + k * kPartStride + lane);
        }
        float* macc = sm.big + kAttnQ;          // [4][64] the waves' partial o sums
        float* mml = sm.big + kAttnQ + 4 * HD;  // [4][2] their maxima and l sums
        cwait(sm.bar, ep_in, lbad);  // every wave has read the qkv input (this region may hold it)
        if (cnt > 0) {
            const float ms = lane < cnt ? tvalue(vm) : -INFINITY, ls = lane < cnt ? tvalue(vl) : 0.f;
            const float Mw = wave_max(ms);
            const float e = lane < cnt ? expf(ms - Mw) : 0.f;
            const float Lw = wave_sum(ls * e);
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (k < cnt) acc = fmaf(tvalue(v[k]), __shfl(e, k), acc);
            macc[wave * HD + lane] = acc;
            if (lane == 0) {
                mml[2 * wave] = Mw;
                mml[2 * wave + 1] = Lw;
            }
        }
        cbar(sm.bar, ep, wave, lane, lbad);
        if (wave == 0) {
            const int nw = (nsplit + Q - 1) / Q;  // waves that hold splits
            float M = mml[0];
            for (int w = 1; w < nw; ++w) M = fmaxf(M, mml[2 * w]);
            float L = 0.f, acc = 0.f;
            for (int w = 0; w < nw; ++w) {
                const float f = expf(mml[2 * w] - M);
                L = fmaf(f, mml[2 * w + 1], L);
                acc = fmaf(f, macc[w * HD + lane], acc);
            }
            tstore(tatt + h * HD + lane, acc / L, tg + T_ATT);
        }
        cbar(sm.bar, ep, wave, lane, lbad);  // macc / mml are read before anything overwrites them
    }
}

// ---- the kernel ------------------------------------------------------------------------------

template <WType WT>
__global__ void __launch_bounds__(kThreads) decode_kernel(DecodeParams p) {
    using F = Fmt<WT>;
    constexpr int NX = F::CPL * F::CPC;
    constexpr bool kDig = WT != WType::BF16;  // gate_up, down and lm_head use the integer dot products
    constexpr bool kQkvDig = WT == WType::INT8;  // and int8's qkv
    // int4 writes the current token's fp16 KV cache rows from the attention workgroup that holds them (one 128-byte
    // store per row) instead of 2-byte stores from 32 waves of the qkv phase: int4 -7 us per step on MI355X; bf16 +3
    // and int8 +1 us, so they keep the qkv phase's stores.
    constexpr bool kKvInAttn = WT == WType::INT4;
    // The quantised kernels score a lane's two tokens in one branch-free loop (int8 -6, int4 -5 us per step with the
    // P.V reduction below); bf16 keeps one branch per token, which measured 3 us faster for it.
    constexpr bool kFastScores = WT != WType::BF16;
    __shared__ Smem<WT> sm;

    if (threadIdx.x < kCW) {
        sm.full[threadIdx.x] = 0;
        sm.done[threadIdx.x] = 0;
        sm.bar[threadIdx.x] = 0;
    }
    __syncthreads();  // the only workgroup-wide barrier: loaders never join another one
    if (p.probe) {  // co-residency probe: arrive, wait (bounded) for every workgroup, leave
        if (threadIdx.x == 0) {
            __hip_atomic_fetch_add(glob(p.probe), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            unsigned spins = 0;
            for (;;) {
                const unsigned n = __hip_atomic_load(glob(p.probe), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const unsigned bad = __hip_atomic_load(glob(p.probe + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (n >= gridDim.x || bad) break;
                if (++spins >= kSpinCap) {
                    __hip_atomic_store(glob(p.probe + 1), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        return;
    }
    {
        const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
        if (w >= kCW) {
            loader<WT>(p, sm, w - kCW, threadIdx.x % kWave);
            return;
        }
    }

    const int G = gridDim.x, NW = G * kCW;
    unsigned* err = p.d_err;
    const int pos = *glob(p.d_pos);
    const int tok = min(max(*glob(p.d_token), 0), VOCAB - 1);
    const unsigned step = *glob(p.d_step);
    // Epochs start at 1: the arena starts zeroed, and a zero tag must never look current.
    const unsigned base = (step + 1u) * kEpochStride;
    const int ctx = pos + 1;
    const int nsplit = (ctx + kAttnChunk - 1) / kAttnChunk;
    const int NS = p.max_seq / kAttnChunk;
    const size_t layer_cache = static_cast<size_t>(NKV) * p.max_seq * HD;

    // An opaque copy of the thread index, renewed at every phase: without it the compiler computes
    // the per-thread addresses of all phases up front and keeps them live across the whole layer.
    int tid = 0, wave = 0, lane = 0, gw = 0;
    auto renew = [&] {
        tid = threadIdx.x;
        asm volatile("" : "+v"(tid)::"memory");
        wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        lane = tid % kWave;
        gw = blockIdx.x * kCW + wave;
    };
    renew();
    unsigned ep = 0;     // compute-barrier epoch
    unsigned ep_in = 0;  // epoch of the last carrive(): every wave has read the phase input in big
    bool lbad = false;   // an in-workgroup wait overran (reported at the end)
    Cons cs;

    stamp(p, 0);
    {
        // The embedding row is layer 0's qkv input: its sum of squares, and for int8 max |x g| (g: layer 0's
        // attn_norm), which the digit prologue of the qkv phase takes as fetch() leaves it for later layers.
        [[maybe_unused]] const float* g0 = kQkvDig ? load_layer(p.layers, 0).attn_norm : nullptr;
        float ss = 0.f, mx = 0.f;
        for (int j = tid; j < H; j += kCT) {
            const float x = embed<WT>(p.emb, p.emb_s, tok, j);
            sm.big[kXin<WT> + j] = x;
            ss += x * x;
            if constexpr (kQkvDig) mx = fmaxf(mx, fabsf(x * gload(g0 + j)));
        }
        ss = wave_sum(ss);
        if (lane == 0) sm.part[wave] = ss;
        if constexpr (kQkvDig) {
            mx = wave_max(mx);
            if (lane == 0) sm.pmax[wave] = mx;
        }
    }
    if (tid < HD / 2) {  // the angles depend only on the position: one sincos per pair per step
        float sn, csn;
        sincosf(static_cast<float>(pos) * gload(p.inv_freq + tid), &sn, &csn);
        sm.rope_s[tid] = sn;
        sm.rope_c[tid] = csn;
    }
    cbar(sm.bar, ep, wave, lane, lbad);
    if (p.residuals && blockIdx.x == 0)
        for (int j = tid; j < H; j += kCT) *glob(p.residuals + j) = sm.big[kXin<WT> + j];

#pragma unroll 1
    for (int l = 0; l < NL; ++l) {
        const DecodeLayer Lw = load_layer(p.layers, l);
        const unsigned tg = base + l * kTagStride;
        uint64_t* tqkv = p.tqkv + static_cast<size_t>(l) * QKV;
        uint64_t* tatt = p.tatt + static_cast<size_t>(l) * H;
        uint64_t* tpart = p.tpart + static_cast<size_t>(l) * NH * NS * kPartStride;
        uint64_t* txa = p.txa + static_cast<size_t>(l) * H;
        uint64_t* tact = p.tact + static_cast<size_t>(l) * INTER;
        uint64_t* txo = p.tx + static_cast<size_t>(l + 1) * H;

        // Attention tasks (kv head, 128-token split) start at workgroup G / 2: at 256 workgroups (MI355X's grid) the
        // second half has one qkv unit per wave and the first half two, so the second half reaches the attention phase
        // sooner (bf16 -8.7, int8 -3.7, int4 -6.5 us per step).  Earlier tokens come from the cache and do not depend
        // on this step, so a task's K/V tile is loaded into registers before its q arrives: the first task's during
        // this workgroup's qkv rows, each later task's (contexts past 4096, more tasks than workgroups) while the
        // task before it computes.
        constexpr int kTile = kAttnChunk * 8 / kCT;  // 16-byte chunks per thread
        const int T = NKV * nsplit;
        const int ab = (static_cast<int>(blockIdx.x) + G / 2) % G;
        u32x4 kt[kTile], vt[kTile];
        auto load_tile = [&](int tt) {
            const int kvh = tt % NKV, t0 = (tt / NKV) * kAttnChunk, n = min(kAttnChunk, ctx - t0);
            const uint16_t* Kg = p.k_cache + l * layer_cache + static_cast<size_t>(kvh) * p.max_seq * HD;
            const uint16_t* Vg = p.v_cache + l * layer_cache + static_cast<size_t>(kvh) * p.max_seq * HD;
#pragma unroll
            for (int k = 0; k < kTile; ++k) {
                const int idx = tid + k * kCT, r = idx / 8, c = idx % 8;
                if (r < n && t0 + r < pos) {
                    kt[k] = load_stream(Kg + static_cast<size_t>(t0 + r) * HD + c * 8);
                    vt[k] = load_stream(Vg + static_cast<size_t>(t0 + r) * HD + c * 8);
                }
            }
        };

        // ---- qkv (+ attn_norm prologue, RoPE, fp16 KV write); unit = RoPE pair (i, i+32) of a head ----
        renew();
        {
            // int8 uses the integer digit dots here too (the digit prologue is about 60 instructions per thread; each
            // row then costs about 40 instead of about 85): int8 -5 us per step.  int4 measured +3 us with them (its
            // float rows were already cheaper than int8's), so it keeps the float path.
            NormW<WT> nw;
            float xr[kQkvDig ? 1 : NX], xsum = 0.f;
            Dig<WT> dg;
            float dsc = 0.f;
            if constexpr (kQkvDig) {
                const Norm8 gn = load_norm8(Lw.attn_norm, tid);
                stall_at(p, kStallQkv);
                if (l > 0) {
                    fetch<H, true, 0, 1, true>(p.tx + static_cast<size_t>(l) * H, tg - kTagStride + T_X, sm.big + kXin<WT>,
                                         sm.part, err, tid, Lw.attn_norm, sm.pmax);
                    cbar(sm.bar, ep, wave, lane, lbad);
                }
                stamp_in(p, l, 0, 0);
                stall_at(p, kStallInputs);
                const float inv = rms_inv(sm.part, p.eps);
                dsc = digits_prologue<WT>(sm, inv, gn, tid, sm.big + kXin<WT>);
                if (lane < kRPW && gw + lane * NW < H) sm.xres[wave * kRPW + lane] = sm.big[kXin<WT> + gw + lane * NW];
                cbar(sm.bar, ep, wave, lane, lbad);
                load_digits<WT>(reinterpret_cast<const uint32_t*>(sm.big + kDigOff), lane, dg);
            } else {
                load_norm<WT>(Lw.attn_norm, lane, nw);
                stall_at(p, kStallQkv);
                if (l > 0) {
                    if constexpr (!kDig) cbar(sm.bar, ep, wave, lane, lbad);  // every wave is done with the down input
                    fetch<H, true>(p.tx + static_cast<size_t>(l) * H, tg - kTagStride + T_X, sm.big + kXin<WT>, sm.part, err,
                                   tid);
                    cbar(sm.bar, ep, wave, lane, lbad);
                }
                stamp_in(p, l, 0, 0);
                stall_at(p, kStallInputs);
                const float inv = rms_inv(sm.part, p.eps);
                lane_inputs<WT, true>(sm.big + kXin<WT>, &nw, inv, xr, xsum, lane);
                if (lane < kRPW && gw + lane * NW < H) sm.xres[wave * kRPW + lane] = sm.big[kXin<WT> + gw + lane * NW];
            }
            ep_in = carrive(sm.bar, ep, wave, lane);  // the attention tiles may now overwrite the input / digit table
            stamp_in(p, l, 0, 1);
            drain();
            if (ab < T) load_tile(ab);
#pragma unroll 1
            for (int u = gw; u < kPairs; u += NW) {
                Row<WT> ra, rb;
                take_row<WT>(sm, cs, wave, lane, lbad, ra);
                take_row<WT>(sm, cs, wave, lane, lbad, rb);
                release_early<WT>(sm, cs, wave, lane);
                float d0, d1;
                if constexpr (kQkvDig) {
                    d0 = row_dot_dig<WT>(ra, dg, dsc);
                    d1 = row_dot_dig<WT>(rb, dg, dsc);
                } else {
                    d0 = row_dot<WT>(ra, xr, xsum);
                    d1 = row_dot<WT>(rb, xr, xsum);
                }
                release_late<WT>(sm, cs, wave, lane);
                if (lane == 0) {
                    const int h = u / 32, i = u % 32, r0 = h * HD + i;
                    float o0 = d0, o1 = d1;
                    if (h < NH + NKV) {
                        o0 = d0 * sm.rope_c[i] - d1 * sm.rope_s[i];
                        o1 = d1 * sm.rope_c[i] + d0 * sm.rope_s[i];
                    }
                    tstore(tqkv + r0, o0, tg + T_QKV);
                    tstore(tqkv + r0 + 32, o1, tg + T_QKV);
                    if (!kKvInAttn && h >= NH) {
                        uint16_t* cache = h < NH + NKV ? p.k_cache : p.v_cache;
                        const size_t off = l * layer_cache + (static_cast<size_t>((h - NH) % NKV) * p.max_seq + pos) * HD;
                        *glob(cache + off + i) = float_to_half_bits(o0);
                        *glob(cache + off + i + 32) = float_to_half_bits(o1);
                    }
                }
            }
        }
        stamp(p, 1 + 6 * l + 0);

        // ---- split-K attention: task = (kv head, 128-token split), one workgroup per task ----
        renew();
        {
            uint32_t* Ks = reinterpret_cast<uint32_t*>(sm.big);       // [128][kKs] fp16 pairs
            u32x4* Vs = reinterpret_cast<u32x4*>(sm.big + kAttnV);     // [128][8]
            float* ps = sm.big + kAttnP;                               // [4][128]
            float* qs = sm.big + kAttnQ;                               // [4][64]
            uint16_t* Ks16 = reinterpret_cast<uint16_t*>(Ks);
            uint16_t* Vs16 = reinterpret_cast<uint16_t*>(Vs);
            stall_at(p, kStallAttn);
#pragma unroll 1
            for (int t = ab; t < T; t += G) {
                const int kvh = t % NKV, split = t / NKV;
                const int t0 = split * kAttnChunk, n = min(kAttnChunk, ctx - t0);
                const bool first = t == ab;
                stamp_attn(p, l, first, 0);
                {
                    if ((!kDig || kQkvDig) && first) cwait(sm.bar, ep_in, lbad);  // every wave has read the qkv input (or its digits)
#pragma unroll
                    for (int k = 0; k < kTile; ++k) {
                        const int idx = tid + k * kCT, r = idx / 8, c = idx % 8;
                        if (r < n && t0 + r < pos) {
                            *reinterpret_cast<u32x4*>(Ks + r * kKs + c * 4) = kt[k];
                            Vs[r * 8 + c] = vt[k];
                        }
                    }
                    if (t + G < T) load_tile(t + G);
                }
                // q of the group's 4 heads (thread = head-in-group x dim) and, in the split holding this
                // token, its k and v, rounded to fp16 exactly as the qkv phase wrote them to the cache.
                const uint64_t* qa = tqkv + (kvh * 4) * HD + tid;
                const bool cur = tid < 2 * HD && t0 + n - 1 == pos;
                float qv, kv;
                wait2(qa, cur ? tqkv + (tid < HD ? NH * HD : (NH + NKV) * HD - HD) + kvh * HD + tid : qa, tg + T_QKV, err,
                      qv, kv);
                qs[tid] = qv;
                if (cur) {
                    // The current token's k (wave 0) and v (wave 1) into the tiles; for int4 also into the fp16 cache,
                    // one 128-byte row per wave (the workgroup of the split holding pos is the one writer per kv head).
                    const int r = pos - t0;
                    const uint16_t hb = float_to_half_bits(kv);
                    if (tid < HD) {
                        Ks16[r * 2 * kKs + tid] = hb;
                        if constexpr (kKvInAttn)
                            *glob(p.k_cache + l * layer_cache + (static_cast<size_t>(kvh) * p.max_seq + pos) * HD + tid) = hb;
                    } else {
                        Vs16[r * HD + tid - HD] = hb;
                        if constexpr (kKvInAttn)
                            *glob(p.v_cache + l * layer_cache + (static_cast<size_t>(kvh) * p.max_seq + pos) * HD + tid - HD) = hb;
                    }
                }
                stamp_attn(p, l, first, 1);
                cbar(sm.bar, ep, wave, lane, lbad);
                if (first) stamp_in(p, l, 1, 0);
                stamp_attn(p, l, first, 2);
                // wave w = query head kvh*4 + w; lane scores tokens lane and lane + 64.
                float s[2];
                {
                    f32x4 qv[HD / 4];
#pragma unroll
                    for (int i = 0; i < HD / 4; ++i) qv[i] = *reinterpret_cast<const f32x4*>(qs + wave * HD + 4 * i);
                    if constexpr (kFastScores) {
                        // Both tokens in one loop, without a branch (rows past n hold stale values and are selected
                        // away below), so the two tokens' FMA chains interleave.
                        float dd[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                        for (int i = 0; i < HD / 8; ++i) {
#pragma unroll
                            for (int k = 0; k < 2; ++k) {
                                const u32x4 kk = *reinterpret_cast<const u32x4*>(Ks + (lane + kWave * k) * kKs + 4 * i);
#pragma unroll
                                for (int e = 0; e < 4; ++e) {
                                    dd[k][e] = fmaf(half_bits_to_float(static_cast<uint16_t>(kk[e])), qv[2 * i + e / 2][2 * (e % 2)], dd[k][e]);
                                    dd[k][e] = fmaf(half_bits_to_float(static_cast<uint16_t>(kk[e] >> 16)), qv[2 * i + e / 2][2 * (e % 2) + 1], dd[k][e]);
                                }
                            }
                        }
#pragma unroll
                        for (int k = 0; k < 2; ++k)  // 4 chains per token: 2.5-5.5 us per step
                            s[k] = lane + kWave * k < n ? 0.125f * ((dd[k][0] + dd[k][1]) + (dd[k][2] + dd[k][3])) : -INFINITY;
                    } else {
#pragma unroll
                        for (int k = 0; k < 2; ++k) {
                            const int j = lane + kWave * k;
                            if (j < n) {
                                float dd[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                                for (int i = 0; i < HD / 8; ++i) {
                                    const u32x4 kk = *reinterpret_cast<const u32x4*>(Ks + j * kKs + 4 * i);
#pragma unroll
                                    for (int e = 0; e < 4; ++e) {
                                        dd[e] = fmaf(half_bits_to_float(static_cast<uint16_t>(kk[e])), qv[2 * i + e / 2][2 * (e % 2)], dd[e]);
                                        dd[e] = fmaf(half_bits_to_float(static_cast<uint16_t>(kk[e] >> 16)), qv[2 * i + e / 2][2 * (e % 2) + 1], dd[e]);
                                    }
                                }
                                s[k] = 0.125f * ((dd[0] + dd[1]) + (dd[2] + dd[3]));  // 4 chains: 2.5-5.5 us per step
                            } else {
                                s[k] = -INFINITY;
                            }
                        }
                    }
                }
                const float m = wave_max(fmaxf(s[0], s[1]));
                const float p0 = lane < n ? expf(s[0] - m) : 0.f;
                const float p1 = lane + kWave < n ? expf(s[1] - m) : 0.f;
                const float lsum = wave_sum(p0 + p1);
                ps[wave * kAttnChunk + lane] = p0;
                ps[wave * kAttnChunk + lane + kWave] = p1;
                stamp_attn(p, l, first, 3);
                // P.V: lane = (token phase g, 8-column group c) takes tokens g, g+8, ... of columns
                // 8c..8c+7; the 8 token phases are then summed across lanes.
                const int g = lane >> 3, c = lane & 7;
                float o[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = 0.f;
                const int iters = (n - g + 7) / 8;  // tokens g + 8 i < n
#pragma unroll 4
                for (int i = 0; i < iters; ++i) {
                    const int j = g + 8 * i;
                    const float pj = ps[wave * kAttnChunk + j];
                    const u32x4 vv = Vs[j * 8 + c];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        o[2 * e] = fmaf(pj, half_bits_to_float(static_cast<uint16_t>(vv[e])), o[2 * e]);
                        o[2 * e + 1] = fmaf(pj, half_bits_to_float(static_cast<uint16_t>(vv[e] >> 16)), o[2 * e + 1]);
                    }
                }
                const int h = kvh * 4 + wave;
                // The 8 token phases summed across lanes: within each 16-lane row by DPP, across rows by the
                // permlane swaps (lanes l and l ^ 16, then l and l ^ 32), without a trip through the LDS unit.
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    o[e] += dpp<kDppRor8>(o[e]);
                    o[e] = sum_lanes_xor<16>(o[e]);
                    o[e] = sum_lanes_xor<32>(o[e]);
                }
                // Every lane holds its column group's 8 sums; lane j takes column j (element j % 8 of group j / 8)
                // through the wave's q slot in LDS (its q is in registers), so the wave writes its 64 outputs with
                // one store: whole 64-byte lines.
                float* ot = qs + wave * HD;
                if (lane < 8) {
                    *reinterpret_cast<f32x4*>(ot + 8 * lane) = f32x4{o[0], o[1], o[2], o[3]};
                    *reinterpret_cast<f32x4*>(ot + 8 * lane + 4) = f32x4{o[4], o[5], o[6], o[7]};
                }
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                const float oj = ot[lane];
                if (nsplit == 1) {
                    tstore(tatt + h * HD + lane, oj * (1.f / lsum), tg + T_ATT);
                } else {
                    uint64_t* pp = tpart + (static_cast<size_t>(h) * NS + split) * kPartStride;
                    tstore(pp + lane, oj, tg + T_ATT_PART);
                    if (lane == 0) {
                        tstore(pp + HD, m, tg + T_ATT_PART);
                        tstore(pp + HD + 1, lsum, tg + T_ATT_PART);
                    }
                }
                stamp_attn(p, l, first, 4);
                cbar(sm.bar, ep, wave, lane, lbad);  // the tiles are overwritten next (or by the wo input)
                stamp_attn(p, l, first, 5);
            }
        }
        stamp(p, 1 + 6 * l + 1);

        // ---- LSE merge of the splits ----
        renew();
        if (nsplit > 1 && nsplit <= kMergeOneWave) {
            // Up to 16 splits, one wave per head: lane s holds split s, and each lane's (m, l) and the o values of
            // every split are in flight at once (one round trip).
#pragma unroll 1
            for (int h = gw; h < NH; h += NW) {
                const uint64_t* pp = tpart + static_cast<size_t>(h) * NS * kPartStride;
                const unsigned tag = tg + T_ATT_PART;
                uint64_t vm = static_cast<uint64_t>(tag) << 32, vl = vm;
                if (lane < nsplit) {
                    vm = tload(pp + lane * kPartStride + HD);
                    vl = tload(pp + lane * kPartStride + HD + 1);
                }
                float M = 0.f, e = 0.f, Lsum = 0.f, acc = 0.f;
#pragma unroll 1
                for (int sb = 0; sb < nsplit; sb += kMergeOneWave) {
                    uint64_t v[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k)
                        v[k] = sb + k < nsplit ? tload(pp + (sb + k) * kPartStride + lane) : static_cast<uint64_t>(tag) << 32;
                    unsigned spins = 0;
                    for (;;) {
                        bool ok = tagged(vm, tag) && tagged(vl, tag);
#pragma unroll
                        for (int k = 0; k < 16; ++k) ok = ok && tagged(v[k], tag);
                        if (ok || give_up(spins, err)) break;
                        if (!tagged(vm, tag)) vm = tload(pp + lane * kPartStride + HD);
                        if (!tagged(vl, tag)) vl = tload(pp + lane * kPartStride + HD + 1);
#pragma unroll
                        for (int k = 0; k < 16; ++k)
                            if (sb + k < nsplit && !tagged(v[k], tag)) v[k] = tload(pp + (sb + k) * kPartStride + lane);
                    }
                    if (sb == 0) {
                        const float ms = lane < nsplit ? tvalue(vm) : -INFINITY;
                        const float ls = lane < nsplit ? tvalue(vl) : 0.f;
                        M = wave_max(ms);
                        e = lane < nsplit ? expf(ms - M) : 0.f;
                        Lsum = wave_sum(ls * e);
                    }
#pragma unroll
                    for (int k = 0; k < 16; ++k)
                        if (sb + k < nsplit) acc = fmaf(tvalue(v[k]), __shfl(e, sb + k), acc);
                }
                tstore(tatt + h * HD + lane, acc / Lsum, tg + T_ATT);
            }
        } else if (nsplit > kMergeOneWave && nsplit <= kWave) {
            merge_par(sm, tpart, tatt, tg, nsplit, NS, ep, ep_in, lbad, err, wave, lane);
        } else if (nsplit > kWave) {
            merge_long(tpart, tatt, tg, nsplit, NS, gw, NW, lane, err);
        }
        stamp(p, 1 + 6 * l + 2);

        // ---- wo + residual ----
        renew();
        {
            stall_at(p, kStallWo);
            if constexpr (!kDig) cwait(sm.bar, ep_in, lbad);  // every wave has read the qkv input (as above)
            fetch<H, false, 0, 0, true>(tatt, tg + T_ATT, sm.big, sm.part, err, tid);
            cbar(sm.bar, ep, wave, lane, lbad);
            stamp_in(p, l, 3, 0);
            stall_at(p, kStallInputs);
            float xr[NX], xsum;
            lane_inputs<WT, false>(sm.big, nullptr, 1.f, xr, xsum, lane);
            ep_in = carrive(sm.bar, ep, wave, lane);  // gate_up's input may now overwrite this one
            stamp_in(p, l, 3, 1);
            drain();
            int k = wave * kRPW;
#pragma unroll 1
            for (int r = gw; r < H; r += NW, ++k) {
                Row<WT> rw;
                take_row<WT>(sm, cs, wave, lane, lbad, rw);
                release_early<WT>(sm, cs, wave, lane);
                const float d = row_dot<WT>(rw, xr, xsum);
                release_late<WT>(sm, cs, wave, lane);
                if (lane == 0) {
                    const float xa = sm.xres[k] + d;
                    tstore(txa + r, xa, tg + T_XA);
                    sm.ares[k] = xa;
                }
            }
        }
        stamp(p, 1 + 6 * l + 3);

        // ---- gate_up (+ ffn_norm prologue, SwiGLU); unit = gate row u and up row u + inter ----
        renew();
        {
            NormW<WT> nw;
            float xr[kDig ? 1 : NX], xsum = 0.f;
            Dig<WT> dg;
            float dsc = 0.f;
            stall_at(p, kStallGateUp);
            if constexpr (kDig) {
                const Norm8 gn = load_norm8(Lw.ffn_norm, tid);
                fetch<H, true, 0, 1, WT == WType::INT8>(txa, tg + T_XA, sm.big + kXgu<WT>, sm.part, err, tid, Lw.ffn_norm, sm.pmax);
                cbar(sm.bar, ep, wave, lane, lbad);
                stamp_in(p, l, 4, 0);
                stall_at(p, kStallInputs);
                const float inv = rms_inv(sm.part, p.eps);
                dsc = digits_prologue<WT>(sm, inv, gn, tid, sm.big + kXgu<WT>);
                cbar(sm.bar, ep, wave, lane, lbad);
                load_digits<WT>(reinterpret_cast<const uint32_t*>(sm.big + kDigOff), lane, dg);
            } else {
                load_norm<WT>(Lw.ffn_norm, lane, nw);
                cwait(sm.bar, ep_in, lbad);  // every wave has read wo's input
                fetch<H, true>(txa, tg + T_XA, sm.big, sm.part, err, tid);
                cbar(sm.bar, ep, wave, lane, lbad);
                stamp_in(p, l, 4, 0);
                stall_at(p, kStallInputs);
                const float inv = rms_inv(sm.part, p.eps);
                lane_inputs<WT, true>(sm.big, &nw, inv, xr, xsum, lane);
                ep_in = carrive(sm.bar, ep, wave, lane);  // the down projection's input may now overwrite it
            }
            stamp_in(p, l, 4, 1);
            drain();
            // Not software-pipelined (unlike lm_head): holding the next unit's rows across the
            // iteration pushed the int4 kernel into VGPR spills, and that build gave wrong, run-to-run
            // varying results once the loader ran a layer ahead (a 13 us stall before the down
            // projection's input was enough).  The pipelined form saved 1.6 us per int4 step.
#pragma unroll 1
            for (int u = gw; u < INTER; u += NW) {
                Row<WT> rg, ru;
                take_row<WT>(sm, cs, wave, lane, lbad, rg);
                take_row<WT>(sm, cs, wave, lane, lbad, ru);
                release_early<WT>(sm, cs, wave, lane);
                float gv, uv;
                if constexpr (kDig) {
                    gv = row_dot_dig<WT>(rg, dg, dsc);
                    uv = row_dot_dig<WT>(ru, dg, dsc);
                } else {
                    gv = row_dot<WT>(rg, xr, xsum);
                    uv = row_dot<WT>(ru, xr, xsum);
                }
                release_late<WT>(sm, cs, wave, lane);
                if (lane == 0) tstore(tact + u, silu_hw(gv) * uv, tg + T_ACT);
            }
        }
        stamp(p, 1 + 6 * l + 4);

        // ---- down + residual (8192-wide rows, inputs read from LDS) ----
        renew();
        {
            stall_at(p, kStallDown);
            [[maybe_unused]] DownSums<WT> dsum;
            [[maybe_unused]] float dsc = 0.f;
            if constexpr (kDig) {
                // Digits, as in gate_up: natural-order inputs, their max, the digit words in registers, a
                // barrier (every thread has read its inputs), then the table over the same LDS.
                fetch<INTER, false, 0, 2>(tact, tg + T_ACT, sm.big, sm.part, err, tid, nullptr, sm.pmax);
                cbar(sm.bar, ep, wave, lane, lbad);
                stamp_in(p, l, 5, 0);
                float m = 0.f;
#pragma unroll
                for (int w = 0; w < kCW; ++w) m = fmaxf(m, sm.pmax[w]);
                const int e = dig_exponent(m);
                dsc = ldexpf(1.f, -e);
                uint32_t dw[4][6];
                if constexpr (WT == WType::INT4) {
                    down_digits(sm.big, e, tid, dw);
                } else {
                    down_digits8(sm.big, e, tid, dw);
                }
                cbar(sm.bar, ep, wave, lane, lbad);
                uint32_t* tab = reinterpret_cast<uint32_t*>(sm.big);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int k = 0; k < 6; ++k) {
                        if constexpr (WT == WType::INT4) {
                            tab[k * kDownWords + tid + kCT * j] = dw[j][k];
                        } else {  // digit k / 2, word 2 m + k % 2 of the 4-column words
                            tab[(k / 2) * 2 * kDownWords + 2 * (tid + kCT * j) + k % 2] = dw[j][k];
                        }
                    }
                cbar(sm.bar, ep, wave, lane, lbad);
            } else {
                cwait(sm.bar, ep_in, lbad);  // every wave has read gate_up's input
                fetch<INTER, false, F::CPC>(tact, tg + T_ACT, sm.big, sm.part, err, tid);
                cbar(sm.bar, ep, wave, lane, lbad);
                stamp_in(p, l, 5, 0);
                stall_at(p, kStallInputs);
                down_sums<WT>(sm.big, lane, dsum);
            }
            stamp_in(p, l, 5, 1);
            drain();
            int k = wave * kRPW;
            int r = gw;
            if constexpr (kDig) {
#pragma unroll 1
                for (; r + NW < H; r += 2 * NW, k += 2) {
                    float d0, d1;
                    if constexpr (WT == WType::INT4) {
                        down_dot2_dig4(sm, cs, reinterpret_cast<const uint32_t*>(sm.big), dsc, wave, lane, lbad, d0, d1);
                    } else {
                        down_dot2_dig8(sm, cs, reinterpret_cast<const uint32_t*>(sm.big), dsc, wave, lane, lbad, d0, d1);
                    }
                    if (lane == 0) {
                        const float x0 = sm.ares[k] + d0, x1 = sm.ares[k + 1] + d1;
                        tstore(txo + r, x0, tg + T_X);
                        tstore(txo + r + NW, x1, tg + T_X);
                        if (p.residuals) {
                            *glob(p.residuals + static_cast<size_t>(l + 1) * H + r) = x0;
                            *glob(p.residuals + static_cast<size_t>(l + 1) * H + r + NW) = x1;
                        }
                    }
                }
            }
#pragma unroll 1
            for (; r < H; r += NW, ++k) {
                float d;
                if constexpr (WT == WType::INT4) {
                    d = down_dot_dig4(sm, cs, reinterpret_cast<const uint32_t*>(sm.big), dsc, wave, lane, lbad);
                } else if constexpr (WT == WType::INT8) {
                    d = down_dot_dig8(sm, cs, reinterpret_cast<const uint32_t*>(sm.big), dsc, wave, lane, lbad);
                } else {
                    d = down_dot<WT>(sm, cs, sm.big, dsum, wave, lane, lbad);
                }
                if (lane == 0) {
                    const float xn = sm.ares[k] + d;
                    tstore(txo + r, xn, tg + T_X);
                    if (p.residuals) *glob(p.residuals + static_cast<size_t>(l + 1) * H + r) = xn;
                }
            }
        }
        stamp(p, 1 + 6 * l + 5);
    }

    // ---- lm_head (+ final norm) with the argmax folded in; unit = kLmR consecutive rows ----
    renew();
    {
        NormW<WT> nw;
        float xr[kDig ? 1 : NX], xsum = 0.f;
        Dig<WT> dg;
        float dsc = 0.f;
        const uint64_t* tfin = p.tx + static_cast<size_t>(NL) * H;
        const unsigned tagfin = base + (NL - 1) * kTagStride + T_X;
        stall_at(p, kStallLmHead);
        if constexpr (kDig) {
            const Norm8 gn = load_norm8(p.final_norm, tid);
            fetch<H, true, 0, true>(tfin, tagfin, sm.big + kXin<WT>, sm.part, err, tid, p.final_norm, sm.pmax);
            cbar(sm.bar, ep, wave, lane, lbad);
            const float inv = rms_inv(sm.part, p.eps);
            dsc = digits_prologue<WT>(sm, inv, gn, tid, sm.big + kXin<WT>);
            cbar(sm.bar, ep, wave, lane, lbad);
            load_digits<WT>(reinterpret_cast<const uint32_t*>(sm.big + kDigOff), lane, dg);
        } else {
            load_norm<WT>(p.final_norm, lane, nw);
            cbar(sm.bar, ep, wave, lane, lbad);  // every wave is done with the down projection's input
            fetch<H, true>(tfin, tagfin, sm.big, sm.part, err, tid);
            cbar(sm.bar, ep, wave, lane, lbad);
            const float inv = rms_inv(sm.part, p.eps);
            lane_inputs<WT, true>(sm.big, &nw, inv, xr, xsum, lane);
        }
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        // Logits are collected across lanes (lane j holds the wave's j-th row) and stored 64 at a time:
        // a store per row would make every iteration wait for the previous one's store to drain.
        float lg = 0.f;
        int lr = 0, nrow = 0;
        drain();
        // Not software-pipelined: a unit's lines are taken and multiplied before the next unit's are read (the
        // take-ahead form held the next unit's rows across the iteration, the pattern that gave layout-dependent
        // wrong results in gate_up).
#pragma unroll 1
        for (int u = gw; u < VOCAB / kLmR<WT>; u += NW) {
            Row<WT> rr[kLmR<WT>];
#pragma unroll
            for (int i = 0; i < kLmR<WT>; ++i) take_row<WT>(sm, cs, wave, lane, lbad, rr[i]);
            release_early<WT>(sm, cs, wave, lane);
            float d[kLmR<WT>];
            if constexpr (kDig) {
                // The unit's rows are summed together: lane l ends with row l mod kLmR, which is the logit it
                // stores (lane nrow + i holds row i) and the only row it compares for the argmax.
#pragma unroll
                for (int i = 0; i < kLmR<WT>; ++i) d[i] = row_part_dig<WT>(rr[i], dg);
                release_late<WT>(sm, cs, wave, lane);
                const float x = rows_sum<kLmR<WT>>(d, lane) * dsc;
                const int r = u * kLmR<WT> + lane % kLmR<WT>;
                if (lane / kLmR<WT> == nrow / kLmR<WT>) {
                    lg = x;
                    lr = r;
                }
                if (arg_better(x, r, bv, bi)) {
                    bv = x;
                    bi = r;
                }
            } else {
#pragma unroll
                for (int i = 0; i < kLmR<WT>; ++i) d[i] = row_dot<WT>(rr[i], xr, xsum);
                release_late<WT>(sm, cs, wave, lane);
#pragma unroll
                for (int i = 0; i < kLmR<WT>; ++i) {
                    const int r = u * kLmR<WT> + i;
                    if (lane == nrow + i) {
                        lg = d[i];
                        lr = r;
                    }
                    if (arg_better(d[i], r, bv, bi)) {
                        bv = d[i];
                        bi = r;
                    }
                }
            }
            nrow += kLmR<WT>;
            if (nrow == kWave) {  // wave-uniform: a branch, so the drain below runs only here
                *glob(p.logits + lr) = lg;
                drain();  // nothing left pending for the hot path
                nrow = 0;
            }
        }
        if (lane < nrow) *glob(p.logits + lr) = lg;
        if constexpr (kDig) {  // lanes l and l' hold the same rows when l = l' mod kLmR: reduce over l mod kLmR
            static_assert(kLmR<WT> <= 8, "the argmax reduction covers up to 8 lanes");
            if constexpr (kLmR<WT> >= 2) arg_dpp<kDppXor1>(bv, bi);
            if constexpr (kLmR<WT> >= 4) arg_dpp<kDppXor2>(bv, bi);
            if constexpr (kLmR<WT> >= 8) arg_dpp<kDppHalfMirror>(bv, bi);
        }
        if (lane == 0) {
            sm.red_v[wave] = bv;
            sm.red_i[wave] = bi;
        }
        cbar(sm.bar, ep, wave, lane, lbad);
        if (tid == 0) {
            for (int w = 1; w < kCW; ++w)
                if (arg_better(sm.red_v[w], sm.red_i[w], bv, bi)) {
                    bv = sm.red_v[w];
                    bi = sm.red_i[w];
                }
            tstore(p.targ + 2 * blockIdx.x, bv, base + T_ARG);
            tstore(p.targ + 2 * blockIdx.x + 1, __builtin_bit_cast(float, bi), base + T_ARG);
        }
        cbar(sm.bar, ep, wave, lane, lbad);  // red_* are reused below
    }
    stamp(p, 97);

    // ---- final argmax over the workgroups' partials (wave trees); token and position advance on device ----
    if (blockIdx.x == 0) {
        float v = -INFINITY;
        int i = 0x7fffffff;
        for (int g = tid; g < G; g += kCT) {
            float gv, gf;
            wait2(p.targ + 2 * g, p.targ + 2 * g + 1, base + T_ARG, err, gv, gf);
            const int gi = __builtin_bit_cast(int, gf);
            if (arg_better(gv, gi, v, i)) {
                v = gv;
                i = gi;
            }
        }
        wave_argmax(v, i);
        if (lane == 0) {
            sm.red_v[wave] = v;
            sm.red_i[wave] = i;
        }
        cbar(sm.bar, ep, wave, lane, lbad);
        if (tid == 0) {
            for (int w = 1; w < kCW; ++w)
                if (arg_better(sm.red_v[w], sm.red_i[w], v, i)) {
                    v = sm.red_v[w];
                    i = sm.red_i[w];
                }
            *glob(p.d_token) = min(max(i, 0), VOCAB - 1);
            *glob(p.d_pos) = pos + 1;
            *glob(p.d_step) = step + 1;
        }
        stamp(p, 98);
    }
    if (lbad) fail(err);
}

}  // namespace dk

int decode_max_grid(WType wt) {
    int b = 0;
    switch (wt) {
        case WType::BF16:
            CLLM_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, dk::decode_kernel<WType::BF16>, kDecodeThreads, 0));
            break;
        case WType::INT8:
            CLLM_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, dk::decode_kernel<WType::INT8>, kDecodeThreads, 0));
            break;
        case WType::INT4:
            CLLM_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, dk::decode_kernel<WType::INT4>, kDecodeThreads, 0));
            break;
    }
    return b * device_cu_count();
}

namespace {

const void* decode_fn(WType wt) {
    switch (wt) {
        case WType::BF16: return reinterpret_cast<const void*>(&dk::decode_kernel<WType::BF16>);
        case WType::INT8: return reinterpret_cast<const void*>(&dk::decode_kernel<WType::INT8>);
        case WType::INT4: return reinterpret_cast<const void*>(&dk::decode_kernel<WType::INT4>);
    }
    throw ArgError("decode: unknown weight type");
}

}  // namespace

// A plain launch.  A cooperative launch (hipLaunchCooperativeKernel) would have the runtime guarantee
// co-residency, but it measured about 18 us per step slower on MI355X for every weight type; the engine
// instead verifies co-residency once with decode_grid_is_resident, and every wait in the kernel is bounded.
void launch_decode(WType wt, const DecodeParams& p, int grid, hipStream_t s) {
    CLLM_REQUIRE(grid >= kDecodeMinGrid && grid <= kDecodeMaxGrid && grid % 8 == 0,
                 "decode: grid must be a multiple of 8 in 64..4096 workgroups");
    CLLM_REQUIRE(p.max_seq > 0 && p.max_seq % kAttnChunk == 0 && p.max_seq <= kDecodeMaxSeq,
                 "decode: max_seq must be a multiple of 128 and at most 131072");
    DecodeParams arg = p;
    void* args[] = {&arg};
    CLLM_HIP(hipLaunchKernel(decode_fn(wt), dim3(grid), dim3(kDecodeThreads), args, 0, s));
}

bool decode_grid_is_resident(WType wt, const DecodeParams& p, int grid, unsigned* probe, hipStream_t s) {
    CLLM_REQUIRE(probe, "decode probe: null counter");
    DecodeParams arg = p;
    arg.probe = probe;
    void* args[] = {&arg};
    CLLM_HIP(hipLaunchKernel(decode_fn(wt), dim3(grid), dim3(kDecodeThreads), args, 0, s));
    unsigned host[2] = {0, 0};
    CLLM_HIP(hipMemcpyAsync(host, probe, sizeof(host), hipMemcpyDeviceToHost, s));
    CLLM_HIP(hipStreamSynchronize(s));
    return host[1] == 0 && host[0] == static_cast<unsigned>(grid);
}

}  // namespace cllm
