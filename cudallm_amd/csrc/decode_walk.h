// The persistent decode kernel's weight schedule for one compute wave, in host and device code: which rows the wave
// multiplies in each phase (the compute side) and the 1 KiB lines its loader streams for them, in order (the loader
// side).  The kernel's loader walks it with real addresses; tests/test_decode_walk.py compiles walk_check.cpp, which
// checks the two sides against each other for many grid sizes.
#pragma once

#include <cstdint>

#include "common.h"

namespace cllm {
namespace walk {

constexpr int kH = 2048, kInter = 8192, kHd = 64, kVocab = 128256;
constexpr int kPairs = (32 + 2 * 8) * kHd / 2;  // RoPE pairs (i, i + 32) of every q/k/v head

// Columns per 16-byte chunk (8 bf16, 16 int8, 32 int4), bytes per row, and side-value bytes per row: the int8 row
// scale (fp32) or the int4 group scales (fp16 per 128 columns); bf16 rows have none.
__host__ __device__ constexpr int cols_per_chunk(WType wt) { return wt == WType::BF16 ? 8 : wt == WType::INT8 ? 16 : 32; }
__host__ __device__ constexpr long row_bytes(WType wt, int cols) { return static_cast<long>(cols) * 16 / cols_per_chunk(wt); }
__host__ __device__ constexpr long side_bytes(WType wt, int cols) { return wt == WType::INT4 ? (cols / 128) * 2L : 4L; }

// Segment s of a layer: 0 qkv (unit = RoPE pair: rows r and r + 32 of one head), 1 wo, 2 gate_up (gate row u, then
// up row u + inter), 3 down (8192 columns); 4 is lm_head (unit = lm_rows consecutive vocabulary rows).  Unit u
// belongs to compute wave gw when u = gw (mod NW); the compute side takes a unit's rows in that order.
struct Seg {
    int units;                        // units of the wave
    int rpu, lpr;                     // rows per unit, lines per row
    long first, sfirst;               // offsets of the wave's first line and of its side values
    long drow, dunit, sdrow, sdunit;  // extra steps at a row's end and at a unit's end
    long sline;                       // side-value step per line (int4: the line's 16 groups; int8: 0)
};

__host__ __device__ inline Seg seg_of(WType wt, int s, int gw, int NW, int lm_rows) {
    int N, r0, krows, urows, rpu, cols;
    if (s == 4) {
        N = kVocab / lm_rows, r0 = gw * lm_rows, krows = 1, urows = NW * lm_rows, rpu = lm_rows, cols = kH;
    } else {
        N = s == 0 ? kPairs : s == 2 ? kInter : kH;
        // qkv: unit u is pair (u % 32) of head u / 32, rows 64 (u / 32) + u % 32 and + 32; with NW a multiple of 32
        // the next unit of the wave, u + NW, starts 2 NW rows further on.
        r0 = s == 0 ? (gw / 32) * kHd + gw % 32 : gw;
        krows = s == 0 ? 32 : s == 2 ? kInter : 0;
        urows = s == 0 ? 2 * NW : NW;
        rpu = (s == 0 || s == 2) ? 2 : 1;
        cols = s == 3 ? kInter : kH;
    }
    const long rb = row_bytes(wt, cols), sb = side_bytes(wt, cols);
    Seg g;
    g.lpr = static_cast<int>(rb / 1024);
    g.rpu = rpu;
    g.units = (N - gw + NW - 1) / NW;
    g.sline = wt == WType::INT4 ? 32 : 0;
    const long kstr = krows * rb, ustr = urows * rb, skstr = krows * sb, sustr = urows * sb;
    // Every line moves on by one line (and sline); a row's end adds drow, a unit's end adds dunit on top.
    g.drow = kstr - g.lpr * 1024L;
    g.sdrow = skstr - g.lpr * g.sline;
    g.dunit = ustr - rpu * kstr;
    g.sdunit = sustr - rpu * skstr;
    g.first = r0 * rb;
    g.sfirst = r0 * sb;
    return g;
}

// A cursor over a segment's lines: P is const char* in the kernel (addresses) and long in the host check (offsets).
// The common step is two additions and a counter: a wave issues one instruction per 4 cycles, and the loader takes
// one step per line, so this bookkeeping bounds the streaming rate of a loader wave.
template <typename P>
struct Walker {
    P cur, scur;
    int lc, rc, ul, lpr, rpu;
    long drow, dunit, sdrow, sdunit, sline;
    bool have;

    __host__ __device__ void start(const Seg& g, P base, P sbase) {
        cur = base + g.first;
        scur = sbase + g.sfirst;
        lc = 0, rc = 0, ul = g.units, lpr = g.lpr, rpu = g.rpu;
        drow = g.drow, dunit = g.dunit, sdrow = g.sdrow, sdunit = g.sdunit, sline = g.sline;
        have = ul > 0;
    }
    // Past the current line; clears `have` at the segment's end (cur then points past the segment and is not read).
    __host__ __device__ __forceinline__ void advance() {
        cur += 1024;
        scur += sline;
        if (++lc < lpr) return;
        lc = 0;
        cur += drow;
        scur += sdrow;
        if (++rc < rpu) return;
        rc = 0;
        cur += dunit;
        scur += sdunit;
        if (--ul == 0) have = false;
    }
};

}  // namespace walk
}  // namespace cllm
