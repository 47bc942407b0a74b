// Host check of the persistent decode kernel's weight walk (cudallm_amd/csrc/decode_walk.h): for every weight type,
// segment and sampled compute wave, the lines the loader streams (seg_of + Walker::advance, run on byte offsets)
// must be exactly the lines of the rows the compute side multiplies, in the same order: row r of a matrix with
// row_bytes B is lines r*B + 1024 c, c < B / 1024, with side values at r*S + 32 c (int4) or r*S (int8).
//
//   walk_check GRID [GRID ...]      prints "ok GRID" per grid that matches, or the first mismatch, and exits 1 on any
//
// The compute side below restates decode.hip's phase loops (u = gw, gw + NW, ... and their row formulas); lm_head
// units of 1, 2, 4 and 8 rows are checked (the kernel uses 2 for bf16 and 8 for int8/int4).
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "decode_walk.h"

using namespace cllm;

namespace {

// Rows of segment s that compute wave gw multiplies, in order (decode.hip: qkv pairs, wo rows, gate_up units,
// down rows, lm_head units).
std::vector<long> compute_rows(int s, int gw, int NW, int lm_rows) {
    std::vector<long> rows;
    switch (s) {
        case 0:
            for (int u = gw; u < walk::kPairs; u += NW) {
                const long r = (u / 32) * walk::kHd + u % 32;
                rows.push_back(r);
                rows.push_back(r + 32);
            }
            break;
        case 1:
        case 3:
            for (int r = gw; r < walk::kH; r += NW) rows.push_back(r);
            break;
        case 2:
            for (int u = gw; u < walk::kInter; u += NW) {
                rows.push_back(u);
                rows.push_back(u + walk::kInter);
            }
            break;
        default:
            for (int u = gw; u < walk::kVocab / lm_rows; u += NW)
                for (int i = 0; i < lm_rows; ++i) rows.push_back(static_cast<long>(u) * lm_rows + i);
    }
    return rows;
}

bool check(WType wt, int s, int gw, int NW, int grid, int lm_rows) {
    const int cols = s == 3 ? walk::kInter : walk::kH;
    const long rb = walk::row_bytes(wt, cols), sb = walk::side_bytes(wt, cols);
    const long lpr = rb / 1024;
    std::vector<long> want, swant;
    for (long r : compute_rows(s, gw, NW, lm_rows))
        for (long c = 0; c < lpr; ++c) {
            want.push_back(r * rb + 1024 * c);
            swant.push_back(r * sb + (wt == WType::INT4 ? 32 * c : 0));
        }
    walk::Walker<long> w;
    w.start(walk::seg_of(wt, s, gw, NW, lm_rows), 0L, 0L);
    size_t n = 0;
    for (; w.have; w.advance(), ++n) {
        if (n >= want.size() || w.cur != want[n] || (wt != WType::BF16 && w.scur != swant[n])) {
            std::printf("mismatch grid %d wtype %d segment %d wave %d (lm rows %d) line %zu: walk %ld/%ld, rows give "
                        "%ld/%ld\n", grid, static_cast<int>(wt), s, gw, lm_rows, n, w.cur, w.scur, n < want.size() ? want[n] : -1L,
                        n < swant.size() ? swant[n] : -1L);
            return false;
        }
    }
    if (n != want.size()) {
        std::printf("mismatch grid %d wtype %d segment %d wave %d: walk has %zu lines, rows give %zu\n", grid,
                    static_cast<int>(wt), s, gw, n, want.size());
        return false;
    }
    return true;
}

}  // namespace

int main(int argc, char** argv) {
    int bad = 0;
    for (int a = 1; a < argc; ++a) {
        const int grid = std::atoi(argv[a]), NW = 4 * grid;
        bool ok = true;
        for (WType wt : {WType::BF16, WType::INT8, WType::INT4})
            for (int s = 0; s < 5 && ok; ++s)
                for (int gw : {0, 1, 31, 32, 33, NW / 2 + 5, NW - 33, NW - 1})
                    for (int lm_rows : {1, 2, 4, 8})
                        if (ok && gw >= 0 && gw < NW) ok = check(wt, s, gw, NW, grid, lm_rows);
        if (ok) std::printf("ok %d\n", grid);
        bad += !ok;
    }
    return bad ? 1 : 0;
}
