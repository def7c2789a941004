// rl_plan.h -- launch planning of the row-per-lane matvec (k_rowlane.hip):
// which form a weight takes (56-, 16- or 8-row workgroups), how many
// workgroups it launches, and the check every launch passes before it is
// issued.  Plain host C++ with no HIP types, so that a CPU test can compile
// it with g++ and sweep the shapes.
#pragma once

#include <stdint.h>

namespace aq {
namespace rl {

constexpr int ROWS56 = 56;    // weight rows per workgroup of the wide form (one row per lane)
constexpr int MAXG = 64;      // groups per row (k <= 16384)
constexpr int MIN_N56 = 200 * ROWS56;  // rows from which the 56-row form is used (up to 32 groups)
constexpr int ROWS16 = 16;    // weight rows per workgroup of the four-group-phase form
constexpr int MIN_N16 = 16 * ROWS16;   // rows from which that form is used (up to 64 groups)
constexpr int ROWS8 = 8;      // weight rows per workgroup of the eight-group-phase form
// ... used from 1025 to 2048 rows (up to 32 groups): at most one 8-row
// workgroup per CU, where 16-row workgroups would leave half the CUs idle
constexpr int MIN_N8 = 64 * ROWS16 + 1, MAX_N8 = 256 * ROWS8;
constexpr int PERSIST_CUS = 256;  // the persistent grid: one workgroup per CU
constexpr int NORM_MAXG = 32;     // the fused norm: rows of up to 8192 elements

// 56-row workgroups: up to two Q4_K-like groups per wavefront (32 groups),
// one Q6_K group (16); Q8_0 (17 pieces) never.
inline bool wide(bool q6, bool q80, int64_t n, int ng) { return !q80 && ng <= (q6 ? 16 : 32) && n >= MIN_N56; }
// 8-row workgroups (otherwise 16 rows), for a shape that is not wide
inline bool narrow8(int64_t n, int ng) { return ng <= 32 && n >= MIN_N8 && n <= MAX_N8; }

struct Plan {
    int rows;         // weight rows per workgroup (56, 16 or 8)
    unsigned grid;    // workgroups launched
    bool persistent;  // a workgroup walks chunks blockIdx, blockIdx + grid, ...
};

// The launch of one weight of n rows and ng groups per row.  A chunk is one
// workgroup's `rows` rows; without persistence every chunk is one
// workgroup, with it (more 56-row chunks than CUs, up to 16 groups) one
// workgroup per CU walks every 256th chunk.
inline Plan plan(bool q6, bool q80, int64_t n, int ng) {
    Plan p;
    p.persistent = false;
    if (wide(q6, q80, n, ng)) {
        p.rows = ROWS56;
        const int64_t nch = (n + ROWS56 - 1) / ROWS56;
        if (ng <= 16 && nch > PERSIST_CUS) {
            p.persistent = true;
            p.grid = PERSIST_CUS;
        } else {
            p.grid = (unsigned)nch;
        }
        return p;
    }
    p.rows = narrow8(n, ng) ? ROWS8 : ROWS16;
    p.grid = (unsigned)((n + p.rows - 1) / p.rows);
    return p;
}

// Every launch passes this before it is issued.  A workgroup past the last
// chunk would address rows past the weight (a chunk's row-block range is
// computed from its index), so a grid must hold exactly one workgroup per
// chunk, or -- persistent -- at most as many workgroups as chunks, each
// owning at least its first one.
inline bool grid_ok(int rows, int64_t n, int64_t grid, bool persistent) {
    if (rows <= 0 || n <= 0 || grid <= 0) return false;
    const int64_t chunks = (n + rows - 1) / rows;
    return persistent ? grid <= chunks : grid == chunks;
}

}  // namespace rl
}  // namespace aq
