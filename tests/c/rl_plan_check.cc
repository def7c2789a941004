// rl_plan_check.cc -- CPU check of the row-per-lane matvec's launch planning
// (arm_ai_amd/csrc/rl_plan.h, the code k_rowlane.hip launches with): every
// planned grid passes the launch check and covers every row, and the check
// refuses grids with a workgroup past the chunks (test infrastructure; built
// and run by tests/test_rowlane_plan.py).
#include <cstdio>

#include "../../arm_ai_amd/csrc/rl_plan.h"

using namespace aq::rl;

static int bad = 0;
static void expect(bool ok, const char *what, long long a, long long b) {
    if (!ok) {
        if (bad < 20) std::printf("FAIL %s (%lld, %lld)\n", what, a, b);
        bad++;
    }
}

int main() {
    long long checked = 0;
    const bool kinds[3][2] = {{false, false}, {true, false}, {false, true}};  // Q4_K-like, Q6_K, Q8_0
    for (const auto &kd : kinds) {
        for (int ng = 1; ng <= MAXG; ng++) {
            for (long long n = 1; n <= 300000; n += (n < 4200 ? 1 : n < 20000 ? 7 : 997)) {
                const Plan p = plan(kd[0], kd[1], n, ng);
                checked++;
                expect(grid_ok(p.rows, n, p.grid, p.persistent), "planned grid refused", n, ng);
                expect(p.persistent || (long long)p.grid * p.rows >= n, "rows left uncovered", n, ng);
                expect(!p.persistent || (p.rows == ROWS56 && p.grid == PERSIST_CUS && ng <= 16), "persistent shape", n, ng);
                expect(p.rows == ROWS56 || p.rows == ROWS16 || p.rows == ROWS8, "row form", n, ng);
            }
        }
    }
    // the grid that faulted in development: 512 persistent workgroups on a
    // 286-chunk shape (the kernel read past the weight), and its neighbours
    const long long n286 = 286LL * ROWS56 - 10;
    expect(!grid_ok(ROWS56, n286, 512, true), "512 persistent on 286 chunks accepted", n286, 512);
    expect(!grid_ok(ROWS56, n286, 287, true), "287 persistent on 286 chunks accepted", n286, 287);
    expect(grid_ok(ROWS56, n286, 256, true), "256 persistent on 286 chunks refused", n286, 256);
    expect(grid_ok(ROWS56, n286, 286, true), "one persistent workgroup per chunk refused", n286, 286);
    expect(!grid_ok(ROWS56, n286, 287, false), "a workgroup past the chunks accepted", n286, 287);
    expect(!grid_ok(ROWS16, 4096, 257, false), "257 on 256 chunks accepted", 4096, 257);
    expect(!grid_ok(ROWS16, 4096, 255, false), "a chunk without a workgroup accepted", 4096, 255);
    expect(grid_ok(ROWS16, 4096, 256, false), "one workgroup per chunk refused", 4096, 256);
    expect(!grid_ok(ROWS8, 0, 1, false), "an empty weight accepted", 0, 1);
    expect(!grid_ok(ROWS8, 8, 0, false), "an empty grid accepted", 8, 0);
    std::printf("checked %lld plans, %d failures\n", checked, bad);
    return bad ? 1 : 0;
}
