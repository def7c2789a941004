// k_launch.hip -- measurement aid for bench.py, built into libaq_bench.so (not
// part of libarm_ai_amd.so or its ABI; no counterpart in the reference).
//
// The cost of one dependent kernel launch on this GPU: bench.py captures a
// chain of launches of this empty kernel in a HIP graph and times a replay.
// The decode step is a chain of such launches, so this is the floor under
// every kernel of it.
#include <hip/hip_runtime.h>

namespace {

__global__ __launch_bounds__(64) void empty_kernel(int *out) {
    if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = 1;
}

}  // namespace

extern "C" {

// One launch of `grid` 64-thread workgroups on `stream`; d_out holds 1 int.
// Returns 0, -1 for bad arguments, -5 for a launch error.
int aq_bench_empty(void *stream, int grid, int *d_out) {
    if (grid <= 0 || !d_out) return -1;
    empty_kernel<<<grid, 64, 0, (hipStream_t)stream>>>(d_out);
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

}  // extern "C"
