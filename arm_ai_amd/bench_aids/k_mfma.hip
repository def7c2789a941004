// k_mfma.hip -- measurement aid for bench.py, built into libaq_bench.so (not
// part of libarm_ai_amd.so or its ABI; no counterpart in the reference).
//
// The rate the matrix cores sustain on this GPU for the MFMA shapes the GEMMs
// use, in a register-only loop: four independent accumulator chains per
// wavefront, no memory traffic inside the loop.  bench.py reports it next to
// the GEMMs' fractions of the published peak, as the practical ceiling of
// the instruction itself.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// KIND 0: v_mfma_i32_32x32x32_i8, 1: v_mfma_i32_16x16x64_i8,
// 2: v_mfma_f32_32x32x16_f16.  Each lane writes one int of out.
template <int KIND>
__global__ __launch_bounds__(256) void mfma_loop(int iters, int *out) {
    const int t = (int)threadIdx.x;
    const v4i a = {t, 1, 2, 3}, b = {3, 2, 1, t};
    const _Float16 h1 = (_Float16)1, h2 = (_Float16)2;
    const v8h ha = {h1, h2, h1, h2, h1, h2, h1, h2};
    v16i c[4] = {};
    v4i e[4] = {};
    v16f f[4] = {};
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (KIND == 0) c[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[u], 0, 0, 0);
            else if (KIND == 1) e[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, e[u], 0, 0, 0);
            else f[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, ha, f[u], 0, 0, 0);
        }
    }
    int s = 0;
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += c[u][r] + (int)f[u][r] + (r < 4 ? e[u][r] : 0);
    out[blockIdx.x * 256 + t] = s;
}

}  // namespace

extern "C" {

// MACs one wavefront's MFMA of `kind` performs (0 for an unknown kind).
long long aq_bench_mfma_macs(int kind) {
    return kind == 0 ? 32LL * 32 * 32 : kind == 1 ? 16LL * 16 * 64 : kind == 2 ? 32LL * 32 * 16 : 0;
}

// One launch of `grid` 256-thread workgroups, each wavefront issuing
// 4 * iters MFMAs of `kind`, on `stream`; d_out holds grid * 256 ints.
// Returns 0, -1 for bad arguments, -5 for a launch error.
int aq_bench_mfma(int kind, void *stream, int grid, int iters, int *d_out) {
    if (kind < 0 || kind > 2 || grid <= 0 || iters <= 0 || !d_out) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (kind == 0) mfma_loop<0><<<grid, 256, 0, s>>>(iters, d_out);
    else if (kind == 1) mfma_loop<1><<<grid, 256, 0, s>>>(iters, d_out);
    else mfma_loop<2><<<grid, 256, 0, s>>>(iters, d_out);
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

}  // extern "C"
