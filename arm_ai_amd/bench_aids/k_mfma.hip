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

// The issue cost of v_mfma_i32_32x32x32_i8 next to VALU work: four
// independent accumulator chains per wavefront on operands loaded from
// memory (random bytes, as a GEMM's), each MFMA followed by NV independent
// f32 fmas, the two kinds interleaved by sched_group_barrier; launch bounds
// (256, 2) and 512 workgroups give two wavefronts per SIMD.  Time per MFMA
// per SIMD against NV shows how much of the VALU work the matrix core hides.
// F16: v_mfma_f32_32x32x16_f16 instead, on random integers as a Q4_K GEMM
// without the scale split would feed it (weights sc*q in 0..945, activations
// -128..127, both exact in f16).
template <int NV, bool F16>
__global__ __launch_bounds__(256, 2) void coexec_loop(const int *src, int iters, int *out) {
    const int t = (int)threadIdx.x;
    v4i a[2], b[2];
    v8h ha[2], hb[2];
    for (int i = 0; i < 2; i++) {
        a[i] = *(const v4i *)(src + 8 * t + 4 * i);
        b[i] = *(const v4i *)(src + 2048 + 8 * t + 4 * i);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            ha[i][j] = (_Float16)(float)((uint32_t)src[8 * t + j + 4 * i] % 946u);
            hb[i][j] = (_Float16)(float)((int)((uint32_t)src[2048 + 8 * t + j + 4 * i] % 256u) - 128);
        }
    }
    float f[8];
    for (int i = 0; i < 8; i++) f[i] = (float)(src[4096 + t + i] & 255);
    const float g = 0.5f + (float)(src[5000 + t] & 1), hh = (float)(src[5100 + t] & 7);
    v16i c[4] = {};
    v16f cf[4] = {};
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (F16) cf[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha[(u >> 1) & 1], hb[u & 1], cf[u], 0, 0, 0);
            else c[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[(u >> 1) & 1], b[u & 1], c[u], 0, 0, 0);
#pragma unroll
            for (int v = 0; v < NV; v++) f[v & 7] = __builtin_fmaf(f[v & 7], g, hh);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA, then the NV fmas
            if (NV) __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
        }
    }
    int s = 0;
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += c[u][r] + (int)cf[u][r];
    for (int i = 0; i < 8; i++) s += (int)f[i];
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

// coexec_loop<nv> for nv in {0, 4, 8, 16}: 512 workgroups (two wavefronts
// per SIMD), each wavefront issuing 4 * iters MFMAs; d_src holds 8192 ints
// (the operands), d_out 512 * 256 ints.  Returns 0, -1 for bad arguments, -5
// for a launch error.
int aq_bench_coexec(int nv, void *stream, int iters, const int *d_src, int *d_out) {
    if (iters <= 0 || !d_src || !d_out) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (nv == 0) coexec_loop<0, false><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else if (nv == 4) coexec_loop<4, false><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else if (nv == 8) coexec_loop<8, false><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else if (nv == 16) coexec_loop<16, false><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

// The same with v_mfma_f32_32x32x16_f16 (coexec_loop<nv, true>).
int aq_bench_coexec_f16(int nv, void *stream, int iters, const int *d_src, int *d_out) {
    if (iters <= 0 || !d_src || !d_out) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (nv == 0) coexec_loop<0, true><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else if (nv == 4) coexec_loop<4, true><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else if (nv == 8) coexec_loop<8, true><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else if (nv == 16) coexec_loop<16, true><<<512, 256, 0, s>>>(d_src, iters, d_out);
    else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

}  // extern "C"
