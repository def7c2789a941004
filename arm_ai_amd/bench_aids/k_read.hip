// k_read.hip -- measurement aid for bench.py, built into libaq_bench.so (not
// part of libarm_ai_amd.so or its ABI; no counterpart in the reference).
//
// A family of kernels that only stream a buffer from HBM.  bench.py times
// every member on the headline matvec's byte count and reports the fastest as
// the read rate a single launch of that many bytes reaches on this GPU: the
// practical ceiling the matvec's roofline fraction is read against.
//
// Members (16-byte nontemporal buffer loads, results folded so the loads stay
// live):
//   one-shot: workgroup b reads its own contiguous span, each thread L loads
//             that are all issued before any is consumed (grid = bytes /
//             (threads * L * 16));
//   strided:  a fixed grid walks the buffer with a grid-stride loop, L loads
//             in flight per thread per step.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../csrc/aq_internal.h"

using namespace aq;

namespace {

template <int L>
__global__ void read_oneshot(const uint8_t *buf, uint32_t bytes, uint32_t *out) {
    const rsrc_t r = buf_rsrc(buf, bytes);
    const uint32_t base = (uint32_t)blockIdx.x * blockDim.x * L * 16 + threadIdx.x * 16;
    u32x4 a[L];
#pragma unroll
    for (int j = 0; j < L; j++) a[j] = __builtin_amdgcn_raw_buffer_load_b128(r, base + j * blockDim.x * 16, 0, BUF_NT);
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < L; j++) acc ^= a[j].x ^ a[j].y ^ a[j].z ^ a[j].w;
    if (acc == 0x9E3779B9u) out[blockIdx.x % 1024] = acc;
}

template <int L>
__global__ void read_strided(const uint8_t *buf, uint32_t bytes, uint32_t *out) {
    const rsrc_t r = buf_rsrc(buf, bytes);
    const uint32_t step = gridDim.x * blockDim.x * L * 16;
    uint32_t acc = 0;
    for (uint32_t base = (uint32_t)blockIdx.x * blockDim.x * L * 16 + threadIdx.x * 16; base < bytes; base += step) {
        u32x4 a[L];
#pragma unroll
        for (int j = 0; j < L; j++) a[j] = __builtin_amdgcn_raw_buffer_load_b128(r, base + j * blockDim.x * 16, 0, BUF_NT);
#pragma unroll
        for (int j = 0; j < L; j++) acc ^= a[j].x ^ a[j].y ^ a[j].z ^ a[j].w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x % 1024] = acc;
}

// The headline matvec's own access pattern, loads only: Q4_K weights of
// rows of ng groups in the row-block tile layout (8-row blocks of ng * 9
// pieces of 128 bytes, one 16-byte piece per row), taken in 56-row chunks;
// lane l of a wavefront is row l of its chunk (lanes 56-63 idle) and
// wavefront w of the chunk group w, P pieces in flight, as the row-per-lane
// kernel walks them.  CM = false: the layout the library stores, so one load
// instruction reads seven 128-byte lines one block (ng * 1152 bytes) apart;
// CM = true: the same pieces stored chunk-major (the chunk's seven lines of a
// piece next to each other), so it reads 896 contiguous bytes.  WAVES
// wavefronts per workgroup, ng / WAVES workgroups per chunk.
// GPW > 1: a wavefront takes GPW consecutive groups of its chunk (NPG * GPW
// pieces, P of them in flight), one workgroup of ng / GPW wavefronts per
// chunk.
template <bool CM, int WAVES, int P, int GPW = 1>
__global__ void read_pattern(const uint8_t *buf, int ng, uint32_t *out) {
    constexpr int NPG = 9, ROWS = 56, NP = NPG * GPW;
    const uint32_t rbs = (uint32_t)ng * NPG * 128;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int per_chunk = ng / (WAVES * GPW);
    const int chunk = blockIdx.x / per_chunk;
    const int g0 = ((blockIdx.x % per_chunk) * WAVES + wave) * GPW;
    const rsrc_t r = buf_rsrc(buf + (size_t)chunk * (ROWS / 8) * rbs, (ROWS / 8) * rbs);
    auto off = [&](int j) -> uint32_t {
        if (lane >= ROWS) return BUF_OOB;
        const int g = g0 + j / NPG, pc = j % NPG;
        return CM ? (uint32_t)((g * NPG + pc) * ROWS * 16 + lane * 16)
                  : (uint32_t)((lane / 8) * rbs + (g * NPG + pc) * 128 + (lane % 8) * 16);
    };
    u32x4 ring[P];
#pragma unroll
    for (int j = 0; j < P; j++) ring[j] = __builtin_amdgcn_raw_buffer_load_b128(r, off(j), 0, BUF_NT);
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < NP; j++) {
        acc ^= ring[j % P].x ^ ring[j % P].y ^ ring[j % P].z ^ ring[j % P].w;
        if (j + P < NP) ring[j % P] = __builtin_amdgcn_raw_buffer_load_b128(r, off(j + P), 0, BUF_NT);
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x % 1024] = acc;
}

struct Pattern {
    const char *name;
    bool cm;
    int waves, p;
};
const Pattern PATTERNS[] = {
    {"matvec pattern: row-block layout, 1024-thread workgroups, 6 pieces in flight", false, 16, 6},
    {"matvec pattern: row-block layout, 1024-thread workgroups, 9 pieces in flight", false, 16, 9},
    {"matvec pattern: row-block layout, 256-thread workgroups, 6 pieces in flight", false, 4, 6},
    {"matvec pattern: chunk-major layout, 1024-thread workgroups, 6 pieces in flight", true, 16, 6},
    {"matvec pattern: chunk-major layout, 256-thread workgroups, 6 pieces in flight", true, 4, 6},
    {"matvec pattern: row-block layout, one 256-thread workgroup per chunk, 4 groups per wavefront, all 36 pieces in flight", false, 4, 36},
    {"matvec pattern: row-block layout, one 256-thread workgroup per chunk, 4 groups per wavefront, 18 pieces in flight", false, 4, 18},
    {"matvec pattern: row-block layout, one 512-thread workgroup per chunk, 2 groups per wavefront, all 18 pieces in flight", false, 8, 18},
};
constexpr int N_PATTERNS = sizeof(PATTERNS) / sizeof(PATTERNS[0]);

struct Member {
    const char *name;
    int oneshot, loads, threads, grid;  // grid 0: one-shot (from the byte count)
};
const Member MEMBERS[] = {
    {"one-shot, 256 threads, 1 load each", 1, 1, 256, 0},
    {"one-shot, 256 threads, 2 loads each", 1, 2, 256, 0},
    {"one-shot, 256 threads, 4 loads each", 1, 4, 256, 0},
    {"one-shot, 512 threads, 4 loads each", 1, 4, 512, 0},
    {"one-shot, 512 threads, 8 loads each", 1, 8, 512, 0},
    {"one-shot, 1024 threads, 8 loads each", 1, 8, 1024, 0},
    {"strided, 2048 x 512 threads, 4 loads in flight", 0, 4, 512, 2048},
    {"strided, 512 x 512 threads, 2 loads in flight", 0, 2, 512, 512},
    {"strided, 1024 x 256 threads, 2 loads in flight", 0, 2, 256, 1024},
};
constexpr int N_MEMBERS = sizeof(MEMBERS) / sizeof(MEMBERS[0]);

}  // namespace

extern "C" {

int aq_bench_read_members(void) { return N_MEMBERS; }

const char *aq_bench_read_name(int member) {
    return member >= 0 && member < N_MEMBERS ? MEMBERS[member].name : "";
}

// Stream d_buf (16-byte aligned, bytes a multiple of 16, < 2^31) through read
// kernel `member` on `stream` (a hipStream_t); d_out: 1024 uint32 of device
// memory (almost never written).  Returns 0, or -1 for bad arguments and -5
// for a launch error.
int aq_bench_read(int member, void *stream, const void *d_buf, size_t bytes, uint32_t *d_out) {
    if (member < 0 || member >= N_MEMBERS || !d_buf || !d_out || bytes < 16 || (bytes & 15) ||
        bytes >= ((size_t)1 << 31) || ((uintptr_t)d_buf & 15))
        return -1;
    const Member &m = MEMBERS[member];
    const hipStream_t s = (hipStream_t)stream;
    const uint8_t *b = (const uint8_t *)d_buf;
    const uint32_t n = (uint32_t)bytes;
    const unsigned grid = m.grid ? (unsigned)m.grid : (unsigned)((bytes + (size_t)m.threads * m.loads * 16 - 1) /
                                                                ((size_t)m.threads * m.loads * 16));
    if (m.oneshot) {
        switch (m.loads) {
        case 1: read_oneshot<1><<<grid, m.threads, 0, s>>>(b, n, d_out); break;
        case 2: read_oneshot<2><<<grid, m.threads, 0, s>>>(b, n, d_out); break;
        case 4: read_oneshot<4><<<grid, m.threads, 0, s>>>(b, n, d_out); break;
        default: read_oneshot<8><<<grid, m.threads, 0, s>>>(b, n, d_out); break;
        }
    } else {
        if (m.loads == 4) read_strided<4><<<grid, m.threads, 0, s>>>(b, n, d_out);
        else read_strided<2><<<grid, m.threads, 0, s>>>(b, n, d_out);
    }
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

int aq_bench_read_patterns(void) { return N_PATTERNS; }

const char *aq_bench_read_pattern_name(int v) { return v >= 0 && v < N_PATTERNS ? PATTERNS[v].name : ""; }

// Read the Q4_K weight of n rows x ng groups (n a multiple of 56, ng a
// multiple of 16, at most 64; n * ng * 144 bytes of d_buf, 16-byte aligned)
// in access pattern v.  Returns 0, -1 for bad arguments (or an ng the
// pattern's wavefronts x groups do not divide), -5 for a launch error.
int aq_bench_read_pattern(int v, void *stream, const void *d_buf, int n, int ng, uint32_t *d_out) {
    if (v < 0 || v >= N_PATTERNS || !d_buf || !d_out || n <= 0 || n % 56 || ng <= 0 || ng % 16 || ng > 64 ||
        (int64_t)n * ng * 144 >= ((int64_t)1 << 31) || ((uintptr_t)d_buf & 15))
        return -1;
    const Pattern &pt = PATTERNS[v];
    const hipStream_t s = (hipStream_t)stream;
    const uint8_t *b = (const uint8_t *)d_buf;
    const int gpw = v >= 5 ? (pt.waves == 4 ? 4 : 2) : 1;  // groups per wavefront
    if (ng % (pt.waves * gpw)) return -1;
    const unsigned grid = (unsigned)(n / 56) * (unsigned)(ng / (pt.waves * gpw));
    const unsigned thr = 64u * pt.waves;
    switch (v) {
    case 0: read_pattern<false, 16, 6><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    case 1: read_pattern<false, 16, 9><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    case 2: read_pattern<false, 4, 6><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    case 3: read_pattern<true, 16, 6><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    case 4: read_pattern<true, 4, 6><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    case 5: read_pattern<false, 4, 36, 4><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    case 6: read_pattern<false, 4, 18, 4><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    default: read_pattern<false, 8, 18, 2><<<grid, thr, 0, s>>>(b, ng, d_out); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -5;
}

}  // extern "C"
