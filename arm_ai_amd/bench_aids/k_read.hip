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

}  // extern "C"
