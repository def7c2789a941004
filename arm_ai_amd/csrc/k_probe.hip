// k_probe.hip -- a measurement aid, not part of the quantized-matmul path:
// a kernel that does nothing but stream a buffer from HBM, so bench.py can
// report, beside the headline matvec, the read rate a read-only kernel of
// the same byte count reaches on this GPU (the practical ceiling the
// matvec's roofline fraction should be read against).
//
// 512 workgroups of 512 threads; each thread keeps two 16-byte nontemporal
// loads in flight per step of a grid-stride loop (the fastest of grids
// 256-2048 and 1-4 loads per thread, measured on a 33 MB buffer).
#include "aq_internal.h"

namespace aq {

namespace {

constexpr int PROBE_THREADS = 512;
constexpr int PROBE_GRID = 512;

__global__ __launch_bounds__(PROBE_THREADS) void stream_read_kernel(const u32x4 *__restrict__ p, int64_t n16,
                                                                    uint32_t *__restrict__ out) {
    uint32_t acc = 0;
    const int64_t step = (int64_t)gridDim.x * PROBE_THREADS * 2;
    for (int64_t i = (int64_t)blockIdx.x * PROBE_THREADS * 2 + threadIdx.x; i < n16; i += step) {
        const u32x4 a = __builtin_nontemporal_load(p + i);
        const u32x4 b = i + PROBE_THREADS < n16 ? __builtin_nontemporal_load(p + i + PROBE_THREADS) : (u32x4){0, 0, 0, 0};
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
    }
    // keeps the loads live; out has one entry per workgroup
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

}  // namespace

int stream_read_grid() { return PROBE_GRID; }

hipError_t launch_stream_read(const void *buf, size_t bytes, uint32_t *out, hipStream_t s) {
    if (!buf || !out || bytes < 16 || (bytes & 15) || ((uintptr_t)buf & 15)) return hipErrorInvalidValue;
    stream_read_kernel<<<PROBE_GRID, PROBE_THREADS, 0, s>>>((const u32x4 *)buf, (int64_t)(bytes / 16), out);
    return hipGetLastError();
}

}  // namespace aq
