// k_quantize.hip -- activation quantizers (Q8_K, Q8_0) and the one-time
// weight repack, for gfx950.
//
// Q8_K follows candle-core 0.8.4 BlockQ8K::from_float (the quantize_row_q8k
// step of k_quants::matmul, reached from native/arm_ai_nif/src/llama_candle.rs:93,
// :119): per 256-element block, the element of largest |x| (first on ties)
// gives iscale = -128/max, q = min(round(iscale*x), 127) with round-half-away,
// bsums are sums of 16 quants, d = 1/iscale.  Q8_0 follows BlockQ8_0::from_float:
// d = amax/127, id = 1/d (0 if d == 0), q = round(x*id), d stored as f16 (RNE).
// Both are bit-exact restatements: IEEE division (no fast-math, no rcp), and
// the (|x|, index) reduction reproduces the sequential first-max rule.
#include "aq_internal.h"

namespace aq {

// One wavefront per 256-element block, four blocks per 256-thread workgroup.
// Lane l holds elements 4l..4l+3.
template <bool VEC>
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float *__restrict__ x, int64_t nblocks,
                                                           int64_t k, ActPlanes a) {
    const int lane = threadIdx.x & 63;
    const int64_t bi = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (bi >= nblocks) return;  // wave-uniform
    const int64_t nb = k / QK_K;
    const int64_t row = bi / nb, sb = bi - row * nb;
    const float *xb = x + row * k + sb * QK_K + 4 * lane;
    float v[4];
    if (VEC) {
        float4 t = *(const float4 *)xb;
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
        for (int i = 0; i < 4; i++) v[i] = xb[i];
    }
    // First index of the largest |x| (candle: `if amax < x.abs()` scanning
    // in order); zeros and NaNs never win.
    float am = 0.0f, mx = 0.0f;
    int idx = 1 << 30;
    for (int i = 0; i < 4; i++) {
        float ax = fabsf(v[i]);
        if (am < ax) {
            am = ax;
            mx = v[i];
            idx = 4 * lane + i;
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        float oam = __shfl_xor(am, off);
        float omx = __shfl_xor(mx, off);
        int oidx = __shfl_xor(idx, off);
        if (oam > am || (oam == am && oidx < idx)) {
            am = oam;
            mx = omx;
            idx = oidx;
        }
    }
    int q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (am != 0.0f) {
        const float iscale = -128.0f / mx;
        for (int i = 0; i < 4; i++) q[i] = sat_i8(fminf(roundf(iscale * v[i]), 127.0f));
        d = 1.0f / iscale;
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s = group_sum_i<2>(s);  // 16 elements = 4 lanes
    uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                      ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    *(uint32_t *)(a.qs + row * k + sb * QK_K + 4 * lane) = packed;
    if ((lane & 3) == 0) a.bsums[row * (k / 16) + sb * 16 + (lane >> 2)] = (int16_t)s;
    if (lane == 0) a.d[row * nb + sb] = d;
}

// Eight lanes per 32-element block, 32 blocks per workgroup.
template <bool VEC>
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x, int64_t nblocks,
                                                            int64_t k, ActPlanes a) {
    const int64_t gb = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    const int sub = threadIdx.x & 7;
    const bool valid = gb < nblocks;
    const int64_t nb = k / QK8_0;
    const int64_t row = valid ? gb / nb : 0, b = valid ? gb - row * nb : 0;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valid) {
        const float *xb = x + row * k + b * QK8_0 + 4 * sub;
        if (VEC) {
            float4 t = *(const float4 *)xb;
            v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
        } else {
            for (int i = 0; i < 4; i++) v[i] = xb[i];
        }
    }
    float am = 0.0f;
    for (int i = 0; i < 4; i++) am = fmaxf(am, fabsf(v[i]));
    am = fmaxf(am, __shfl_xor(am, 1));
    am = fmaxf(am, __shfl_xor(am, 2));
    am = fmaxf(am, __shfl_xor(am, 4));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    if (!valid) return;
    uint32_t packed = 0;
    for (int i = 0; i < 4; i++) packed |= (uint32_t)(sat_i8(roundf(v[i] * id)) & 0xff) << (8 * i);
    *(uint32_t *)(a.qs + row * k + b * QK8_0 + 4 * sub) = packed;
    if (sub == 0) {
        const uint16_t h = f32_to_f16_rne(d);
        a.d16[row * nb + b] = h;
        a.d[row * nb + b] = f16_bits_to_f32(h);
    }
}

hipError_t launch_quantize_q8k(const float *x, int64_t m, int64_t k, ActPlanes a, hipStream_t s) {
    if (!x || m < 0 || k <= 0 || k % QK_K) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    const int64_t nblocks = m * (k / QK_K);
    const int64_t grid = (nblocks + 3) / 4;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) == 0)
        quantize_q8k_kernel<true><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, nblocks, k, a);
    else
        quantize_q8k_kernel<false><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, nblocks, k, a);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float *x, int64_t m, int64_t k, ActPlanes a, hipStream_t s) {
    if (!x || m < 0 || k <= 0 || k % QK8_0) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    const int64_t nblocks = m * (k / QK8_0);
    const int64_t grid = (nblocks + 31) / 32;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) == 0)
        quantize_q8_0_kernel<true><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, nblocks, k, a);
    else
        quantize_q8_0_kernel<false><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, nblocks, k, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Weight repack: GGUF array-of-blocks -> planes (layout in aq_internal.h).
// One thread per byte of a block; grid-stride over all bytes.
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ src, int64_t nblk,
                                                     uint8_t *__restrict__ qs, uint8_t *__restrict__ qh,
                                                     uint8_t *__restrict__ meta, uint8_t *__restrict__ dpl) {
    constexpr int BYTES = TYPE == TYPE_Q4_K ? 144 : TYPE == TYPE_Q6_K ? 210 : 34;
    const int64_t total = nblk * BYTES;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = i / BYTES;
        const int o = (int)(i - b * BYTES);
        if (TYPE == TYPE_Q4_K) {
            // bytes 0..15 -> meta (d, dmin, scales), 16..143 -> qs
            if (o < 16) meta[b * 16 + o] = src[i];
            else qs[b * 128 + (o - 16)] = src[i];
        } else if (TYPE == TYPE_Q6_K) {
            if (o < 128) {
                // destination piece p takes source piece perm[p]
                const int p = o >> 4, w = o & 15;
                const int sp = (p & 4) | ((p & 1) << 1) | ((p >> 1) & 1);  // 0,2,1,3,4,6,5,7
                qs[b * 128 + o] = src[b * BYTES + sp * 16 + w];
            } else if (o < 192) {
                qh[b * 64 + (o - 128)] = src[i];
            } else if (o < 208) {
                meta[b * 16 + (o - 192)] = src[i];
            } else {
                dpl[b * 2 + (o - 208)] = src[i];
            }
        } else {
            if (o < 2) dpl[b * 2 + o] = src[i];
            else qs[b * 32 + (o - 2)] = src[i];
        }
    }
}

hipError_t launch_repack(int type, const uint8_t *src, int64_t n, int64_t k, uint8_t *qs, uint8_t *qh,
                         uint8_t *meta, uint8_t *dp, hipStream_t s) {
    if (!src || n <= 0 || k <= 0) return hipErrorInvalidValue;
    const int blk = type == TYPE_Q8_0 ? QK8_0 : QK_K;
    if (k % blk) return hipErrorInvalidValue;
    const int64_t nblk = n * (k / blk);
    const unsigned grid = 8192;
    switch (type) {
    case TYPE_Q4_K:
        if (!qs || !meta) return hipErrorInvalidValue;
        repack_kernel<TYPE_Q4_K><<<grid, 256, 0, s>>>(src, nblk, qs, qh, meta, dp);
        break;
    case TYPE_Q6_K:
        if (!qs || !qh || !meta || !dp) return hipErrorInvalidValue;
        repack_kernel<TYPE_Q6_K><<<grid, 256, 0, s>>>(src, nblk, qs, qh, meta, dp);
        break;
    case TYPE_Q8_0:
        if (!qs || !dp) return hipErrorInvalidValue;
        repack_kernel<TYPE_Q8_0><<<grid, 256, 0, s>>>(src, nblk, qs, qh, meta, dp);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace aq
