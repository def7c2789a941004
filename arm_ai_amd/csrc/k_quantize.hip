// k_quantize.hip -- activation quantizers (Q8_K, Q8_0) and the one-time
// weight repack into the row-block tile layout, for gfx950.
//
// Q8_K follows candle-core 0.8.4 BlockQ8K::from_float (the quantize_row_q8k
// step of k_quants::matmul, reached from native/arm_ai_nif/src/llama_candle.rs:93,
// :119); Q8_0 follows BlockQ8_0::from_float.  The per-block arithmetic lives in
// q8k_block_wave / q8_0_block_8lanes (aq_internal.h), which the fused matvec
// prologue calls too, so both paths produce the same bytes.
#include "aq_internal.h"

namespace aq {

// One wavefront per 256-element block, lane l holding elements 4l..4l+3
// (q8k_block_wave, the fused prologues' code): four blocks per 256-thread
// workgroup.  The block's row and index within the row are wave-uniform
// (scalar arithmetic).
template <bool VEC>
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float *__restrict__ x, int64_t nblocks,
                                                           int64_t k, ActPlanes a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t bi = (int64_t)blockIdx.x * 4 + wave;
    if (bi >= nblocks) return;  // uniform over the wavefront
    const int64_t nb = k / QK_K;
    const int64_t row = bi / nb, sb = bi - row * nb;
    const int64_t e0 = row * k + sb * QK_K + 4 * lane;
    float v[4];
    if (VEC) {
        const float4 t = *(const float4 *)(x + e0);
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = x[e0 + i];
    }
    int bsum;
    float d;
    const uint32_t packed = q8k_block_wave(v, lane, &bsum, &d);
    store_q8k_block64(a, row, k, sb, lane, packed, bsum, d);
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
            const float4 t = *(const float4 *)xb;
            v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
        } else {
            for (int i = 0; i < 4; i++) v[i] = xb[i];
        }
    }
    uint16_t h;
    const uint32_t packed = q8_0_block_8lanes(v, &h);
    if (!valid) return;
    *(uint32_t *)(a.qs + row * k + b * QK8_0 + 4 * sub) = packed;
    if (sub == 0) {
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
// Weight repack: GGUF array-of-blocks -> row-block tiles (aq_internal.h).
// One thread per source byte; grid-stride over all bytes of the n rows.
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ src, int64_t n, int64_t nblk,
                                                     int ng, uint8_t *__restrict__ slab, uint16_t *__restrict__ dpl) {
    constexpr int BYTES = TYPE == TYPE_Q4_K ? 144 : TYPE == TYPE_Q5_K ? 176 : TYPE == TYPE_Q6_K ? 210
                        : TYPE == TYPE_Q4_0 ? 18 : TYPE == TYPE_Q2_K ? 84 : TYPE == TYPE_Q3_K ? 110
                        : TYPE == TYPE_Q5_0 ? 22 : 34;
    constexpr int S = slabs_of(TYPE);
    const int64_t rb_stride = (int64_t)ng * S * 128;
    const int64_t total = n * nblk * BYTES;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t blk = i / BYTES;  // block index over all rows
        const int o = (int)(i - blk * BYTES);
        const int64_t row = blk / nblk, b = blk - row * nblk;
        uint8_t *rbp = slab + (row >> 3) * rb_stride + (row & 7) * 16;  // + (g * S + piece) * 128 + byte
        if (TYPE == TYPE_Q4_K) {
            // bytes 0..15 (d, dmin, scales) -> piece 0; qs byte j -> piece 1 + j/16
            const int piece = o < 16 ? 0 : 1 + (o - 16) / 16;
            const int w = o < 16 ? o : (o - 16) & 15;
            rbp[(b * S + piece) * 128 + w] = src[i];
        } else if (TYPE == TYPE_Q4_0) {
            // Q4_0 block b = 8g + j: d -> piece 8 bytes 2j..2j+1; qs byte q -> piece j byte q
            const int64_t g = b >> 3;
            const int j = (int)(b & 7);
            if (o < 2) rbp[(g * S + 8) * 128 + 2 * j + o] = src[i];
            else rbp[(g * S + j) * 128 + (o - 2)] = src[i];
        } else if (TYPE == TYPE_Q5_0) {
            // Q5_0 block b = 8g + j: d -> piece 10 bytes 2j..2j+1; qh -> piece 8 + j/4 bytes 4(j%4)..;
            // qs byte q -> piece j byte q
            const int64_t g = b >> 3;
            const int j = (int)(b & 7);
            if (o < 2) rbp[(g * S + 10) * 128 + 2 * j + o] = src[i];
            else if (o < 6) rbp[(g * S + 8 + (j >> 2)) * 128 + 4 * (j & 3) + (o - 2)] = src[i];
            else rbp[(g * S + j) * 128 + (o - 6)] = src[i];
        } else if (TYPE == TYPE_Q2_K) {
            // scales 0..15 -> piece 0, qs 16..79 -> pieces 1..4, d / dmin 80..83 -> the plane's 32-bit entry
            if (o < 80) rbp[(b * S + (o >> 4)) * 128 + (o & 15)] = src[i];
            else ((uint8_t *)(dpl + (((row >> 3) * ng + b) * 8 + (row & 7)) * 2))[o - 80] = src[i];
        } else if (TYPE == TYPE_Q5_K || TYPE == TYPE_Q3_K) {
            // the block's bytes are its pieces in order: byte o -> piece o / 16
            rbp[(b * S + (o >> 4)) * 128 + (o & 15)] = src[i];
        } else if (TYPE == TYPE_Q6_K) {
            if (o < 208) {
                // ql 0..127 -> pieces 0..7, qh 128..191 -> 8..11, scales 192..207 -> 12
                rbp[(b * S + (o >> 4)) * 128 + (o & 15)] = src[i];
            } else {
                ((uint8_t *)(dpl + ((row >> 3) * ng + b) * 8 + (row & 7)))[o - 208] = src[i];
            }
        } else {
            // Q8_0 block b = 8g + j: d -> piece 16 bytes 2j..2j+1; qs byte q -> piece 2j + q/16
            const int64_t g = b >> 3;
            const int j = (int)(b & 7);
            if (o < 2) rbp[(g * S + 16) * 128 + 2 * j + o] = src[i];
            else {
                const int q = o - 2;
                rbp[(g * S + 2 * j + (q >> 4)) * 128 + (q & 15)] = src[i];
            }
        }
    }
}

// Q4_0 / Q5_0 -> Q8_0 tiles: one thread per source byte.  Block b = 8g + j
// of a row: d -> piece 16 bytes 2j, 2j+1; qs byte t (elements t and t + 16)
// -> piece 2j byte t and piece 2j + 1 byte t, the values q - 8 (Q4_0) or,
// with bits t and t + 16 of qh as the fifth bits, q - 16 (Q5_0).
template <int TYPE>
__global__ __launch_bounds__(256) void expand_q80_kernel(const uint8_t *__restrict__ src, int64_t n, int64_t nblk,
                                                         int ng, uint8_t *__restrict__ slab) {
    constexpr int S = slabs_of(TYPE_Q8_0);
    constexpr int BYTES = TYPE == TYPE_Q5_0 ? 22 : 18, QS = TYPE == TYPE_Q5_0 ? 6 : 2;
    const int64_t rb_stride = (int64_t)ng * S * 128;
    const int64_t total = n * nblk * BYTES;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t blk = i / BYTES;
        const int o = (int)(i - blk * BYTES);
        const int64_t row = blk / nblk, b = blk - row * nblk;
        uint8_t *rbp = slab + (row >> 3) * rb_stride + (row & 7) * 16;
        const int64_t g = b >> 3;
        const int j = (int)(b & 7);
        const uint8_t v = src[i];
        if (o < 2) {
            rbp[(g * S + 16) * 128 + 2 * j + o] = v;
        } else if (o >= QS) {
            const int t = o - QS;
            int lo = v & 15, hi = v >> 4;
            if (TYPE == TYPE_Q5_0) {
                const uint8_t *qh = src + blk * BYTES + 2;
                const uint32_t h = (uint32_t)qh[0] | ((uint32_t)qh[1] << 8) | ((uint32_t)qh[2] << 16) | ((uint32_t)qh[3] << 24);
                lo = (lo | (((h >> t) & 1) << 4)) - 16;
                hi = (hi | (((h >> (t + 16)) & 1) << 4)) - 16;
            } else {
                lo -= 8;
                hi -= 8;
            }
            rbp[(g * S + 2 * j) * 128 + t] = (uint8_t)(int8_t)lo;
            rbp[(g * S + 2 * j + 1) * 128 + t] = (uint8_t)(int8_t)hi;
        }
    }
}

hipError_t launch_expand_q80(int type, const uint8_t *src, int64_t n, int64_t k, uint8_t *dst_slab, hipStream_t s) {
    if (!src || !dst_slab || n <= 0 || k <= 0 || k % QK8_0) return hipErrorInvalidValue;
    if (type != TYPE_Q4_0 && type != TYPE_Q5_0) return hipErrorInvalidValue;
    const int64_t nblk = k / QK8_0;
    const int ng = groups_of(type, k);
    const int64_t total = n * nblk * (type == TYPE_Q5_0 ? 22 : 18);
    const int64_t blocks = (total + 255) / 256, grid = blocks < 65536 ? blocks : 65536;
    if (type == TYPE_Q5_0) expand_q80_kernel<TYPE_Q5_0><<<(unsigned)grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab);
    else expand_q80_kernel<TYPE_Q4_0><<<(unsigned)grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab);
    return hipGetLastError();
}

hipError_t launch_repack(int type, const uint8_t *src, int64_t n, int64_t k, uint8_t *dst_slab, uint16_t *dst_d,
                         hipStream_t s) {
    if (!src || !dst_slab || n <= 0 || k <= 0) return hipErrorInvalidValue;
    const int blk = act_q80(type) ? QK8_0 : QK_K;
    if (k % blk) return hipErrorInvalidValue;
    const int64_t nblk = k / blk;
    const int ng = groups_of(type, k);
    const unsigned grid = 8192;
    switch (type) {
    case TYPE_Q4_K: repack_kernel<TYPE_Q4_K><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d); break;
    case TYPE_Q5_K: repack_kernel<TYPE_Q5_K><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d); break;
    case TYPE_Q6_K:
        if (!dst_d) return hipErrorInvalidValue;
        repack_kernel<TYPE_Q6_K><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d);
        break;
    case TYPE_Q8_0: repack_kernel<TYPE_Q8_0><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d); break;
    case TYPE_Q4_0: repack_kernel<TYPE_Q4_0><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d); break;
    case TYPE_Q2_K:
        if (!dst_d) return hipErrorInvalidValue;
        repack_kernel<TYPE_Q2_K><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d);
        break;
    case TYPE_Q3_K: repack_kernel<TYPE_Q3_K><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d); break;
    case TYPE_Q5_0: repack_kernel<TYPE_Q5_0><<<grid, 256, 0, s>>>(src, n, nblk, ng, dst_slab, dst_d); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace aq
