// aq_internal.h -- device layouts and helpers shared by the gfx950 kernels
// of libarm_ai_amd.so.  Not part of the public ABI (include/aq.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace aq {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int TYPE_Q8_0 = 8;
constexpr int TYPE_Q4_K = 12;
constexpr int TYPE_Q6_K = 14;
constexpr int TYPE_Q8_K = 15;

// ---------------------------------------------------------------------------
// Weight layout in HBM.  GGUF blocks arrive array-of-structs (Q4_K 144 B,
// Q6_K 210 B, Q8_0 34 B); Q6_K and Q8_0 blocks are not 16-byte multiples, so
// every type is repacked once at upload into 16-byte aligned planes.  The
// repack is lossless and moves no byte across rows; the planes hold exactly
// the GGUF bytes (algorithmic bytes per block are unchanged):
//   Q4_K: qs   [n][nb][128]  quants (GGUF order)
//         meta [n][nb][16]   f16 d, f16 dmin, u8 scales[12]
//   Q6_K: qs   [n][nb][128]  ql, 16-byte pieces in the order 0,2,1,3,4,6,5,7 so
//                            that the 32 bytes one lane needs are contiguous
//         qh   [n][nb][64]   (GGUF order)
//         meta [n][nb][16]   i8 scales[16]
//         d    [n][nb]       f16
//   Q8_0: qs   [n][k]        i8 quants
//         d    [n][nb]       f16
// ---------------------------------------------------------------------------
struct WPlanes {
    const uint8_t *qs;
    const uint8_t *qh;
    const uint8_t *meta;
    const uint16_t *d;
};

// Quantised activation planes (written by the quantizer kernels):
//   qs    [m][k]      i8
//   d     [m][k/256]  f32 (Q8_K) or [m][k/32] f32 value of the f16 d (Q8_0)
//   d16   [m][k/32]   f16 bits of the Q8_0 d
//   bsums [m][k/16]   i16 (Q8_K)
struct ActPlanes {
    int8_t *qs;
    float *d;
    uint16_t *d16;
    int16_t *bsums;
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Sizes of the activation planes for m rows of k (bytes, each plane 256-B aligned).
struct ActSizes {
    size_t qs, d, d16, bsums, total;
};
inline ActSizes act_sizes(int64_t m, int64_t k) {
    ActSizes s;
    s.qs = align_up((size_t)m * k, 256);
    s.d = align_up((size_t)m * (k / 32) * 4, 256);  // large enough for Q8_K (k/256) and Q8_0 (k/32)
    s.d16 = align_up((size_t)m * (k / 32) * 2, 256);
    s.bsums = align_up((size_t)m * (k / 16) * 2, 256);
    s.total = s.qs + s.d + s.d16 + s.bsums;
    return s;
}
inline ActPlanes act_planes(void *base, int64_t m, int64_t k) {
    ActSizes s = act_sizes(m, k);
    uint8_t *p = (uint8_t *)base;
    ActPlanes a;
    a.qs = (int8_t *)p;
    a.d = (float *)(p + s.qs);
    a.d16 = (uint16_t *)(p + s.qs + s.d);
    a.bsums = (int16_t *)(p + s.qs + s.d + s.d16);
    return a;
}

// ---------------------------------------------------------------------------
// Kernel launchers (defined in k_quantize.hip, k_matvec.hip, k_gemm.hip).
// Each checks the shapes its grid assumes and returns hipErrorInvalidValue
// rather than launching out of bounds.
// ---------------------------------------------------------------------------
hipError_t launch_quantize_q8k(const float *x, int64_t m, int64_t k, ActPlanes a, hipStream_t s);
hipError_t launch_quantize_q8_0(const float *x, int64_t m, int64_t k, ActPlanes a, hipStream_t s);
// GGUF blocks of n rows (device memory) -> the planes of those rows.
hipError_t launch_repack(int type, const uint8_t *src, int64_t n, int64_t k, uint8_t *qs, uint8_t *qh,
                         uint8_t *meta, uint8_t *dp, hipStream_t s);
// Matvec for small m (the decode path); m may be any size, it is cut into
// slices of at most 8 rows.  S/Smin non-null selects the integer-dump epilogue.
hipError_t launch_matvec(int type, const WPlanes &w, int64_t n, int64_t k, const ActPlanes &x,
                         int64_t m, float *y, int32_t *S, int32_t *Smin, hipStream_t s);
// Prefill GEMM on MFMA (m > 8).  Returns hipErrorNotSupported for shapes it
// does not take; the caller then uses launch_matvec.
hipError_t launch_gemm(int type, const WPlanes &w, int64_t n, int64_t k, const ActPlanes &x,
                       int64_t m, float *y, int32_t *S, int32_t *Smin, void *ws, size_t ws_bytes,
                       hipStream_t s);
size_t gemm_workspace_bytes(int type, int64_t m, int64_t n, int64_t k);

}  // namespace aq

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
#ifdef __HIPCC__
namespace aq {

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// DPP lane permutations within a row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

// Sum over groups of 2^LOG consecutive lanes (LOG <= 4); every lane of the
// group gets the group sum.  All 64 lanes must be active.
template <int LOG>
__device__ __forceinline__ int group_sum_i(int v) {
    if (LOG >= 1) v += dpp_i<DPP_QUAD_XOR1>(v);
    if (LOG >= 2) v += dpp_i<DPP_QUAD_XOR2>(v);
    if (LOG >= 3) v += dpp_i<DPP_HALF_MIRROR>(v);
    if (LOG >= 4) v += dpp_i<DPP_ROW_MIRROR>(v);
    return v;
}

// Sum over all 64 lanes; the result is uniform.  All lanes must be active.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<DPP_QUAD_XOR1>(v);
    v += dpp_f<DPP_QUAD_XOR2>(v);
    v += dpp_f<DPP_HALF_MIRROR>(v);
    v += dpp_f<DPP_ROW_MIRROR>(v);
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// f16 -> f32 (exact; v_cvt_f32_f16 with f16 denormals preserved, the HIP
// default mode -- tests cover subnormal d values).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

// IEEE binary32 -> binary16, round to nearest even (the `half` crate's
// from_f32), done on integers so it does not depend on the f16 denormal mode.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u) | (man >> 13));
    int e = (int)exp - 112;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        int shift = 14 - e;
        if (shift > 24) return (uint16_t)sign;
        uint32_t m24 = man | 0x800000u;
        uint32_t r = m24 >> shift;
        uint32_t rem = m24 & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

// Rust `v as i8` for an integral-valued float: saturating, NaN -> 0.
__device__ __forceinline__ int sat_i8(float v) {
    if (v != v) return 0;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int)v;
}

}  // namespace aq
#endif
