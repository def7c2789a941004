/*
 * oracle.c -- CPU restatement of candle-core 0.8.4's quantized matmul
 * (the arithmetic behind native/arm_ai_nif/src/llama_candle.rs:93 and
 * :119).  TEST INFRASTRUCTURE ONLY: the parity checker for tests/ and
 * smoke(), and the CPU "port" baseline timed by bench.py.  The product
 * library never links this file.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, x86-64 baseline ISA,
 * OpenMP).  No fast-math and no FMA contraction: every f32 operation below
 * is one IEEE operation in the order candle's generic `vec_dot_unopt`
 * performs it (Rust does not contract a*b+c).
 *
 * Pinning (what checks each function; tests/test_oracle.py):
 *  - f16 conversions: numpy float16 (IEEE RNE) over all 65536 half values
 *    and a dense f32 sweep.
 *  - quantize_row_q8k: closed-form known answers (ties-away rounding case
 *    2.5 -> 3, first-max tie break, clamp of +128 -> 127, all-zero block),
 *    invariants (bsums, first max maps to -128, |d*q - x| <= |d|/2).
 *  - quantize_row_q8_0: known answers and invariants; d stored as f16 RNE.
 *  - vec_dot_*: f64 dequantize-then-dot computed from the generator's
 *    unpacked element arrays (not from this file's unpacking), and the
 *    integer block sums compared bit-exactly against sums built from the
 *    same unpacked arrays; Q6_K bit layout also against a restatement of
 *    the reference's own dequantize_q6_k (shape_ops.rs:2848-2899) on blocks
 *    where its sub-scale indexing quirk cannot matter.
 *  - Q4_0 (GGML block_q4_0, restated): hand-built blocks whose single
 *    nibble must land on element j or j + 16 with value q - 8.
 *  - Q5_K (GGML block_q5_K, restated; the reference holds no source for
 *    it): hand-built blocks whose single qh bit or nibble must land on the
 *    element dequantize_row_q5_K assigns it, and the unit-scale case.
 *  - Q5_0 (GGML block_q5_0, restated): hand-built blocks whose single qh
 *    bit or nibble must land on element j or j + 16 with value q - 16.
 *  - Q2_K and Q3_K (GGML block_q2_K / block_q3_K, restated; no source for
 *    them in the reference): hand-built blocks whose single 2-bit quant,
 *    hmask bit or scale must land on the element and sub-block
 *    dequantize_row_q2_K / q3_K assign it, closed-form sums of uniform
 *    blocks, and the f64 dequantize-then-dot of the generator's arrays.
 *  - the f32 combine order (candle vec_dot_unopt) is pinned only by the
 *    candle source, which is not in this image: "parity unpinned" for the
 *    exact f32 rounding sequence; the value is pinned to f64 truth.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- f16 */

/* half::f16::to_f32 (exact widening).  The reference uses the `half`
 * crate for f16<->f32 (shape_ops.rs:1492-1503). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: normalise */
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* half::f16::from_f32: round to nearest, ties to even; overflow -> inf;
 * NaN keeps its top mantissa bits with the quiet bit set. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        uint32_t nan_bit = man ? 0x200u : 0u;
        return (uint16_t)(sign | 0x7c00u | nan_bit | (man >> 13));
    }
    int32_t e = (int32_t)exp - 112; /* f16 biased exponent */
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* f16 subnormal (or zero): mantissa = man24 >> (14 - e) */
        int32_t shift = 14 - e;
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

/* ------------------------------------------------------------- helpers */

static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd_u32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float rd_f32(const uint8_t *p) {
    float f;
    memcpy(&f, p, 4);
    return f;
}
static inline int16_t rd_i16(const uint8_t *p) { return (int16_t)rd_u16(p); }

/* Rust `f as i8`: saturating, NaN -> 0. */
static inline int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

size_t orc_type_block_bytes(int type) {
    switch (type) {
    case ORC_Q2_K: return ORC_Q2K_BYTES;
    case ORC_Q3_K: return ORC_Q3K_BYTES;
    case ORC_Q4_K: return ORC_Q4K_BYTES;
    case ORC_Q5_K: return ORC_Q5K_BYTES;
    case ORC_Q6_K: return ORC_Q6K_BYTES;
    case ORC_Q8_0: return ORC_Q8_0_BYTES;
    case ORC_Q4_0: return ORC_Q4_0_BYTES;
    case ORC_Q5_0: return ORC_Q5_0_BYTES;
    case ORC_Q8_K: return ORC_Q8K_BYTES;
    default: return 0;
    }
}

int64_t orc_type_block_elems(int type) {
    switch (type) {
    case ORC_Q2_K:
    case ORC_Q3_K:
    case ORC_Q4_K:
    case ORC_Q5_K:
    case ORC_Q6_K:
    case ORC_Q8_K: return ORC_QK_K;
    case ORC_Q8_0:
    case ORC_Q4_0:
    case ORC_Q5_0: return ORC_QK8_0;
    default: return 0;
    }
}

/* ------------------------------------------------------- quantizers */

/* BlockQ8K::from_float (candle k_quants.rs, quantize_row_q8k).
 * Per 256-block: max = the element of largest |x|, the FIRST one on ties
 * (strict `amax < |x|`).  amax == 0 -> d = 0, qs = 0, bsums = 0.  Else
 * iscale = -128/max, qs = min(round(iscale*x), 127) (round = ties away
 * from zero, Rust f32::round), bsums[g] = sum of qs[16g..16g+16] as i16,
 * d = 1/iscale. */
int orc_quantize_row_q8k(const float *x, int64_t k, uint8_t *out) {
    if (k % ORC_QK_K != 0) return -1;
    int64_t nb = k / ORC_QK_K;
    for (int64_t b = 0; b < nb; b++) {
        const float *xb = x + b * ORC_QK_K;
        uint8_t *y = out + b * ORC_Q8K_BYTES;
        int8_t *qs = (int8_t *)(y + 4);
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < ORC_QK_K; j++) {
            float ax = fabsf(xb[j]);
            if (amax < ax) {
                amax = ax;
                max = xb[j];
            }
        }
        float d = 0.0f;
        int16_t bsums[16];
        if (amax == 0.0f) {
            memset(qs, 0, ORC_QK_K);
            memset(bsums, 0, sizeof bsums);
        } else {
            float iscale = -128.0f / max;
            for (int j = 0; j < ORC_QK_K; j++) {
                float v = roundf(iscale * xb[j]);
                qs[j] = sat_i8(fminf(v, 127.0f));
            }
            for (int g = 0; g < 16; g++) {
                int32_t s = 0;
                for (int i = 0; i < 16; i++) s += qs[16 * g + i];
                bsums[g] = (int16_t)s;
            }
            d = 1.0f / iscale;
        }
        memcpy(y, &d, 4);
        memcpy(y + 260, bsums, 32);
    }
    return 0;
}

/* BlockQ8_0::from_float (quantize_row_q8_0): per 32-block
 * amax = max |x| (f32::max), d = amax/127, id = d != 0 ? 1/d : 0,
 * stored d = f16::from_f32(d) (RNE), qs = round(x*id) as i8 with the
 * UNROUNDED f32 id. */
int orc_quantize_row_q8_0(const float *x, int64_t k, uint8_t *out) {
    if (k % ORC_QK8_0 != 0) return -1;
    int64_t nb = k / ORC_QK8_0;
    for (int64_t b = 0; b < nb; b++) {
        const float *xb = x + b * ORC_QK8_0;
        uint8_t *y = out + b * ORC_Q8_0_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK8_0; j++) amax = fmaxf(amax, fabsf(xb[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = orc_f32_to_f16(d);
        y[0] = (uint8_t)(dh & 0xff);
        y[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < ORC_QK8_0; j++) y[2 + j] = (uint8_t)sat_i8(roundf(xb[j] * id));
    }
    return 0;
}

/* ----------------------------------------------------- Q4_K unpack */

/* candle's 6-bit scale/min extraction (the utmp / KMASK form of GGML's
 * get_scale_min_k4), restated. */
static void q4k_scales_mins(const uint8_t *sc12, uint8_t scales[8], uint8_t mins[8]) {
    const uint32_t KMASK1 = 0x3f3f3f3fu, KMASK2 = 0x0f0f0f0fu, KMASK3 = 0x03030303u;
    uint32_t utmp[4];
    utmp[0] = rd_u32(sc12);
    utmp[1] = rd_u32(sc12 + 4);
    utmp[2] = rd_u32(sc12 + 8);
    utmp[3] = ((utmp[2] >> 4) & KMASK2) | (((utmp[1] >> 6) & KMASK3) << 4);
    uint32_t uaux = utmp[1] & KMASK1;
    utmp[1] = (utmp[2] & KMASK2) | (((utmp[0] >> 6) & KMASK3) << 4);
    utmp[2] = uaux;
    utmp[0] &= KMASK1;
    for (int i = 0; i < 4; i++) {
        scales[i] = (uint8_t)(utmp[0] >> (8 * i));
        scales[4 + i] = (uint8_t)(utmp[1] >> (8 * i));
        mins[i] = (uint8_t)(utmp[2] >> (8 * i));
        mins[4 + i] = (uint8_t)(utmp[3] >> (8 * i));
    }
}

/* Element order of a Q4_K block: for chunk c<4, l<32:
 * e = 64c+l -> qs[32c+l] & 0xF, e = 64c+32+l -> qs[32c+l] >> 4. */
static void q4k_unpack(const uint8_t *qs, int8_t aux8[256]) {
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            aux8[64 * c + l] = (int8_t)(qs[32 * c + l] & 0xF);
            aux8[64 * c + 32 + l] = (int8_t)(qs[32 * c + l] >> 4);
        }
}

/* Q5_K (GGML block_q5_K; candle BlockQ5K): the Q4_K nibbles plus a fifth
 * bit, bit s of qh[l] for element 32s + l (sub-block s):
 *   element 64c + l      = (qs[32c+l] & 0xF) + 16 * (qh[l] >> 2c & 1)
 *   element 64c + 32 + l = (qs[32c+l] >> 4)  + 16 * (qh[l] >> (2c+1) & 1) */
static void q5k_unpack(const uint8_t *qh, const uint8_t *qs, int8_t aux8[256]) {
    q4k_unpack(qs, aux8);
    for (int s = 0; s < 8; s++)
        for (int l = 0; l < 32; l++) aux8[32 * s + l] = (int8_t)(aux8[32 * s + l] + 16 * ((qh[l] >> s) & 1));
}

/* Q6_K element order (h<2, l<32; QL = ql+64h, QH = qh+32h, base 128h):
 * e = base+l    : (QL[l]    & 0xF) | ((QH[l] >> 0 & 3) << 4)
 * e = base+32+l : (QL[l+32] & 0xF) | ((QH[l] >> 2 & 3) << 4)
 * e = base+64+l : (QL[l]    >> 4)  | ((QH[l] >> 4 & 3) << 4)
 * e = base+96+l : (QL[l+32] >> 4)  | ((QH[l] >> 6 & 3) << 4)
 * each minus 32.  Same bit mapping as shape_ops.rs:2868-2882. */
static void q6k_unpack(const uint8_t *ql, const uint8_t *qh, int8_t aux8[256]) {
    for (int h = 0; h < 2; h++) {
        const uint8_t *QL = ql + 64 * h;
        const uint8_t *QH = qh + 32 * h;
        int8_t *a = aux8 + 128 * h;
        for (int l = 0; l < 32; l++) {
            a[l] = (int8_t)(((QL[l] & 0xF) | (((QH[l] >> 0) & 3) << 4)) - 32);
            a[l + 32] = (int8_t)(((QL[l + 32] & 0xF) | (((QH[l] >> 2) & 3) << 4)) - 32);
            a[l + 64] = (int8_t)(((QL[l] >> 4) | (((QH[l] >> 4) & 3) << 4)) - 32);
            a[l + 96] = (int8_t)(((QL[l + 32] >> 4) | (((QH[l] >> 6) & 3) << 4)) - 32);
        }
    }
}

/* Q2_K (GGML block_q2_K: scales[16] @0, qs[64] @16, f16 d @80, f16 dmin
 * @82; candle BlockQ2K).  For half hf < 2, shift j < 4, l < 32:
 *   element 128hf + 32j + l = (qs[32hf + l] >> 2j) & 3,
 * in 16-element group 8hf + 2j + l/16, whose scales byte holds the scale
 * (low nibble) and the min (high nibble). */
static void q2k_unpack(const uint8_t *qs, int8_t aux8[256]) {
    for (int hf = 0; hf < 2; hf++)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) aux8[128 * hf + 32 * j + l] = (int8_t)((qs[32 * hf + l] >> (2 * j)) & 3);
}

/* Q3_K (GGML block_q3_K: hmask[32] @0, qs[64] @32, scales[12] @96, f16 d
 * @108; candle BlockQ3K).  For half hf < 2, shift j < 4, l < 32:
 *   element 128hf + 32j + l = ((qs[32hf + l] >> 2j) & 3) - (hmask[l] bit (4hf + j) ? 0 : 4),
 * 16-element group g = e/16 with the 6-bit scale of candle's auxs form
 * (low nibbles of bytes 0..7, then their high nibbles, each with two bits
 * of bytes 8..11 on top), used as scale - 32. */
static void q3k_unpack(const uint8_t *hm, const uint8_t *qs, int8_t aux8[256]) {
    for (int hf = 0; hf < 2; hf++)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) {
                const int q = (qs[32 * hf + l] >> (2 * j)) & 3;
                const int h = (hm[l] >> (4 * hf + j)) & 1;
                aux8[128 * hf + 32 * j + l] = (int8_t)(q - (h ? 0 : 4));
            }
}

static void q3k_scales(const uint8_t *sc12, int8_t scales[16]) {
    const uint32_t KMASK1 = 0x03030303u, KMASK2 = 0x0f0f0f0fu;
    uint32_t a[4];
    a[0] = rd_u32(sc12);
    a[1] = rd_u32(sc12 + 4);
    const uint32_t tmp = rd_u32(sc12 + 8);
    a[2] = ((a[0] >> 4) & KMASK2) | (((tmp >> 4) & KMASK1) << 4);
    a[3] = ((a[1] >> 4) & KMASK2) | (((tmp >> 6) & KMASK1) << 4);
    a[0] = (a[0] & KMASK2) | ((tmp & KMASK1) << 4);
    a[1] = (a[1] & KMASK2) | (((tmp >> 2) & KMASK1) << 4);
    for (int i = 0; i < 16; i++) scales[i] = (int8_t)((int)((a[i / 4] >> (8 * (i % 4))) & 0xffu) - 32);
}

/* --------------------------------------------------------- vec dots */

/* BlockQ4K::vec_dot_unopt (vec_dot_q4k_q8k), candle's generic order:
 * per block, 8 i32 lane sums aux32[l] += scale * (q8*q4) over groups of 8;
 * sums[l] += (f16(d_w)*d_x) * aux32[l]; sumf -= (f16(dmin_w)*d_x) * sumi
 * with sumi = sum_{j<16} bsums[j]*mins[j/2]; return sumf + sum(sums). */
static float q45k_vec_dot(int five, int64_t k, const uint8_t *w, const uint8_t *xq) {
    int64_t nb = k / ORC_QK_K;
    int8_t aux8[256];
    float sums[8] = {0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *x = w + b * (five ? ORC_Q5K_BYTES : ORC_Q4K_BYTES);
        const uint8_t *y = xq + b * ORC_Q8K_BYTES;
        const int8_t *q8 = (const int8_t *)(y + 4);
        int32_t aux32[8] = {0};
        if (five)
            q5k_unpack(x + 16, x + 48, aux8);
        else
            q4k_unpack(x + 16, aux8);
        uint8_t scales[8], mins[8];
        q4k_scales_mins(x + 4, scales, mins);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)rd_i16(y + 260 + 2 * j) * (int32_t)mins[j / 2];
        const int8_t *a = aux8;
        for (int s = 0; s < 8; s++) {
            int32_t scale = scales[s];
            for (int g = 0; g < 4; g++) {
                for (int l = 0; l < 8; l++) {
                    int16_t aux16 = (int16_t)(q8[l] * a[l]);
                    aux32[l] += scale * (int32_t)aux16;
                }
                q8 += 8;
                a += 8;
            }
        }
        float yd = rd_f32(y);
        float d = orc_f16_to_f32(rd_u16(x)) * yd;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = orc_f16_to_f32(rd_u16(x + 2)) * yd;
        sumf -= dmin * (float)sumi;
    }
    float t = 0.0f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return sumf + t;
}

float orc_vec_dot_q4k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq) { return q45k_vec_dot(0, k, w, xq); }

/* BlockQ2K::vec_dot_unopt (vec_dot_q2k_q8k): per block
 * summs = sum_g bsums[g] * (scales[g] >> 4), isum = sum_g (scales[g] & 15) *
 * sum_{e in g} q8 * q2 (i32), sumf += (d_x * f16(d_w)) * isum - (d_x *
 * f16(dmin_w)) * summs. */
float orc_vec_dot_q2k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq) {
    int64_t nb = k / ORC_QK_K;
    int8_t aux8[256];
    float sumf = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *x = w + b * ORC_Q2K_BYTES;
        const uint8_t *y = xq + b * ORC_Q8K_BYTES;
        const int8_t *q8 = (const int8_t *)(y + 4);
        int32_t summs = 0, isum = 0;
        for (int g = 0; g < 16; g++) summs += (int32_t)rd_i16(y + 260 + 2 * g) * (int32_t)(x[g] >> 4);
        q2k_unpack(x + 16, aux8);
        for (int g = 0; g < 16; g++) {
            int32_t isuml = 0;
            for (int e = 16 * g; e < 16 * g + 16; e++) isuml += (int32_t)q8[e] * aux8[e];
            isum += (int32_t)(x[g] & 0xF) * isuml;
        }
        const float yd = rd_f32(y);
        const float dall = yd * orc_f16_to_f32(rd_u16(x + 80));
        const float dmin = yd * orc_f16_to_f32(rd_u16(x + 82));
        sumf += dall * (float)isum - dmin * (float)summs;
    }
    return sumf;
}

/* BlockQ3K::vec_dot_unopt (vec_dot_q3k_q8k): the 8-lane order of Q4_K's,
 * aux32[l] += (scale_g - 32) * (q8 * q3) per half group of 8, sums[l] +=
 * (f16(d_w) * d_x) * aux32[l]; return sum(sums). */
float orc_vec_dot_q3k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq) {
    int64_t nb = k / ORC_QK_K;
    int8_t aux8[256], sc[16];
    float sums[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *x = w + b * ORC_Q3K_BYTES;
        const uint8_t *y = xq + b * ORC_Q8K_BYTES;
        const int8_t *q8 = (const int8_t *)(y + 4);
        int32_t aux32[8] = {0};
        q3k_unpack(x, x + 32, aux8);
        q3k_scales(x + 96, sc);
        for (int g = 0; g < 16; g++)
            for (int hh = 0; hh < 2; hh++)
                for (int l = 0; l < 8; l++) {
                    const int e = 16 * g + 8 * hh + l;
                    int16_t aux16 = (int16_t)(q8[e] * aux8[e]);
                    aux32[l] += (int32_t)sc[g] * (int32_t)aux16;
                }
        const float d = orc_f16_to_f32(rd_u16(x + 108)) * rd_f32(y);
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
    }
    float t = 0.0f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return t;
}

/* BlockQ5K::vec_dot_unopt (vec_dot_q5k_q8k): the same order as Q4_K's with
 * the 5-bit quants of q5k_unpack (|q8*q5| <= 3968 still fits the i16 aux16). */
float orc_vec_dot_q5k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq) { return q45k_vec_dot(1, k, w, xq); }

/* BlockQ6K::vec_dot_unopt (vec_dot_q6k_q8k): per 16-element sub-block j,
 * two 8-lane halves, aux32[l] += (f32)scale_j * (f32)(q8*q6) kept in f32
 * (exact: |aux32| < 2^24 for any input), sums[l] += aux32[l] * (f16(d_w)*d_x);
 * return sum(sums). */
float orc_vec_dot_q6k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq) {
    int64_t nb = k / ORC_QK_K;
    int8_t aux8[256];
    float sums[8] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *x = w + b * ORC_Q6K_BYTES;
        const uint8_t *y = xq + b * ORC_Q8K_BYTES;
        const int8_t *q8 = (const int8_t *)(y + 4);
        const int8_t *sc = (const int8_t *)(x + 192);
        float aux32[8] = {0};
        q6k_unpack(x, x + 128, aux8);
        for (int j = 0; j < 16; j++) {
            float scale = (float)sc[j];
            for (int hh = 0; hh < 2; hh++) {
                const int8_t *q = q8 + 16 * j + 8 * hh;
                const int8_t *a = aux8 + 16 * j + 8 * hh;
                for (int l = 0; l < 8; l++) {
                    int16_t aux16 = (int16_t)(q[l] * a[l]);
                    aux32[l] += scale * (float)aux16;
                }
            }
        }
        float d = orc_f16_to_f32(rd_u16(x + 208)) * rd_f32(y);
        for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
    }
    float t = 0.0f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return t;
}

/* BlockQ8_0::vec_dot_unopt: sumf += (f32)(sum_i qw*qx) * f16(d_w) * f16(d_x). */
float orc_vec_dot_q8_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *xq) {
    int64_t nb = k / ORC_QK8_0;
    float sumf = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *x = w + b * ORC_Q8_0_BYTES;
        const uint8_t *y = xq + b * ORC_Q8_0_BYTES;
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)x[2 + j] * (int32_t)(int8_t)y[2 + j];
        sumf += (float)s * orc_f16_to_f32(rd_u16(x)) * orc_f16_to_f32(rd_u16(y));
    }
    return sumf;
}

/* BlockQ4_0::vec_dot_unopt (Q4_0 . Q8_0): per 32-block
 * sum_i = sum_{j<16} ((qs[j] & 15) - 8) * qx[j] + ((qs[j] >> 4) - 8) * qx[j+16]
 * (i32), sumf += (f32)sum_i * f16(d_w) * f16(d_x). */
float orc_vec_dot_q4_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *xq) {
    int64_t nb = k / ORC_QK8_0;
    float sumf = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *x = w + b * ORC_Q4_0_BYTES;
        const uint8_t *y = xq + b * ORC_Q8_0_BYTES;
        int32_t s = 0;
        for (int j = 0; j < 16; j++) {
            const int32_t v0 = (int32_t)(x[2 + j] & 0x0F) - 8, v1 = (int32_t)(x[2 + j] >> 4) - 8;
            s += v0 * (int32_t)(int8_t)y[2 + j] + v1 * (int32_t)(int8_t)y[2 + 16 + j];
        }
        sumf += (float)s * orc_f16_to_f32(rd_u16(x)) * orc_f16_to_f32(rd_u16(y));
    }
    return sumf;
}

/* Q5_0 (GGML block_q5_0: f16 d @0, u32 qh @2, qs[16] @6; candle BlockQ5_0):
 * element j < 16 = (qs[j] & 15) | (qh >> j & 1) << 4, element j + 16 =
 * (qs[j] >> 4) | (qh >> (j + 16) & 1) << 4, each minus 16. */
static int32_t q5_0_block_sum(const uint8_t *x, const uint8_t *y) {
    const uint32_t qh = rd_u32(x + 2);
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        const int32_t v0 = (int32_t)((x[6 + j] & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
        const int32_t v1 = (int32_t)((x[6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
        s += v0 * (int32_t)(int8_t)y[2 + j] + v1 * (int32_t)(int8_t)y[2 + 16 + j];
    }
    return s;
}

/* BlockQ5_0::vec_dot_unopt (Q5_0 . Q8_0): sumf += (f32)sum_i * f16(d_w) * f16(d_x). */
float orc_vec_dot_q5_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *xq) {
    int64_t nb = k / ORC_QK8_0;
    float sumf = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *x = w + b * ORC_Q5_0_BYTES;
        const uint8_t *y = xq + b * ORC_Q8_0_BYTES;
        sumf += (float)q5_0_block_sum(x, y) * orc_f16_to_f32(rd_u16(x)) * orc_f16_to_f32(rd_u16(y));
    }
    return sumf;
}

void orc_block_sums(int type, int64_t k, const uint8_t *w, const uint8_t *xq, int32_t *S,
                    int32_t *Smin) {
    int8_t aux8[256];
    if (type == ORC_Q4_K || type == ORC_Q5_K) {
        const int five = type == ORC_Q5_K;
        int64_t nb = k / ORC_QK_K;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *x = w + b * (five ? ORC_Q5K_BYTES : ORC_Q4K_BYTES);
            const uint8_t *y = xq + b * ORC_Q8K_BYTES;
            const int8_t *q8 = (const int8_t *)(y + 4);
            uint8_t scales[8], mins[8];
            q4k_scales_mins(x + 4, scales, mins);
            if (five)
                q5k_unpack(x + 16, x + 48, aux8);
            else
                q4k_unpack(x + 16, aux8);
            int32_t s = 0, sm = 0;
            for (int j = 0; j < 8; j++) {
                int32_t isum = 0;
                for (int e = 32 * j; e < 32 * j + 32; e++) isum += (int32_t)q8[e] * aux8[e];
                s += (int32_t)scales[j] * isum;
            }
            for (int g = 0; g < 16; g++) sm += (int32_t)rd_i16(y + 260 + 2 * g) * (int32_t)mins[g / 2];
            S[b] = s;
            if (Smin) Smin[b] = sm;
        }
    } else if (type == ORC_Q2_K) {
        int64_t nb = k / ORC_QK_K;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *x = w + b * ORC_Q2K_BYTES;
            const uint8_t *y = xq + b * ORC_Q8K_BYTES;
            const int8_t *q8 = (const int8_t *)(y + 4);
            q2k_unpack(x + 16, aux8);
            int32_t s = 0, sm = 0;
            for (int g = 0; g < 16; g++) {
                int32_t isum = 0;
                for (int e = 16 * g; e < 16 * g + 16; e++) isum += (int32_t)q8[e] * aux8[e];
                s += (int32_t)(x[g] & 0xF) * isum;
                sm += (int32_t)rd_i16(y + 260 + 2 * g) * (int32_t)(x[g] >> 4);
            }
            S[b] = s;
            if (Smin) Smin[b] = sm;
        }
    } else if (type == ORC_Q3_K) {
        int64_t nb = k / ORC_QK_K;
        int8_t sc[16];
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *x = w + b * ORC_Q3K_BYTES;
            const uint8_t *y = xq + b * ORC_Q8K_BYTES;
            const int8_t *q8 = (const int8_t *)(y + 4);
            q3k_unpack(x, x + 32, aux8);
            q3k_scales(x + 96, sc);
            int32_t s = 0;
            for (int g = 0; g < 16; g++) {
                int32_t isum = 0;
                for (int e = 16 * g; e < 16 * g + 16; e++) isum += (int32_t)q8[e] * aux8[e];
                s += (int32_t)sc[g] * isum;
            }
            S[b] = s;
            if (Smin) Smin[b] = 0;
        }
    } else if (type == ORC_Q6_K) {
        int64_t nb = k / ORC_QK_K;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *x = w + b * ORC_Q6K_BYTES;
            const uint8_t *y = xq + b * ORC_Q8K_BYTES;
            const int8_t *q8 = (const int8_t *)(y + 4);
            const int8_t *sc = (const int8_t *)(x + 192);
            q6k_unpack(x, x + 128, aux8);
            int32_t s = 0;
            for (int j = 0; j < 16; j++) {
                int32_t isum = 0;
                for (int e = 16 * j; e < 16 * j + 16; e++) isum += (int32_t)q8[e] * aux8[e];
                s += (int32_t)sc[j] * isum;
            }
            S[b] = s;
            if (Smin) Smin[b] = 0;
        }
    } else if (type == ORC_Q4_0) {
        int64_t nb = k / ORC_QK8_0;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *x = w + b * ORC_Q4_0_BYTES;
            const uint8_t *y = xq + b * ORC_Q8_0_BYTES;
            int32_t s = 0;
            for (int j = 0; j < 16; j++)
                s += ((int32_t)(x[2 + j] & 0x0F) - 8) * (int32_t)(int8_t)y[2 + j] +
                     ((int32_t)(x[2 + j] >> 4) - 8) * (int32_t)(int8_t)y[2 + 16 + j];
            S[b] = s;
            if (Smin) Smin[b] = 0;
        }
    } else if (type == ORC_Q5_0) {
        int64_t nb = k / ORC_QK8_0;
        for (int64_t b = 0; b < nb; b++) {
            S[b] = q5_0_block_sum(w + b * ORC_Q5_0_BYTES, xq + b * ORC_Q8_0_BYTES);
            if (Smin) Smin[b] = 0;
        }
    } else if (type == ORC_Q8_0) {
        int64_t nb = k / ORC_QK8_0;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *x = w + b * ORC_Q8_0_BYTES;
            const uint8_t *y = xq + b * ORC_Q8_0_BYTES;
            int32_t s = 0;
            for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)x[2 + j] * (int32_t)(int8_t)y[2 + j];
            S[b] = s;
            if (Smin) Smin[b] = 0;
        }
    }
}

/* Block sums for every (row of xq, weight row): S and Smin [m][n][nblk],
 * rows in parallel.  Same arithmetic as orc_block_sums. */
int orc_block_sums_mat(int type, int64_t m, int64_t n, int64_t k, const uint8_t *w, const uint8_t *xq,
                       int32_t *S, int32_t *Smin, int nthreads) {
    if (!orc_known_type(type)) return -2;
    int64_t wblk = orc_type_block_elems(type);
    if (k <= 0 || k % wblk != 0 || m < 0 || n < 0) return -3;
    const int64_t nblk = k / wblk;
    const size_t row_w = (size_t)nblk * orc_type_block_bytes(type);
    const int at = type == ORC_Q8_0 || type == ORC_Q4_0 || type == ORC_Q5_0 ? ORC_Q8_0 : ORC_Q8_K;
    const size_t row_x = (size_t)(k / orc_type_block_elems(at)) * orc_type_block_bytes(at);
    if (nthreads <= 0) nthreads = orc_max_threads();
#pragma omp parallel for schedule(dynamic, 64) num_threads(nthreads)
    for (int64_t i = 0; i < m * n; i++) {
        const int64_t r = i / n, c = i % n;
        orc_block_sums(type, k, w + (size_t)c * row_w, xq + (size_t)r * row_x, S + (size_t)i * nblk,
                       Smin + (size_t)i * nblk);
    }
    return 0;
}

/* ---------------------------------------------------------- matmul */

int orc_known_type(int type) {
    return type == ORC_Q2_K || type == ORC_Q3_K || type == ORC_Q4_K || type == ORC_Q5_K || type == ORC_Q6_K ||
           type == ORC_Q8_0 || type == ORC_Q4_0 || type == ORC_Q5_0;
}

static int act_type_for(int type) { return type == ORC_Q8_0 || type == ORC_Q4_0 || type == ORC_Q5_0 ? ORC_Q8_0 : ORC_Q8_K; }

static float vec_dot(int type, int64_t k, const uint8_t *w, const uint8_t *xq) {
    switch (type) {
    case ORC_Q2_K: return orc_vec_dot_q2k_q8k(k, w, xq);
    case ORC_Q3_K: return orc_vec_dot_q3k_q8k(k, w, xq);
    case ORC_Q4_K: return orc_vec_dot_q4k_q8k(k, w, xq);
    case ORC_Q5_K: return orc_vec_dot_q5k_q8k(k, w, xq);
    case ORC_Q4_0: return orc_vec_dot_q4_0_q8_0(k, w, xq);
    case ORC_Q5_0: return orc_vec_dot_q5_0_q8_0(k, w, xq);
    case ORC_Q6_K: return orc_vec_dot_q6k_q8k(k, w, xq);
    default: return orc_vec_dot_q8_0_q8_0(k, w, xq);
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Inner part of k_quants::matmul: for each row, the n columns are
 * computed independently (candle: rayon par_iter with_min_len(128) /
 * with_max_len(512); here OpenMP dynamic chunks of 256 columns). */
int orc_matmul_preq(int type, int64_t m, int64_t k, int64_t n, const uint8_t *xq, float *dst,
                    const uint8_t *w, int nthreads) {
    if (!orc_known_type(type)) return -2;
    int64_t wblk = orc_type_block_elems(type);
    if (k <= 0 || k % wblk != 0 || m < 0 || n < 0) return -3;
    size_t row_w = (size_t)(k / wblk) * orc_type_block_bytes(type);
    int at = act_type_for(type);
    size_t row_x = (size_t)(k / orc_type_block_elems(at)) * orc_type_block_bytes(at);
    if (nthreads <= 0) nthreads = orc_max_threads();
    for (int64_t r = 0; r < m; r++) {
        const uint8_t *xr = xq + (size_t)r * row_x;
        float *dr = dst + (size_t)r * n;
#pragma omp parallel for schedule(dynamic, 256) num_threads(nthreads)
        for (int64_t c = 0; c < n; c++) dr[c] = vec_dot(type, k, w + (size_t)c * row_w, xr);
    }
    return 0;
}

/* k_quants::matmul<T>((m,k,n), lhs, rhs_t, dst): quantize every lhs row
 * serially with T::VecDotType::from_float, then the column loop. */
int orc_matmul(int type, int64_t m, int64_t k, int64_t n, const float *lhs, const uint8_t *w,
               float *dst, int nthreads) {
    if (!orc_known_type(type)) return -2;
    int64_t wblk = orc_type_block_elems(type);
    if (k <= 0 || k % wblk != 0 || m < 0 || n < 0) return -3;
    int at = act_type_for(type);
    size_t row_x = (size_t)(k / orc_type_block_elems(at)) * orc_type_block_bytes(at);
    uint8_t *xq = (uint8_t *)calloc((size_t)(m > 0 ? m : 1), row_x);
    if (!xq) return -6;
    for (int64_t r = 0; r < m; r++) {
        if (at == ORC_Q8_K)
            orc_quantize_row_q8k(lhs + (size_t)r * k, k, xq + (size_t)r * row_x);
        else
            orc_quantize_row_q8_0(lhs + (size_t)r * k, k, xq + (size_t)r * row_x);
    }
    int rc = orc_matmul_preq(type, m, k, n, xq, dst, w, nthreads);
    free(xq);
    return rc;
}

/* GGML dequantisation of one weight row (value = d*sc*q - dmin*m for
 * Q2_K, Q4_K and Q5_K, d*sc*q for Q3_K and Q6_K, d*q for Q8_0), f32. */
int orc_dequantize_row(int type, const uint8_t *w, int64_t k, float *out) {
    int8_t aux8[256];
    if (type == ORC_Q4_K) {
        if (k % ORC_QK_K) return -3;
        for (int64_t b = 0; b < k / ORC_QK_K; b++) {
            const uint8_t *x = w + b * ORC_Q4K_BYTES;
            uint8_t sc[8], mn[8];
            q4k_scales_mins(x + 4, sc, mn);
            q4k_unpack(x + 16, aux8);
            float d = orc_f16_to_f32(rd_u16(x)), dmin = orc_f16_to_f32(rd_u16(x + 2));
            for (int e = 0; e < 256; e++)
                out[b * 256 + e] = d * (float)sc[e / 32] * (float)aux8[e] - dmin * (float)mn[e / 32];
        }
        return 0;
    }
    if (type == ORC_Q5_K) {
        if (k % ORC_QK_K) return -3;
        for (int64_t b = 0; b < k / ORC_QK_K; b++) {
            const uint8_t *x = w + b * ORC_Q5K_BYTES;
            uint8_t sc[8], mn[8];
            q4k_scales_mins(x + 4, sc, mn);
            q5k_unpack(x + 16, x + 48, aux8);
            float d = orc_f16_to_f32(rd_u16(x)), dmin = orc_f16_to_f32(rd_u16(x + 2));
            for (int e = 0; e < 256; e++)
                out[b * 256 + e] = d * (float)sc[e / 32] * (float)aux8[e] - dmin * (float)mn[e / 32];
        }
        return 0;
    }
    if (type == ORC_Q2_K) {
        if (k % ORC_QK_K) return -3;
        for (int64_t b = 0; b < k / ORC_QK_K; b++) {
            const uint8_t *x = w + b * ORC_Q2K_BYTES;
            q2k_unpack(x + 16, aux8);
            float d = orc_f16_to_f32(rd_u16(x + 80)), dmin = orc_f16_to_f32(rd_u16(x + 82));
            for (int e = 0; e < 256; e++)
                out[b * 256 + e] = d * (float)(x[e / 16] & 0xF) * (float)aux8[e] - dmin * (float)(x[e / 16] >> 4);
        }
        return 0;
    }
    if (type == ORC_Q3_K) {
        if (k % ORC_QK_K) return -3;
        int8_t sc[16];
        for (int64_t b = 0; b < k / ORC_QK_K; b++) {
            const uint8_t *x = w + b * ORC_Q3K_BYTES;
            q3k_unpack(x, x + 32, aux8);
            q3k_scales(x + 96, sc);
            float d = orc_f16_to_f32(rd_u16(x + 108));
            for (int e = 0; e < 256; e++) out[b * 256 + e] = d * (float)(sc[e / 16] * aux8[e]);
        }
        return 0;
    }
    if (type == ORC_Q6_K) {
        if (k % ORC_QK_K) return -3;
        for (int64_t b = 0; b < k / ORC_QK_K; b++) {
            const uint8_t *x = w + b * ORC_Q6K_BYTES;
            const int8_t *sc = (const int8_t *)(x + 192);
            q6k_unpack(x, x + 128, aux8);
            float d = orc_f16_to_f32(rd_u16(x + 208));
            for (int e = 0; e < 256; e++) out[b * 256 + e] = d * (float)(sc[e / 16] * aux8[e]);
        }
        return 0;
    }
    if (type == ORC_Q4_0) {
        if (k % ORC_QK8_0) return -3;
        for (int64_t b = 0; b < k / ORC_QK8_0; b++) {
            const uint8_t *x = w + b * ORC_Q4_0_BYTES;
            float d = orc_f16_to_f32(rd_u16(x));
            for (int j = 0; j < 16; j++) {
                out[b * 32 + j] = (float)((int32_t)(x[2 + j] & 0x0F) - 8) * d;
                out[b * 32 + j + 16] = (float)((int32_t)(x[2 + j] >> 4) - 8) * d;
            }
        }
        return 0;
    }
    if (type == ORC_Q5_0) {
        if (k % ORC_QK8_0) return -3;
        for (int64_t b = 0; b < k / ORC_QK8_0; b++) {
            const uint8_t *x = w + b * ORC_Q5_0_BYTES;
            const uint32_t qh = rd_u32(x + 2);
            float d = orc_f16_to_f32(rd_u16(x));
            for (int j = 0; j < 16; j++) {
                out[b * 32 + j] = (float)((int32_t)((x[6 + j] & 0x0F) | (((qh >> j) & 1) << 4)) - 16) * d;
                out[b * 32 + j + 16] = (float)((int32_t)((x[6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16) * d;
            }
        }
        return 0;
    }
    if (type == ORC_Q8_0) {
        if (k % ORC_QK8_0) return -3;
        for (int64_t b = 0; b < k / ORC_QK8_0; b++) {
            const uint8_t *x = w + b * ORC_Q8_0_BYTES;
            float d = orc_f16_to_f32(rd_u16(x));
            for (int e = 0; e < 32; e++) out[b * 32 + e] = d * (float)(int8_t)x[2 + e];
        }
        return 0;
    }
    return -2;
}

/* Array forms of the f16 conversions (for exhaustive checks). */
void orc_f16_to_f32_n(const uint16_t *h, int64_t n, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(h[i]);
}

void orc_f32_to_f16_n(const float *f, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(f[i]);
}
