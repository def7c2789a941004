/*
 * crate_ops.c -- CPU restatement of the arm_ai NIF crate's own int8 / int4
 * kernels (native/arm_ai_nif/src/shape_ops.rs), the secondary quantized
 * matmuls next to candle's QMatMul.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the product library never links
 * this code.  Each function restates the reference function cited in its
 * header comment, in the same operation order, with IEEE f32 arithmetic and
 * no FMA contraction (the Rust code performs separate multiplies and adds).
 *
 * Rust semantics restated here:
 *   f32::round      -> roundf (ties away from zero)
 *   `x as i32`      -> saturating conversion, NaN -> 0
 *   clamp(lo, hi)   -> min(max(x, lo), hi)
 *   f32::abs / max  -> fabsf / fmaxf (max ignores a NaN operand)
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

static inline int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

static inline int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* int8_dot, the portable form (shape_ops.rs:1361-1370): exact i32 sum.  The
 * NEON forms (:1305-1358) sum the same products in another order, which an
 * i32 sum without overflow does not see. */
static int32_t int8_dot(const int8_t *a, const int8_t *w, int64_t k) {
    int32_t t = 0;
    for (int64_t i = 0; i < k; i++) t += (int32_t)a[i] * (int32_t)w[i];
    return t;
}

/* int8_matmul_f32 (shape_ops.rs:1169-1211):
 * out[i][j] = (acc as f32) * act_scale * w_scales[j]. */
void orc_int8_matmul_f32(const int8_t *a, const int8_t *w, float act_scale, const float *w_scales, int64_t m,
                         int64_t n, int64_t k, float *out) {
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
            const int32_t acc = int8_dot(a + i * k, w + j * k, k);
            out[i * n + j] = ((float)acc * act_scale) * w_scales[j];
        }
}

/* int8_matmul_f32_per_token (shape_ops.rs:1222-1264):
 * out[i][j] = (acc as f32) * act_scales[i] * w_scales[j]. */
void orc_int8_matmul_f32_per_token(const int8_t *a, const int8_t *w, const float *act_scales, const float *w_scales,
                                   int64_t m, int64_t n, int64_t k, float *out) {
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
            const int32_t acc = int8_dot(a + i * k, w + j * k, k);
            out[i * n + j] = ((float)acc * act_scales[i]) * w_scales[j];
        }
}

/* quantize_int8_per_token (shape_ops.rs:1273-1292): per row
 * max_abs = fold(0, max(|x|)); scale = max_abs > 0 ? max_abs / 127 : 1;
 * q = clamp(round(x / scale) as i32, -127, 127). */
void orc_quantize_int8_per_token(const float *a, int64_t m, int64_t k, int8_t *q, float *scales) {
    for (int64_t i = 0; i < m; i++) {
        const float *row = a + i * k;
        float max_abs = 0.0f;
        for (int64_t j = 0; j < k; j++) max_abs = fmaxf(max_abs, fabsf(row[j]));
        const float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
        scales[i] = scale;
        for (int64_t j = 0; j < k; j++) q[i * k + j] = (int8_t)clamp_i32(sat_i32(roundf(row[j] / scale)), -127, 127);
    }
}

/* dequant_matmul_int8_f32 (shape_ops.rs:1525-1582): for each (batch, row,
 * column): acc = sequential sum of a[kk] * (w[kk] as f32); out = acc * s. */
void orc_dequant_matmul_int8_f32(const float *act, const int8_t *w, const float *scales, int64_t b, int64_t m,
                                 int64_t n, int64_t k, float *out) {
    for (int64_t r = 0; r < b * m; r++)
        for (int64_t j = 0; j < n; j++) {
            float acc = 0.0f;
            for (int64_t kk = 0; kk < k; kk++) acc += act[r * k + kk] * (float)w[j * k + kk];
            out[r * n + j] = acc * scales[j];
        }
}

/* dequant_matmul_f16_f32, the portable form (shape_ops.rs:1463-1490):
 * total = sequential sum of a[kk] * f16_to_f32(w[kk]).  (The aarch64 form,
 * :1386-1461, sums four lanes and a tail; same terms, another order.) */
void orc_dequant_matmul_f16_f32(const float *act, const uint16_t *w, int64_t b, int64_t m, int64_t n, int64_t k,
                                float *out) {
    for (int64_t r = 0; r < b * m; r++)
        for (int64_t j = 0; j < n; j++) {
            float total = 0.0f;
            for (int64_t kk = 0; kk < k; kk++) total += act[r * k + kk] * orc_f16_to_f32(w[j * k + kk]);
            out[r * n + j] = total;
        }
}

/* int4_matmul_f32 (shape_ops.rs:3175-3236): Q4_0-style packed weights,
 * [N][K/2] bytes (low nibble = even k), [N][K/32] f32 scales; per group
 * group_acc += a_lo * lo + a_hi * hi (lo, hi = nibble - 8), then
 * acc += group_acc * scale. */
void orc_int4_matmul_f32(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t m, int64_t n,
                         int64_t k, float *out) {
    const int64_t ng = k / 32, bpr = k / 2;
    for (int64_t mi = 0; mi < m; mi++)
        for (int64_t ni = 0; ni < n; ni++) {
            const uint8_t *wr = w_packed + ni * bpr;
            const float *sr = w_scales + ni * ng;
            const float *ar = a + mi * k;
            float acc = 0.0f;
            for (int64_t g = 0; g < ng; g++) {
                float group_acc = 0.0f;
                for (int j = 0; j < 16; j++) {
                    const uint8_t byte = wr[g * 16 + j];
                    const int lo = (byte & 0x0F) - 8, hi = ((byte >> 4) & 0x0F) - 8;
                    const float t = ar[g * 32 + 2 * j] * (float)lo + ar[g * 32 + 2 * j + 1] * (float)hi;
                    group_acc += t;
                }
                acc += group_acc * sr[g];
            }
            out[mi * n + ni] = acc;
        }
}

/* int4_matmul_gemv_neon (shape_ops.rs:3059-3166), its aarch64 order: per
 * group, four chunks of 8 weights in k order, each chunk summed as
 * vaddvq(prod_lo + prod_hi) = ((p0 + p4) + (p1 + p5)) + ((p2 + p6) + (p3 + p7)),
 * group_acc = c0 + c8 + c16 + c24, total += group_acc * scale. */
void orc_int4_matmul_gemv(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n, int64_t k,
                          float *out) {
    const int64_t ng = k / 32, bpr = k / 2;
    for (int64_t j = 0; j < n; j++) {
        float total = 0.0f;
        for (int64_t g = 0; g < ng; g++) {
            float wv[32];
            for (int b = 0; b < 16; b++) {
                const uint8_t byte = w_packed[j * bpr + g * 16 + b];
                wv[2 * b] = (float)((byte & 0x0F) - 8);
                wv[2 * b + 1] = (float)(((byte >> 4) & 0x0F) - 8);
            }
            const float *ag = a + g * 32;
            float c[4];
            for (int ch = 0; ch < 4; ch++) {
                float p[8];
                for (int i = 0; i < 8; i++) p[i] = ag[8 * ch + i] * wv[8 * ch + i];
                const float s0 = p[0] + p[4], s1 = p[1] + p[5], s2 = p[2] + p[6], s3 = p[3] + p[7];
                c[ch] = (s0 + s1) + (s2 + s3);
            }
            const float group_acc = ((c[0] + c[1]) + c[2]) + c[3];
            total += group_acc * w_scales[j * ng + g];
        }
        out[j] = total;
    }
}

/* The activation quantisation of int4_matmul_gemv_q4_x_q8_neon
 * (shape_ops.rs:2936-2954): per group of 32, max_abs (strict > scan),
 * scale = max_abs > 0 ? max_abs / 127 : 1, inv = 1 / scale,
 * q = clamp(round(x * inv), -128, 127) as i8. */
void orc_quantize_q8_groups(const float *a, int64_t k, int8_t *q, float *scales) {
    for (int64_t g = 0; g < k / 32; g++) {
        const float *grp = a + g * 32;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; i++) {
            const float av = fabsf(grp[i]);
            if (av > max_abs) max_abs = av;
        }
        const float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
        scales[g] = scale;
        const float inv = 1.0f / scale;
        for (int i = 0; i < 32; i++) {
            const float v = roundf(grp[i] * inv);
            /* Rust f32::clamp keeps a NaN, and `NaN as i8` is 0 */
            q[g * 32 + i] = (int8_t)(v != v ? 0 : (int)fminf(fmaxf(v, -128.0f), 127.0f));
        }
    }
}

/* int4_matmul_gemv_q4_x_q8_neon (shape_ops.rs:2923-3028), aarch64 form:
 * the activation quantised as above; per group the exact i32 dot of the
 * (nibble - 8) weights with the i8 activation;
 * total += (group_dot as f32) * w_scale * a_scale, groups in order.
 * aq [k] and as [k/32] receive the quantised activation. */
void orc_int4_matmul_gemv_q4_x_q8(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n,
                                  int64_t k, float *out, int8_t *aq, float *as) {
    const int64_t ng = k / 32, bpr = k / 2;
    orc_quantize_q8_groups(a, k, aq, as);
    for (int64_t j = 0; j < n; j++) {
        float total = 0.0f;
        for (int64_t g = 0; g < ng; g++) {
            int32_t dot = 0;
            for (int b = 0; b < 16; b++) {
                const uint8_t byte = w_packed[j * bpr + g * 16 + b];
                dot += ((byte & 0x0F) - 8) * (int32_t)aq[g * 32 + 2 * b];
                dot += (((byte >> 4) & 0x0F) - 8) * (int32_t)aq[g * 32 + 2 * b + 1];
            }
            total += ((float)dot * w_scales[j * ng + g]) * as[g];
        }
        out[j] = total;
    }
}

/* quantize_int4_q4_0 (shape_ops.rs:3242-3275): per group of 32,
 * scale = max_abs > 0 ? max_abs / 7 : 1; q = clamp(round(x / scale) as i32,
 * -8, 7) + 8; byte j = (q_hi << 4) | q_lo for k = 2j (lo) and 2j + 1 (hi). */
void orc_quantize_int4_q4_0(const float *w, int64_t n, int64_t k, uint8_t *packed, float *scales) {
    const int64_t ng = k / 32;
    for (int64_t ni = 0; ni < n; ni++)
        for (int64_t g = 0; g < ng; g++) {
            const float *grp = w + ni * k + g * 32;
            float max_abs = 0.0f;
            for (int i = 0; i < 32; i++) max_abs = fmaxf(max_abs, fabsf(grp[i]));
            const float scale = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
            scales[ni * ng + g] = scale;
            for (int j = 0; j < 16; j++) {
                const int ql = clamp_i32(sat_i32(roundf(grp[2 * j] / scale)), -8, 7) + 8;
                const int qh = clamp_i32(sat_i32(roundf(grp[2 * j + 1] / scale)), -8, 7) + 8;
                packed[ni * (k / 2) + g * 16 + j] = (uint8_t)((qh << 4) | ql);
            }
        }
}

/* dequantize_q6_k as the crate has it (shape_ops.rs:2848-2899), including
 * its sub-scale index: elements l, l+32, l+64, l+96 of half n use scales
 * 8n+0, 8n+2, 8n+4, 8n+6 for every l (GGML uses 8n + l/16 + {0,2,4,6}).
 * value = d * (s * q) as f32, q = 6-bit value - 32. */
void orc_dequantize_q6_k_crate(const uint8_t *in, int64_t n_blocks, float *out) {
    for (int64_t b = 0; b < n_blocks; b++) {
        const uint8_t *blk = in + b * 210;
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float d = orc_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
        float *o = out + b * 256;
        for (int nh = 0; nh < 2; nh++) {
            const int qlb = nh * 64, qhb = nh * 32, sb = nh * 8, ob = nh * 128;
            for (int l = 0; l < 32; l++) {
                const int qhi = qh[qhb + l];
                const int q1 = ((ql[qlb + l] & 0xF) | (((qhi >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[qlb + l + 32] & 0xF) | (((qhi >> 2) & 3) << 4)) - 32;
                const int q3 = (((ql[qlb + l] >> 4) & 0xF) | (((qhi >> 4) & 3) << 4)) - 32;
                const int q4 = (((ql[qlb + l + 32] >> 4) & 0xF) | (((qhi >> 6) & 3) << 4)) - 32;
                o[ob + l] = d * (float)(sc[sb + 0] * q1);
                o[ob + l + 32] = d * (float)(sc[sb + 2] * q2);
                o[ob + l + 64] = d * (float)(sc[sb + 4] * q3);
                o[ob + l + 96] = d * (float)(sc[sb + 6] * q4);
            }
        }
    }
}

/* q4_0_dequant_row_f32 (shape_ops.rs:2780-2808): out[2j] = (lo - 8) * scale,
 * out[2j + 1] = (hi - 8) * scale per group of 32. */
void orc_q4_0_dequant_row(const uint8_t *packed, const float *scales, int64_t row, int64_t k, float *out) {
    const int64_t ng = k / 32, bpr = k / 2;
    for (int64_t g = 0; g < ng; g++) {
        const float s = scales[row * ng + g];
        for (int j = 0; j < 16; j++) {
            const uint8_t byte = packed[row * bpr + g * 16 + j];
            out[g * 32 + 2 * j] = (float)((byte & 0x0F) - 8) * s;
            out[g * 32 + 2 * j + 1] = (float)(((byte >> 4) & 0x0F) - 8) * s;
        }
    }
}

/* q8_0_dequant_row_f32 (shape_ops.rs:2812-2832): out = (w as f32) * scale. */
void orc_q8_0_dequant_row(const int8_t *w, const float *scales, int64_t row, int64_t k, float *out) {
    const int64_t ng = k / 32;
    for (int64_t g = 0; g < ng; g++)
        for (int i = 0; i < 32; i++) out[g * 32 + i] = (float)w[row * k + g * 32 + i] * scales[row * ng + g];
}
