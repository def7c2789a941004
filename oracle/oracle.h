/*
 * oracle.h -- CPU restatement of the quantized-matmul path that
 * mlainez/arm_ai runs through candle-core 0.8.4 (k_quants.rs).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links or
 * calls this code.  It is used by tests/ (as the parity checker),
 * __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline
 * leg (as the timed CPU port of the reference algorithm).
 *
 * The reference crate reaches this arithmetic through
 *   native/arm_ai_nif/src/llama_candle.rs:93, :119  (ModelWeights::forward)
 *   -> candle_transformers quantized_llama -> QMatMul::forward
 *   -> candle_core::quantized::k_quants::matmul<T>
 * candle-core 0.8.4 is pinned by native/arm_ai_nif/Cargo.lock (candle-core
 * 0.8.4, registry crate, not vendored under /root/reference).  Its source
 * is not present in this image, so each function below restates the
 * published candle / GGML algorithm; the header comment of each function
 * says which part of candle it follows and how it is pinned.
 *
 * Block formats (GGUF, little endian):
 *   Q4_K 144 B: f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qs[128] @16
 *   Q5_K 176 B: f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qh[32] @16, u8 qs[128] @48
 *   Q6_K 210 B: u8 ql[128] @0, u8 qh[64] @128, i8 scales[16] @192, f16 d @208
 *   Q8_0  34 B: f16 d @0, i8 qs[32] @2
 *   Q4_0  18 B: f16 d @0, u8 qs[16] @2 (element j = qs[j] & 15, j+16 = qs[j] >> 4; value d*(q-8))
 *   Q8_K 292 B: f32 d @0, i8 qs[256] @4, i16 bsums[16] @260
 */
#ifndef ARM_AI_ORACLE_H
#define ARM_AI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_Q4_0 = 2,
    ORC_Q5_0 = 6,
    ORC_Q8_0 = 8,
    ORC_Q2_K = 10,
    ORC_Q3_K = 11,
    ORC_Q4_K = 12,
    ORC_Q5_K = 13,
    ORC_Q6_K = 14,
    ORC_Q8_K = 15,
};

#define ORC_QK_K 256
#define ORC_QK8_0 32
#define ORC_Q2K_BYTES 84
#define ORC_Q3K_BYTES 110
#define ORC_Q4K_BYTES 144
#define ORC_Q5K_BYTES 176
#define ORC_Q6K_BYTES 210
#define ORC_Q8_0_BYTES 34
#define ORC_Q4_0_BYTES 18
#define ORC_Q5_0_BYTES 22
#define ORC_Q8K_BYTES 292

/* IEEE binary16 <-> binary32 as the `half` crate does it (RNE). */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_n(const uint16_t *h, int64_t n, float *out);
void orc_f32_to_f16_n(const float *f, int64_t n, uint16_t *out);

/* Bytes of one block and elements per block for a GGUF type id; 0 if unknown. */
size_t orc_type_block_bytes(int type);
int orc_known_type(int type); /* 1 for the weight types below */
int64_t orc_type_block_elems(int type);

/* Activation quantizers (one row of k floats -> k/blk blocks). Return 0 or -1 (k % blk != 0). */
int orc_quantize_row_q8k(const float *x, int64_t k, uint8_t *out);
int orc_quantize_row_q8_0(const float *x, int64_t k, uint8_t *out);

/* vec_dot_unopt: one weight row (k elements, packed) . one quantized activation row. */
float orc_vec_dot_q2k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq);
float orc_vec_dot_q3k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq);
float orc_vec_dot_q4k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq);
float orc_vec_dot_q5k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq);
float orc_vec_dot_q6k_q8k(int64_t k, const uint8_t *w, const uint8_t *xq);
float orc_vec_dot_q8_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *xq);
float orc_vec_dot_q4_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *xq);
float orc_vec_dot_q5_0_q8_0(int64_t k, const uint8_t *w, const uint8_t *xq);

/* Integer intermediates per block (the bit-exact gate).
 * Q4_K, Q5_K: S[b] = sum_j sc_j * sum_{e in j} q_e*qx_e ; Smin[b] = sum_g bsums_g * m_{g/2}
 * Q6_K: S[b] = sum_j sc_j * sum_{e in j} q6_e*qx_e ; Smin unused
 * Q8_0: S[b] = sum_{32} qw*qx (per 32-block)
 * Q4_0: S[b] = sum_{32} (q-8)*qx (per 32-block)                                 */
void orc_block_sums(int type, int64_t k, const uint8_t *w, const uint8_t *xq,
                    int32_t *S, int32_t *Smin);

/* orc_block_sums for all m x n (activation row, weight row) pairs:
 * S, Smin [m][n][blocks].  OpenMP over the pairs. */
int orc_block_sums_mat(int type, int64_t m, int64_t n, int64_t k, const uint8_t *w, const uint8_t *xq,
                       int32_t *S, int32_t *Smin, int nthreads);

/* k_quants::matmul<T>: dst[m][n] = lhs[m][k] . W[n][k]^T.
 * Serial per-row activation quantisation, then columns in parallel
 * (nthreads OpenMP threads, chunks of 256 columns).  Returns 0, or a
 * negative code for a bad type / shape. */
int orc_matmul(int type, int64_t m, int64_t k, int64_t n, const float *lhs,
               const uint8_t *w, float *dst, int nthreads);

/* Same as orc_matmul but with the activation already quantised
 * (m rows of k/256 Q8_K blocks, or k/32 Q8_0 blocks for Q8_0 weights). */
int orc_matmul_preq(int type, int64_t m, int64_t k, int64_t n, const uint8_t *xq,
                    float *dst, const uint8_t *w, int nthreads);

/* Dequantize one weight row to f32 (GGML value formula).  For error analysis. */
int orc_dequantize_row(int type, const uint8_t *w, int64_t k, float *out);

/* Number of OpenMP threads the library would use by default. */
int orc_max_threads(void);

/* ---- the NIF crate's own int8 / int4 kernels (crate_ops.c;
 *      native/arm_ai_nif/src/shape_ops.rs) ---- */
void orc_int8_matmul_f32(const int8_t *a, const int8_t *w, float act_scale, const float *w_scales, int64_t m,
                         int64_t n, int64_t k, float *out);
void orc_int8_matmul_f32_per_token(const int8_t *a, const int8_t *w, const float *act_scales, const float *w_scales,
                                   int64_t m, int64_t n, int64_t k, float *out);
void orc_quantize_int8_per_token(const float *a, int64_t m, int64_t k, int8_t *q, float *scales);
void orc_dequant_matmul_int8_f32(const float *act, const int8_t *w, const float *scales, int64_t b, int64_t m,
                                 int64_t n, int64_t k, float *out);
void orc_dequant_matmul_f16_f32(const float *act, const uint16_t *w, int64_t b, int64_t m, int64_t n, int64_t k,
                                float *out);
void orc_int4_matmul_f32(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t m, int64_t n,
                         int64_t k, float *out);
void orc_int4_matmul_gemv(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n, int64_t k,
                          float *out);
void orc_quantize_q8_groups(const float *a, int64_t k, int8_t *q, float *scales);
void orc_int4_matmul_gemv_q4_x_q8(const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n,
                                  int64_t k, float *out, int8_t *aq, float *as);
void orc_quantize_int4_q4_0(const float *w, int64_t n, int64_t k, uint8_t *packed, float *scales);
void orc_dequantize_q6_k_crate(const uint8_t *in, int64_t n_blocks, float *out);
void orc_q4_0_dequant_row(const uint8_t *packed, const float *scales, int64_t row, int64_t k, float *out);
void orc_q8_0_dequant_row(const int8_t *w, const float *scales, int64_t row, int64_t k, float *out);

#ifdef __cplusplus
}
#endif
#endif
