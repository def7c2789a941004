/*
 * aq.h -- C ABI of the MI355X (gfx950) quantized-weight matmul library
 * (libarm_ai_amd.so).
 *
 * This is the drop-in boundary for the hot path of mlainez/arm_ai's
 * ArmAI.LlamaCandle: GGUF block-quantized weights (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0) times
 * f32 activations that are quantized to Q8_K (Q8_0 for Q8_0 weights), as
 * candle-core 0.8.4's QMatMul does on the CPU.  The reference reaches that
 * code through
 *   native/arm_ai_nif/src/llama_candle.rs:35-48   load_model -> ModelWeights::from_gguf
 *   native/arm_ai_nif/src/llama_candle.rs:93, :119 ModelWeights::forward -> QMatMul::forward
 *   candle-core 0.8.4 QuantizedType::matmul_t((m,k,n), lhs, dst) -> k_quants::matmul<T>
 * (candle-core is pinned by native/arm_ai_nif/Cargo.lock; it is a registry
 * crate and not vendored).  A Rust caller binds these functions with
 * `extern "C"` declarations of the same names and argument types
 * (native/arm_ai_nif/src/aq_sys.rs holds them).
 *
 * Conventions
 *  - Every function returns an aq_status (0 = AQ_OK, negative = error) and
 *    never aborts the process; aq_last_error() gives the calling thread's
 *    last message.
 *  - Weight type ids are GGUF/GGML dtype ids (Q4_0 = 2, Q5_0 = 6, Q8_0 = 8,
 *    Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14).  Every type
 *    runs the batch-1..8 matvec.  For m > 8, Q4_K, Q5_K, Q6_K, Q8_0, Q4_0
 *    and Q5_0 run a prefill GEMM (Q4_0 and Q5_0 on an int8 copy that the
 *    upload expands into the Q8_0 layout, 34 bytes per 32 weights beside
 *    their 18- or 22-byte decode tiles);
 *    Q2_K and Q3_K run the matvec in passes of 8 rows.
 *  - A weight is n rows (output features) by k columns (input features),
 *    row-major blocks, exactly candle's QTensor storage of shape (n, k).
 *  - Host-pointer entry points are synchronous at return.  Device-pointer
 *    entry points are asynchronous on the context's stream.
 *  - One aq_ctx owns one HIP stream and its scratch; use it from one thread
 *    at a time (the reference serialises each model behind a Mutex,
 *    llama_candle.rs:27-29, :80).
 */
#ifndef ARM_AI_AMD_AQ_H
#define ARM_AI_AMD_AQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum aq_status {
    AQ_OK = 0,
    AQ_ERR_INVALID_ARG = -1,      /* null pointer, negative size */
    AQ_ERR_UNSUPPORTED_TYPE = -2, /* weight / activation dtype not handled */
    AQ_ERR_SHAPE = -3,            /* k not a multiple of the block, lhs len != m*k, ... */
    AQ_ERR_NO_DEVICE = -4,        /* no HIP device, or device index out of range */
    AQ_ERR_HIP = -5,              /* a HIP runtime call failed */
    AQ_ERR_OOM = -6               /* device or pinned host allocation failed */
} aq_status;

typedef enum aq_type {
    AQ_TYPE_Q4_0 = 2,
    AQ_TYPE_Q5_0 = 6,
    AQ_TYPE_Q8_0 = 8,
    AQ_TYPE_Q2_K = 10,
    AQ_TYPE_Q3_K = 11,
    AQ_TYPE_Q4_K = 12,
    AQ_TYPE_Q5_K = 13,
    AQ_TYPE_Q6_K = 14,
    AQ_TYPE_Q8_K = 15
} aq_type;

typedef struct aq_ctx aq_ctx;
typedef struct aq_qweight aq_qweight;

/* Version of this ABI (bumped on any incompatible change). */
int aq_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *aq_last_error(void);

/* Number of visible HIP devices (0 on a machine without a GPU; returns AQ_OK). */
int aq_device_count(int *count);

/* Context = device + stream + grow-only scratch.
 * Replaces the Device::Cpu set up in llama_candle.rs:36 and :81. */
int aq_ctx_create(int device, aq_ctx **out);
int aq_ctx_destroy(aq_ctx *ctx);
int aq_ctx_synchronize(aq_ctx *ctx);
/* The context's hipStream_t, for callers that enqueue their own work. */
int aq_ctx_stream(aq_ctx *ctx, void **stream);

/* Upload a GGUF-block weight of n rows by k columns (nbytes must equal
 * n * k/block * block_bytes) to device memory, repacked into the kernel
 * layout.  Replaces QTensor construction in ModelWeights::from_gguf
 * (llama_candle.rs:42) -- the weight is uploaded once and stays in HBM. */
int aq_qweight_upload(aq_ctx *ctx, int type, const void *blocks, size_t nbytes, int64_t n,
                      int64_t k, aq_qweight **out);
/* Same, from GGUF blocks already in device memory (d_blocks). */
int aq_qweight_upload_device(aq_ctx *ctx, int type, const void *d_blocks, size_t nbytes,
                             int64_t n, int64_t k, aq_qweight **out);
int aq_qweight_free(aq_qweight *w);
int aq_qweight_info(const aq_qweight *w, int *type, int64_t *n, int64_t *k, size_t *device_bytes);

/* QMatMul::forward / QuantizedType::matmul_t((m,k,n), lhs, dst) with host
 * buffers: lhs f32 [m][k] row-major, dst f32 [m][n].  The activation rows
 * are quantised to Q8_K (Q8_0 for Q8_0 weights) on the GPU, then the
 * integer block dot products and f32 scaling run on the GPU.
 * k must equal the weight's k (candle: "last dim != k" is an error). */
int aq_qmatmul_f32(aq_ctx *ctx, const aq_qweight *w, const float *lhs, int64_t m, int64_t k,
                   float *dst);

/* Same with device pointers (d_lhs, d_dst in device memory), asynchronous
 * on the context stream. */
int aq_qmatmul_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_lhs, int64_t m,
                          int64_t k, float *d_dst);

/* aq_qmatmul_f32_device without any allocation (no counterpart in the
 * reference): for callers that cannot allocate device memory during a call,
 * such as code under HIP graph capture or a serving loop that forbids
 * hipMalloc.  The quantised activation and the prefill GEMM's workspace live
 * in a fixed array of aq_fixed_scratch_bytes() (32 MiB) per GPU, held until
 * the process ends; a call whose m, k and n need more returns AQ_ERR_SHAPE
 * (aq_qmatmul_f32_device has no such limit).  Every call on one GPU shares
 * that array, so calls that overlap on one GPU (two streams, two threads)
 * race: serialise them.  Same results as aq_qmatmul_f32_device. */
int aq_qmatmul_f32_device_noalloc(aq_ctx *ctx, const aq_qweight *w, const float *d_lhs, int64_t m, int64_t k,
                                  float *d_dst);
size_t aq_fixed_scratch_bytes(void);

/* Quantise-once / reuse.  candle's quantized_llama feeds the same input to
 * several QMatMuls (wq/wk/wv, w1/w3), each quantising it again inside
 * k_quants::matmul; these two calls let a caller quantise once on the device
 * and run several matmuls on the result.  The activation buffer layout is
 * private to this library; size it with aq_act_bytes.
 *   act_type: AQ_TYPE_Q8_K (for Q4_K / Q5_K / Q6_K weights) or AQ_TYPE_Q8_0 (for Q8_0 / Q4_0). */
size_t aq_act_bytes(int act_type, int64_t m, int64_t k);
int aq_quantize_act_device(aq_ctx *ctx, int act_type, const float *d_x, int64_t m, int64_t k, void *d_act);
int aq_qmatmul_preq_device(aq_ctx *ctx, const aq_qweight *w, const void *d_act, int64_t m, int64_t k,
                           float *d_dst);
/* Two QMatMul::forward calls on the same pre-quantised activation, w1's
 * result in d_y1 [m][w1 n] and w2's in d_y2 [m][w2 n] (llama's wq|wk and wv
 * on the attention norm's output, candle quantized_llama's attention block,
 * reached from llama_candle.rs:93).  A Q4_K w1 with a Q6_K or Q5_K w2 at a
 * GEMM-sized m runs as one launch (the two GEMMs in separate workgroups, w1
 * not split over k; w2's split partials then summed by a small second
 * launch); other cases make the two aq_qmatmul_preq_device calls.  Same
 * results as those calls up to the f32 summation order of w1's partials. */
int aq_qmatmul2_preq_device(aq_ctx *ctx, const aq_qweight *w1, const aq_qweight *w2, const void *d_act, int64_t m,
                            int64_t k, float *d_y1, float *d_y2);

/* BlockQ8K::from_float on the GPU: host f32 [m][k] -> host Q8_K blocks
 * (m * k/256 blocks of 292 bytes: f32 d, i8 qs[256], i16 bsums[16]). */
int aq_quantize_q8k(aq_ctx *ctx, const float *x, int64_t m, int64_t k, void *out_blocks);

/* BlockQ8_0::from_float on the GPU: host f32 [m][k] -> host Q8_0 blocks
 * (m * k/32 blocks of 34 bytes: f16 d, i8 qs[32]). */
int aq_quantize_q8_0(aq_ctx *ctx, const float *x, int64_t m, int64_t k, void *out_blocks);

/* The integer intermediates of the GPU dot products, for bit-exact checks:
 * S[m][n][nblk] and Smin[m][n][nblk] (int32), per weight block of the row:
 *   Q4_K, Q5_K: S = sum_j sc_j * sum_{e in sub-block j} q_e*qx_e,  Smin = sum_g bsums_g * m_{g/2}
 *   Q6_K: S = sum_j sc_j * sum_{e in sub-block j} q6_e*qx_e, Smin = 0
 *   Q8_0: S = sum_{32} qw*qx per 32-block,                    Smin = 0
 *   Q4_0: S = sum_{32} (q-8)*qx per 32-block,                 Smin = 0
 * computed by the same kernel code as aq_qmatmul_f32 (batch <= 8 path)
 * or the prefill GEMM (m > 8) with an integer epilogue.  Host buffers. */
int aq_qmatmul_block_sums(aq_ctx *ctx, const aq_qweight *w, const float *lhs, int64_t m,
                          int64_t k, int32_t *S, int32_t *Smin);

/* ===================================================================
 * Crate kernels: the NIF crate's own int8 / int4 kernels
 * (native/arm_ai_nif/src/shape_ops.rs), the secondary quantized matmuls that
 * the NIFs in native/arm_ai_nif/src/lib.rs expose next to candle's QMatMul.
 * Arguments keep the NIFs' meaning and order (binaries become pointers plus
 * the sizes the NIFs derive).  Integer dots, the int8 matmul scalings, the
 * quantizers and the dequantizers are bit-identical to the crate's scalar
 * code; the weight-only matmuls' f32 sums are reordered (tolerance-bound).
 * =================================================================== */

/* Weight formats of aq_weight_only_matmul_device / aq_dequant_rows_device. */
typedef enum aq_crate_weight {
    AQ_CRATE_W_Q4_0 = 0, /* [N][K/2] packed nibbles (low = even k), [N][K/32] f32 scales; value (q - 8) * s */
    AQ_CRATE_W_I8 = 1,   /* [N][K] int8, [N] f32 per-row scales (matmul) or [N][K/32] (row tables) */
    AQ_CRATE_W_F16 = 2   /* [N][K] IEEE binary16 */
} aq_crate_weight;

/* int8_matmul_f32 (shape_ops.rs:1169-1211; NIF int8_matmul_f32_op, lib.rs:216-236):
 * out[m][n] = (f32)(sum_k a[m][k] * w[n][k]) * act_scale * w_scales[n]. */
int aq_int8_matmul_f32(aq_ctx *ctx, const int8_t *a, const int8_t *w, const float *w_scales, float act_scale,
                       int64_t m, int64_t n, int64_t k, float *out);
/* int8_matmul_f32_per_token (shape_ops.rs:1222-1264; NIF lib.rs:240-266):
 * as above with act_scales[m] per row. */
int aq_int8_matmul_f32_per_token(aq_ctx *ctx, const int8_t *a, const int8_t *w, const float *act_scales,
                                 const float *w_scales, int64_t m, int64_t n, int64_t k, float *out);
/* Both, on device memory (d_act_scales null: act_scale for every row). */
int aq_int8_matmul_f32_device(aq_ctx *ctx, const int8_t *d_a, const int8_t *d_w, const float *d_act_scales,
                              float act_scale, const float *d_w_scales, int64_t m, int64_t n, int64_t k, float *d_out);

/* quantize_int8_per_token (shape_ops.rs:1273-1292; NIF lib.rs:269-296):
 * per row scale = max|x| / 127 (1 for a zero row), q = clamp(round(x / scale), -127, 127). */
int aq_quantize_int8_per_token(aq_ctx *ctx, const float *a, int64_t m, int64_t k, int8_t *q, float *scales);
int aq_quantize_int8_per_token_device(aq_ctx *ctx, const float *d_a, int64_t m, int64_t k, int8_t *d_q,
                                      float *d_scales);

/* dequant_matmul_int8_f32 (shape_ops.rs:1525-1582; NIF lib.rs:508-532):
 * out[b][m][n] = (sum_k act[b][m][k] * (f32)w[n][k]) * scales[n]. */
int aq_dequant_matmul_int8_f32(aq_ctx *ctx, const float *act, const int8_t *w, const float *scales, int64_t b,
                               int64_t m, int64_t n, int64_t k, float *out);
/* dequant_matmul_f16_f32 (shape_ops.rs:1386-1490; NIF lib.rs:176-195): f16 weights. */
int aq_dequant_matmul_f16_f32(aq_ctx *ctx, const float *act, const uint16_t *w, int64_t b, int64_t m, int64_t n,
                              int64_t k, float *out);
/* int4_matmul_f32 (shape_ops.rs:3175-3236; NIF lib.rs:451-475) and its M = 1
 * form int4_matmul_gemv_neon (shape_ops.rs:3059-3166; NIF lib.rs:428-448):
 * Q4_0-style weights, K a multiple of 32. */
int aq_int4_matmul_f32(aq_ctx *ctx, const float *a, const uint8_t *w_packed, const float *w_scales, int64_t m,
                       int64_t n, int64_t k, float *out);
int aq_int4_matmul_gemv(aq_ctx *ctx, const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n,
                        int64_t k, float *out);
/* The three weight-only matmuls on device memory (d_scales: per-group for
 * Q4_0, per-row for I8, unused for F16). */
int aq_weight_only_matmul_device(aq_ctx *ctx, int weight_format, const float *d_act, const void *d_w,
                                 const float *d_scales, int64_t m, int64_t n, int64_t k, float *d_out);

/* int4_matmul_gemv_q4_x_q8_neon (shape_ops.rs:2923-3028; NIF lib.rs:404-425):
 * the activation quantised per group of 32 (scale = max|x| / 127, 1 for a
 * zero group; q = clamp(round(x / scale), -128, 127)), exact integer group
 * dots with the (nibble - 8) weights, out[n] = sum_g (f32)dot * w_scale * a_scale. */
int aq_int4_matmul_gemv_q4_x_q8(aq_ctx *ctx, const float *a, const uint8_t *w_packed, const float *w_scales,
                                int64_t n, int64_t k, float *out);
/* Device form; d_act: aq_q4_x_q8_act_bytes(k) of scratch; d_q [k] and
 * d_qscales [k/32] (optional, may be null) receive the quantised activation. */
size_t aq_q4_x_q8_act_bytes(int64_t k);
int aq_int4_matmul_gemv_q4_x_q8_device(aq_ctx *ctx, const float *d_a, const uint8_t *d_w_packed,
                                       const float *d_w_scales, int64_t n, int64_t k, float *d_out, void *d_act,
                                       int8_t *d_q, float *d_qscales);

/* quantize_int4_q4_0 (shape_ops.rs:3242-3275; NIF lib.rs:478-505): per group of
 * 32, scale = max|x| / 7 (1 for a zero group), q = clamp(round(x / scale), -8, 7) + 8,
 * byte j = (q[2j+1] << 4) | q[2j]. */
int aq_quantize_int4_q4_0(aq_ctx *ctx, const float *w, int64_t n, int64_t k, uint8_t *packed, float *scales);

/* dequantize_q6_k as the crate has it (shape_ops.rs:2848-2899; NIF
 * dequantize_q6_k_op, lib.rs:346-355), including its sub-scale index
 * (8h + {0,2,4,6} for all 32 elements of a group; GGML uses 8h + l/16 + ...). */
int aq_dequantize_q6_k(aq_ctx *ctx, const void *blocks, size_t nbytes, int64_t n_elements, float *out);
int aq_dequantize_q6_k_device(aq_ctx *ctx, const void *d_blocks, int64_t n_elements, float *d_out);

/* q4_0_dequant_row_f32 / q8_0_dequant_row_f32 (shape_ops.rs:2780-2808,
 * :2812-2832; NIFs lib.rs:358-399): one row of an n_rows-row table. */
int aq_q4_0_dequant_row(aq_ctx *ctx, const uint8_t *packed, const float *scales, int64_t n_rows, int64_t row,
                        int64_t k, float *out);
int aq_q8_0_dequant_row(aq_ctx *ctx, const int8_t *w, const float *scales, int64_t n_rows, int64_t row, int64_t k,
                        float *out);
/* Batched device form (an embedding lookup): out[i] = row d_rows[i] of the
 * table; an index outside 0..n_rows-1 yields a zero row. */
int aq_dequant_rows_device(aq_ctx *ctx, int weight_format, const void *d_table, const float *d_scales, int64_t n_rows,
                           const int64_t *d_rows, int64_t n_out, int64_t k, float *d_out);

/* ===================================================================
 * Decode-step glue: the f32 operations between the quantized matmuls of
 * one Llama decode step, as candle-transformers 0.8.4 quantized_llama runs
 * them per generated token (reached from llama_candle.rs:119; next-token
 * pick as llama_candle.rs:154-176).  They are not QMatMul replacements: they
 * let a caller keep the whole step on the GPU (and capture it in a HIP
 * graph) around aq_qmatmul_f32_device.  Device pointers, asynchronous on the
 * context stream.  f32 sums are reordered relative to candle's CPU loops
 * (tolerance-bound, not bit-exact).
 * =================================================================== */
/* d_out[hidden] = row *d_tok of the f32 table [vocab][hidden] (zeros for an
 * id outside 0..vocab-1). */
int aq_llama_embed(aq_ctx *ctx, const float *d_table, int64_t vocab, const int64_t *d_tok, int64_t hidden,
                   float *d_out);
/* Per row of m rows of n: d_x += d_delta when d_delta is non-null (the
 * residual add, written back to d_x), then
 * d_out = d_x / sqrt(sum(d_x^2) / n + eps) * d_w (candle rms_norm). */
int aq_llama_rmsnorm(aq_ctx *ctx, float *d_x, const float *d_delta, const float *d_w, int64_t m, int64_t n, float eps,
                     float *d_out);
/* d_out[i] = silu(g[i]) * u[i] for i < n, with d_gu = [g (n) | u (n)]. */
int aq_llama_silu_mul(aq_ctx *ctx, const float *d_gu, int64_t n, float *d_out);
/* The prompt's forms of embed and silu_mul (m rows, m <= 65535 for silu):
 * d_out row r = table row d_tok[r]; d_out[r][i] = silu(d_g[r*ld + i]) *
 * d_u[r*ld + i] for i < n (the merged w1|w3 output: d_u = d_g + n, ld = 2n). */
int aq_llama_embed_rows(aq_ctx *ctx, const float *d_table, int64_t vocab, const int64_t *d_tok, int64_t m,
                        int64_t hidden, float *d_out);
int aq_llama_silu_mul_rows(aq_ctx *ctx, const float *d_g, const float *d_u, int64_t ld, int64_t m, int64_t n,
                           float *d_out);
/* Attention of one query position *d_pos (0 <= pos < max_seq): d_qk =
 * [q (n_head*head_dim) | k (n_kv*head_dim)], d_v (n_kv*head_dim), before
 * rotary embedding; d_cos / d_sin [max_seq][head_dim/2]; caches
 * [n_kv][max_seq][head_dim] for one layer.  Rotates q and k (interleaved
 * pairs), stores k and v at pos, and writes softmax(q.k/sqrt(head_dim)).v
 * over positions 0..pos for each query head to d_out (n_head*head_dim).
 * head_dim must divide 256 and be a multiple of 4; max_seq <= 8192; caches
 * and d_out 16-byte aligned.  For head_dim 64 or 128 with 1, 2, 3, 4 or 8 query
 * heads per kv head, the context is split over workgroups whose partial
 * results go to the context's attention workspace and are combined by a
 * second launch: calls on one context must not overlap (they are ordered
 * on its stream). */
int aq_llama_attn_decode(aq_ctx *ctx, const float *d_qk, const float *d_v, const float *d_cos, const float *d_sin,
                         const int64_t *d_pos, float *d_kcache, float *d_vcache, int64_t n_head, int64_t n_kv,
                         int64_t head_dim, int64_t max_seq, float *d_out);
/* Attention of the m prompt positions index_pos .. index_pos + m - 1
 * (index_pos + m <= max_seq; candle feeds the prompt at offset 0,
 * llama_candle.rs:93): row r of q, k, v starts at d_q + r*ldq, d_k + r*ldk,
 * d_v + r*ldv (n_head*head_dim, n_kv*head_dim, n_kv*head_dim values, before
 * rotary embedding).  Rotates k and stores k and v of every row in the
 * caches, then writes the causal softmax(q.k/sqrt(head_dim)).v over
 * positions 0 .. its own for every row and query head to d_out
 * [m][n_head*head_dim].  head_dim 64 or 128 (AQ_ERR_SHAPE otherwise); caches
 * and d_out 16-byte aligned. */
int aq_llama_attn_prefill(aq_ctx *ctx, const float *d_q, int64_t ldq, const float *d_k, int64_t ldk, const float *d_v,
                          int64_t ldv, const float *d_cos, const float *d_sin, int64_t index_pos, int64_t m,
                          float *d_kcache, float *d_vcache, int64_t n_head, int64_t n_kv, int64_t head_dim,
                          int64_t max_seq, float *d_out);
/* aq_qmatmul_f32_device for one row (m = 1) whose input is formed inside the
 * matmul kernel, so the step needs no separate launch for it:
 * rmsnorm: input = rms_norm(d_x + d_delta) * d_norm_w (eps as aq_llama_rmsnorm;
 *   d_delta may be null), and when d_h_out is non-null it receives
 *   d_x + d_delta (the residual stream), written once.  d_h_out must not
 *   alias d_x or d_delta.  AQ_ERR_SHAPE when k is too long to fuse
 *   (k > 8192 for Q4_K / Q6_K); then run aq_llama_rmsnorm and
 *   aq_qmatmul_f32_device instead.
 * silu_mul: d_gu = [g (k) | u (k)], input = silu(g) * u.
 * All pointers 16-byte aligned. */
int aq_qmatmul_rmsnorm_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_x, const float *d_delta,
                                  const float *d_norm_w, float eps, int64_t k, float *d_h_out, float *d_dst);
int aq_qmatmul_silu_mul_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_gu, int64_t k, float *d_dst);
/* Two aq_qmatmul_rmsnorm_f32_device calls on the same input (w1 -> d_dst1,
 * w2 -> d_dst2, both k columns) with the same results as the two calls;
 * d_h_out is written once.  For the projections that share an input but not
 * a type (TinyLlama Q4_K_M: wq|wk and wv).  One kernel launch for two Q4_K /
 * Q6_K weights, and for two Q5_0 / Q8_0 weights (a Q4_K_M file's types for
 * rows that are not whole 256-element groups, SmolLM-135M's 576); the two
 * calls for other pairs. */
int aq_qmatmul2_rmsnorm_f32_device(aq_ctx *ctx, const aq_qweight *w1, const aq_qweight *w2, const float *d_x,
                                   const float *d_delta, const float *d_norm_w, float eps, int64_t k, float *d_h_out,
                                   float *d_dst1, float *d_dst2);
/* Paired gate|up weights (the SwiGLU MLP, silu(w1 x) * (w3 x)).  A weight
 * holding the gate (w1) and up (w3) rows in pairs of four -- row 8b + j is
 * gate row 4b + j for j < 4 and up row 4b + j - 4 for j >= 4; n = 2 * ffn,
 * ffn a multiple of 4 (arm_ai_amd.llama.swiglu_pair_rows builds it) --
 * yields silu(g) * u without splitting its output:
 * aq_llama_swiglu_pairs: d_out[r][i] = silu(g) * u, i < ffn, of row r of
 *   such a weight's output d_y (row stride ld >= 2 * ffn; m <= 65535).
 * aq_qmatmul_rmsnorm_swiglu_f32_device: aq_qmatmul_rmsnorm_f32_device on such
 *   a weight, writing the ffn values silu(g) * u to d_dst in place of the n
 *   sums; the same values as the fused-norm matmul followed by
 *   aq_llama_swiglu_pairs (the row-per-lane forms apply silu in the matmul
 *   kernel; other shapes run those two steps, the matmul output in the
 *   context's scratch). */
int aq_llama_swiglu_pairs(aq_ctx *ctx, const float *d_y, int64_t ld, int64_t m, int64_t ffn, float *d_out);
/* The prompt's norm (aq_llama_rmsnorm) and SwiGLU pairs
 * (aq_llama_swiglu_pairs) with the result quantised to Q8_K in the same
 * launch, into the activation planes at d_act (aq_act_bytes(AQ_TYPE_Q8_K, m,
 * n or ffn) bytes, 256-byte aligned; the planes include the f16 copy of the
 * quants that the Q6_K / Q5_K GEMMs read) for aq_qmatmul_preq_device.  The
 * values are those of the unfused call followed by aq_quantize_act_device,
 * bit for bit; d_out, when non-null, receives the f32 values as well.  n is
 * a multiple of 256 up to 8192, ffn a multiple of 256 with m <= 65535 and ld
 * a multiple of 4; x, delta, w, y and out 16-byte aligned.  No counterpart
 * in the reference, whose prompt runs candle's rms_norm and silu ops and
 * then QMatMul::forward (which quantises its input again,
 * llama_candle.rs:93); these fold the quantisation into the op before the
 * GEMM. */
int aq_llama_rmsnorm_act(aq_ctx *ctx, float *d_x, const float *d_delta, const float *d_w, int64_t m, int64_t n,
                         float eps, float *d_out, void *d_act);
int aq_llama_swiglu_pairs_act(aq_ctx *ctx, const float *d_y, int64_t ld, int64_t m, int64_t ffn, float *d_out,
                              void *d_act);
/* 1 when aq_qmatmul_rmsnorm_swiglu_f32_device forms silu(g) * u inside the
 * matmul launch for a paired weight of this type (AQ_TYPE_*) and shape (n
 * rows, k columns), else 0 (it would run the matmul and the pairs as two
 * launches, and a caller keeping the two halves apart -- rows concatenated,
 * aq_qmatmul_silu_mul_f32_device on [g | u] -- launches fewer kernels).  No
 * GPU call. */
int aq_swiglu_fused(int type, int64_t n, int64_t k);
int aq_qmatmul_rmsnorm_swiglu_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_x, const float *d_delta,
                                         const float *d_norm_w, float eps, int64_t k, float *d_h_out, float *d_dst);
/* The end of a decode step and the start of the next, as
 * aq_qmatmul_rmsnorm_f32_device on the output head w (d_logits, w->n =
 * vocab values, no residual written), aq_llama_argmax over the logits
 * (d_tok, d_hist[*d_pos], *d_pos += 1) and aq_llama_embed of that token from
 * the f32 table d_table [vocab][hidden] into d_x_next (written after the
 * head has read d_x and d_delta, so it may be either): the same values.  Where the head takes the row-per-lane
 * matvec with the fused norm, each of its workgroups also keeps its largest
 * logit and row, and one more launch picks the token from those and writes
 * its embedding row (two launches in place of three, the argmax reading a
 * few KB in place of the logits).  Uses the context's head workspace: calls
 * on one context must not overlap. */
int aq_llama_head_argmax_embed(aq_ctx *ctx, const aq_qweight *w, const float *d_x, const float *d_delta,
                               const float *d_norm_w, float eps, int64_t k, float *d_logits, int64_t *d_tok,
                               int64_t *d_pos, int64_t *d_hist, int64_t hist_len, const float *d_table,
                               int64_t hidden, float *d_x_next);
/* Greedy pick: the first index of the largest of d_x[0..n) (d_x 16-byte
 * aligned, any n >= 1) goes to *d_tok and, when d_hist is non-null and
 * 0 <= *d_pos < hist_len, to d_hist[*d_pos]; then *d_pos += 1. */
int aq_llama_argmax(aq_ctx *ctx, const float *d_x, int64_t n, int64_t *d_tok, int64_t *d_pos, int64_t *d_hist,
                    int64_t hist_len);

#ifdef __cplusplus
}
#endif
#endif /* ARM_AI_AMD_AQ_H */
