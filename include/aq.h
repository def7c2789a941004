/*
 * aq.h -- C ABI of the MI355X (gfx950) quantized-weight matmul library
 * (libarm_ai_amd.so).
 *
 * This is the drop-in boundary for the hot path of mlainez/arm_ai's
 * ArmAI.LlamaCandle: GGUF block-quantized weights (Q4_K, Q6_K, Q8_0) times
 * f32 activations that are quantized to Q8_K (Q8_0 for Q8_0 weights), as
 * candle-core 0.8.4's QMatMul does on the CPU.  The reference reaches that
 * code through
 *   native/arm_ai_nif/src/llama_candle.rs:35-48   load_model -> ModelWeights::from_gguf
 *   native/arm_ai_nif/src/llama_candle.rs:93, :119 ModelWeights::forward -> QMatMul::forward
 *   candle-core 0.8.4 QuantizedType::matmul_t((m,k,n), lhs, dst) -> k_quants::matmul<T>
 * (candle-core is pinned by native/arm_ai_nif/Cargo.lock; it is a registry
 * crate and not vendored).  A Rust caller binds these functions with
 * `extern "C"` declarations; the binding is spelled out in INTEGRATION.md.
 *
 * Conventions
 *  - Every function returns an aq_status (0 = AQ_OK, negative = error) and
 *    never aborts the process; aq_last_error() gives the calling thread's
 *    last message.
 *  - Weight type ids are GGUF/GGML dtype ids (Q8_0 = 8, Q4_K = 12, Q6_K = 14).
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
    AQ_TYPE_Q8_0 = 8,
    AQ_TYPE_Q4_K = 12,
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

/* Quantise-once / reuse.  candle's quantized_llama feeds the same input to
 * several QMatMuls (wq/wk/wv, w1/w3), each quantising it again inside
 * k_quants::matmul; these two calls let a caller quantise once on the device
 * and run several matmuls on the result.  The activation buffer layout is
 * private to this library; size it with aq_act_bytes.
 *   act_type: AQ_TYPE_Q8_K (for Q4_K / Q6_K weights) or AQ_TYPE_Q8_0 (for Q8_0). */
size_t aq_act_bytes(int act_type, int64_t m, int64_t k);
int aq_quantize_act_device(aq_ctx *ctx, int act_type, const float *d_x, int64_t m, int64_t k, void *d_act);
int aq_qmatmul_preq_device(aq_ctx *ctx, const aq_qweight *w, const void *d_act, int64_t m, int64_t k,
                           float *d_dst);

/* BlockQ8K::from_float on the GPU: host f32 [m][k] -> host Q8_K blocks
 * (m * k/256 blocks of 292 bytes: f32 d, i8 qs[256], i16 bsums[16]). */
int aq_quantize_q8k(aq_ctx *ctx, const float *x, int64_t m, int64_t k, void *out_blocks);

/* BlockQ8_0::from_float on the GPU: host f32 [m][k] -> host Q8_0 blocks
 * (m * k/32 blocks of 34 bytes: f16 d, i8 qs[32]). */
int aq_quantize_q8_0(aq_ctx *ctx, const float *x, int64_t m, int64_t k, void *out_blocks);

/* The integer intermediates of the GPU dot products, for bit-exact checks:
 * S[m][n][nblk] and Smin[m][n][nblk] (int32), per weight block of the row:
 *   Q4_K: S = sum_j sc_j * sum_{e in sub-block j} q_e*qx_e,  Smin = sum_g bsums_g * m_{g/2}
 *   Q6_K: S = sum_j sc_j * sum_{e in sub-block j} q6_e*qx_e, Smin = 0
 *   Q8_0: S = sum_{32} qw*qx per 32-block,                    Smin = 0
 * computed by the same kernel code as aq_qmatmul_f32 (batch <= 8 path)
 * or the prefill GEMM (m > 8) with an integer epilogue.  Host buffers. */
int aq_qmatmul_block_sums(aq_ctx *ctx, const aq_qweight *w, const float *lhs, int64_t m,
                          int64_t k, int32_t *S, int32_t *Smin);

#ifdef __cplusplus
}
#endif
#endif /* ARM_AI_AMD_AQ_H */
