//! Raw FFI of libarm_ai_amd.so: every function of include/aq.h, with the
//! header's argument names and C types (int -> c_int, int64_t -> i64,
//! size_t -> usize, pointers keep their constness).  tests/test_rust_shim.py
//! checks this file against the header, function by function.
//!
//! Conventions (include/aq.h): every call returns an aq_status (0 = AQ_OK,
//! negative = error) and never aborts; `last_error()` gives the calling
//! thread's message.  Host-pointer calls are synchronous at return;
//! `_device` calls are asynchronous on the context's HIP stream.
#![allow(non_camel_case_types, dead_code)]
use std::os::raw::{c_char, c_int, c_void};

#[repr(C)]
pub struct AqCtx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct AqQWeight {
    _p: [u8; 0],
}

pub const AQ_OK: c_int = 0;
pub const AQ_ERR_INVALID_ARG: c_int = -1;
pub const AQ_ERR_UNSUPPORTED_TYPE: c_int = -2;
pub const AQ_ERR_SHAPE: c_int = -3;
pub const AQ_ERR_NO_DEVICE: c_int = -4;
pub const AQ_ERR_HIP: c_int = -5;
pub const AQ_ERR_OOM: c_int = -6;

// GGUF / GGML dtype ids (candle's GgmlDType discriminants)
pub const AQ_TYPE_Q4_0: c_int = 2;
pub const AQ_TYPE_Q5_0: c_int = 6;
pub const AQ_TYPE_Q8_0: c_int = 8;
pub const AQ_TYPE_Q2_K: c_int = 10;
pub const AQ_TYPE_Q3_K: c_int = 11;
pub const AQ_TYPE_Q4_K: c_int = 12;
pub const AQ_TYPE_Q5_K: c_int = 13;
pub const AQ_TYPE_Q6_K: c_int = 14;
pub const AQ_TYPE_Q8_K: c_int = 15;

// weight formats of the crate kernels' device entries
pub const AQ_CRATE_W_Q4_0: c_int = 0;
pub const AQ_CRATE_W_I8: c_int = 1;
pub const AQ_CRATE_W_F16: c_int = 2;

extern "C" {
pub fn aq_abi_version() -> c_int;
    pub fn aq_last_error() -> *const c_char;
    pub fn aq_device_count(count: *mut c_int) -> c_int;
    pub fn aq_ctx_create(device: c_int, out: *mut *mut AqCtx) -> c_int;
    pub fn aq_ctx_destroy(ctx: *mut AqCtx) -> c_int;
    pub fn aq_ctx_synchronize(ctx: *mut AqCtx) -> c_int;
    pub fn aq_ctx_stream(ctx: *mut AqCtx, stream: *mut *mut c_void) -> c_int;
    pub fn aq_qweight_upload(ctx: *mut AqCtx, ty: c_int, blocks: *const c_void, nbytes: usize, n: i64, k: i64,
        out: *mut *mut AqQWeight) -> c_int;
    pub fn aq_qweight_upload_device(ctx: *mut AqCtx, ty: c_int, d_blocks: *const c_void, nbytes: usize, n: i64,
        k: i64, out: *mut *mut AqQWeight) -> c_int;
    pub fn aq_qweight_free(w: *mut AqQWeight) -> c_int;
    pub fn aq_qweight_info(w: *const AqQWeight, ty: *mut c_int, n: *mut i64, k: *mut i64, device_bytes: *mut usize) -> c_int;
    pub fn aq_qmatmul_f32(ctx: *mut AqCtx, w: *const AqQWeight, lhs: *const f32, m: i64, k: i64, dst: *mut f32) -> c_int;
    pub fn aq_qmatmul_f32_device(ctx: *mut AqCtx, w: *const AqQWeight, d_lhs: *const f32, m: i64, k: i64,
        d_dst: *mut f32) -> c_int;
    pub fn aq_qmatmul_f32_device_noalloc(ctx: *mut AqCtx, w: *const AqQWeight, d_lhs: *const f32, m: i64, k: i64,
        d_dst: *mut f32) -> c_int;
    pub fn aq_fixed_scratch_bytes() -> usize;
    pub fn aq_act_bytes(act_type: c_int, m: i64, k: i64) -> usize;
    pub fn aq_quantize_act_device(ctx: *mut AqCtx, act_type: c_int, d_x: *const f32, m: i64, k: i64,
        d_act: *mut c_void) -> c_int;
    pub fn aq_qmatmul_preq_device(ctx: *mut AqCtx, w: *const AqQWeight, d_act: *const c_void, m: i64, k: i64,
        d_dst: *mut f32) -> c_int;
    pub fn aq_qmatmul2_preq_device(ctx: *mut AqCtx, w1: *const AqQWeight, w2: *const AqQWeight, d_act: *const c_void,
        m: i64, k: i64, d_y1: *mut f32, d_y2: *mut f32) -> c_int;
    pub fn aq_quantize_q8k(ctx: *mut AqCtx, x: *const f32, m: i64, k: i64, out_blocks: *mut c_void) -> c_int;
    pub fn aq_quantize_q8_0(ctx: *mut AqCtx, x: *const f32, m: i64, k: i64, out_blocks: *mut c_void) -> c_int;
    pub fn aq_qmatmul_block_sums(ctx: *mut AqCtx, w: *const AqQWeight, lhs: *const f32, m: i64, k: i64, S: *mut i32,
        Smin: *mut i32) -> c_int;
    pub fn aq_int8_matmul_f32(ctx: *mut AqCtx, a: *const i8, w: *const i8, w_scales: *const f32, act_scale: f32,
        m: i64, n: i64, k: i64, out: *mut f32) -> c_int;
    pub fn aq_int8_matmul_f32_per_token(ctx: *mut AqCtx, a: *const i8, w: *const i8, act_scales: *const f32,
        w_scales: *const f32, m: i64, n: i64, k: i64, out: *mut f32) -> c_int;
    pub fn aq_int8_matmul_f32_device(ctx: *mut AqCtx, d_a: *const i8, d_w: *const i8, d_act_scales: *const f32,
        act_scale: f32, d_w_scales: *const f32, m: i64, n: i64, k: i64, d_out: *mut f32) -> c_int;
    pub fn aq_quantize_int8_per_token(ctx: *mut AqCtx, a: *const f32, m: i64, k: i64, q: *mut i8, scales: *mut f32) -> c_int;
    pub fn aq_quantize_int8_per_token_device(ctx: *mut AqCtx, d_a: *const f32, m: i64, k: i64, d_q: *mut i8,
        d_scales: *mut f32) -> c_int;
    pub fn aq_dequant_matmul_int8_f32(ctx: *mut AqCtx, act: *const f32, w: *const i8, scales: *const f32, b: i64,
        m: i64, n: i64, k: i64, out: *mut f32) -> c_int;
    pub fn aq_dequant_matmul_f16_f32(ctx: *mut AqCtx, act: *const f32, w: *const u16, b: i64, m: i64, n: i64, k: i64,
        out: *mut f32) -> c_int;
    pub fn aq_int4_matmul_f32(ctx: *mut AqCtx, a: *const f32, w_packed: *const u8, w_scales: *const f32, m: i64,
        n: i64, k: i64, out: *mut f32) -> c_int;
    pub fn aq_int4_matmul_gemv(ctx: *mut AqCtx, a: *const f32, w_packed: *const u8, w_scales: *const f32, n: i64,
        k: i64, out: *mut f32) -> c_int;
    pub fn aq_weight_only_matmul_device(ctx: *mut AqCtx, weight_format: c_int, d_act: *const f32, d_w: *const c_void,
        d_scales: *const f32, m: i64, n: i64, k: i64, d_out: *mut f32) -> c_int;
    pub fn aq_int4_matmul_gemv_q4_x_q8(ctx: *mut AqCtx, a: *const f32, w_packed: *const u8, w_scales: *const f32,
        n: i64, k: i64, out: *mut f32) -> c_int;
    pub fn aq_q4_x_q8_act_bytes(k: i64) -> usize;
    pub fn aq_int4_matmul_gemv_q4_x_q8_device(ctx: *mut AqCtx, d_a: *const f32, d_w_packed: *const u8,
        d_w_scales: *const f32, n: i64, k: i64, d_out: *mut f32, d_act: *mut c_void, d_q: *mut i8, d_qscales: *mut f32) -> c_int;
    pub fn aq_quantize_int4_q4_0(ctx: *mut AqCtx, w: *const f32, n: i64, k: i64, packed: *mut u8, scales: *mut f32) -> c_int;
    pub fn aq_dequantize_q6_k(ctx: *mut AqCtx, blocks: *const c_void, nbytes: usize, n_elements: i64, out: *mut f32) -> c_int;
    pub fn aq_dequantize_q6_k_device(ctx: *mut AqCtx, d_blocks: *const c_void, n_elements: i64, d_out: *mut f32) -> c_int;
    pub fn aq_q4_0_dequant_row(ctx: *mut AqCtx, packed: *const u8, scales: *const f32, n_rows: i64, row: i64, k: i64,
        out: *mut f32) -> c_int;
    pub fn aq_q8_0_dequant_row(ctx: *mut AqCtx, w: *const i8, scales: *const f32, n_rows: i64, row: i64, k: i64,
        out: *mut f32) -> c_int;
    pub fn aq_dequant_rows_device(ctx: *mut AqCtx, weight_format: c_int, d_table: *const c_void,
        d_scales: *const f32, n_rows: i64, d_rows: *const i64, n_out: i64, k: i64, d_out: *mut f32) -> c_int;
    pub fn aq_llama_embed(ctx: *mut AqCtx, d_table: *const f32, vocab: i64, d_tok: *const i64, hidden: i64,
        d_out: *mut f32) -> c_int;
    pub fn aq_llama_rmsnorm(ctx: *mut AqCtx, d_x: *mut f32, d_delta: *const f32, d_w: *const f32, m: i64, n: i64,
        eps: f32, d_out: *mut f32) -> c_int;
    pub fn aq_llama_silu_mul(ctx: *mut AqCtx, d_gu: *const f32, n: i64, d_out: *mut f32) -> c_int;
    pub fn aq_llama_embed_rows(ctx: *mut AqCtx, d_table: *const f32, vocab: i64, d_tok: *const i64, m: i64,
        hidden: i64, d_out: *mut f32) -> c_int;
    pub fn aq_llama_silu_mul_rows(ctx: *mut AqCtx, d_g: *const f32, d_u: *const f32, ld: i64, m: i64, n: i64,
        d_out: *mut f32) -> c_int;
    pub fn aq_llama_attn_decode(ctx: *mut AqCtx, d_qk: *const f32, d_v: *const f32, d_cos: *const f32,
        d_sin: *const f32, d_pos: *const i64, d_kcache: *mut f32, d_vcache: *mut f32, n_head: i64, n_kv: i64,
        head_dim: i64, max_seq: i64, d_out: *mut f32) -> c_int;
    pub fn aq_llama_attn_prefill(ctx: *mut AqCtx, d_q: *const f32, ldq: i64, d_k: *const f32, ldk: i64,
        d_v: *const f32, ldv: i64, d_cos: *const f32, d_sin: *const f32, index_pos: i64, m: i64, d_kcache: *mut f32,
        d_vcache: *mut f32, n_head: i64, n_kv: i64, head_dim: i64, max_seq: i64, d_out: *mut f32) -> c_int;
    pub fn aq_qmatmul_rmsnorm_f32_device(ctx: *mut AqCtx, w: *const AqQWeight, d_x: *const f32, d_delta: *const f32,
        d_norm_w: *const f32, eps: f32, k: i64, d_h_out: *mut f32, d_dst: *mut f32) -> c_int;
    pub fn aq_qmatmul_silu_mul_f32_device(ctx: *mut AqCtx, w: *const AqQWeight, d_gu: *const f32, k: i64,
        d_dst: *mut f32) -> c_int;
    pub fn aq_qmatmul2_rmsnorm_f32_device(ctx: *mut AqCtx, w1: *const AqQWeight, w2: *const AqQWeight,
        d_x: *const f32, d_delta: *const f32, d_norm_w: *const f32, eps: f32, k: i64, d_h_out: *mut f32,
        d_dst1: *mut f32, d_dst2: *mut f32) -> c_int;
    pub fn aq_llama_swiglu_pairs(ctx: *mut AqCtx, d_y: *const f32, ld: i64, m: i64, ffn: i64, d_out: *mut f32)
        -> c_int;
    pub fn aq_llama_rmsnorm_act(ctx: *mut AqCtx, d_x: *mut f32, d_delta: *const f32, d_w: *const f32, m: i64,
        n: i64, eps: f32, d_out: *mut f32, d_act: *mut c_void) -> c_int;
    pub fn aq_llama_swiglu_pairs_act(ctx: *mut AqCtx, d_y: *const f32, ld: i64, m: i64, ffn: i64, d_out: *mut f32,
        d_act: *mut c_void) -> c_int;
    pub fn aq_swiglu_fused(wtype: c_int, n: i64, k: i64) -> c_int;
    pub fn aq_llama_head_argmax_embed(ctx: *mut AqCtx, w: *const AqQWeight, d_x: *const f32, d_delta: *const f32,
        d_norm_w: *const f32, eps: f32, k: i64, d_logits: *mut f32, d_tok: *mut i64, d_pos: *mut i64,
        d_hist: *mut i64, hist_len: i64, d_table: *const f32, hidden: i64, d_x_next: *mut f32) -> c_int;
    pub fn aq_qmatmul_rmsnorm_swiglu_f32_device(ctx: *mut AqCtx, w: *const AqQWeight, d_x: *const f32,
        d_delta: *const f32, d_norm_w: *const f32, eps: f32, k: i64, d_h_out: *mut f32, d_dst: *mut f32) -> c_int;
    pub fn aq_llama_argmax(ctx: *mut AqCtx, d_x: *const f32, n: i64, d_tok: *mut i64, d_pos: *mut i64,
        d_hist: *mut i64, hist_len: i64) -> c_int;
}

/// The calling thread's last error message.
pub fn last_error() -> String {
    unsafe { std::ffi::CStr::from_ptr(aq_last_error()) }.to_string_lossy().into_owned()
}

/// `Err(message)` for a failed status, naming the call.
pub fn check(rc: c_int, what: &str) -> Result<(), String> {
    if rc == AQ_OK {
        Ok(())
    } else {
        Err(format!("{what}: {} (status {rc})", last_error()))
    }
}
