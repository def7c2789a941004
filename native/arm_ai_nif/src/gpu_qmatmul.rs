//! candle's QMatMul on one MI355X: the projection's GGUF blocks uploaded once
//! (aq_qweight_upload), `forward` = QuantizedType::matmul_t((m, k, n), lhs,
//! dst) through aq_qmatmul_f32 (host tensors) or aq_qmatmul_f32_device
//! (device pointers, on the context's stream).  Replaces the QMatMul::forward
//! calls that quantized_llama makes from llama_candle.rs:93 and :119.
use crate::aq_sys::*;
use candle_core::quantized::{GgmlDType, QTensor};
use candle_core::{bail, Result, Tensor};

/// One library context (device + HIP stream); one per model, used behind the
/// model's Mutex (llama_candle.rs:27-29), as include/aq.h requires.
pub struct GpuCtx(pub *mut AqCtx);

unsafe impl Send for GpuCtx {}

impl GpuCtx {
    pub fn new(device: i32) -> std::result::Result<Self, String> {
        let mut ctx = std::ptr::null_mut();
        check(unsafe { aq_ctx_create(device, &mut ctx) }, "aq_ctx_create")?;
        Ok(Self(ctx))
    }
    pub fn stream(&self) -> std::result::Result<*mut std::os::raw::c_void, String> {
        let mut s = std::ptr::null_mut();
        check(unsafe { aq_ctx_stream(self.0, &mut s) }, "aq_ctx_stream")?;
        Ok(s)
    }
    pub fn synchronize(&self) -> std::result::Result<(), String> {
        check(unsafe { aq_ctx_synchronize(self.0) }, "aq_ctx_synchronize")
    }
}

impl Drop for GpuCtx {
    fn drop(&mut self) {
        unsafe {
            aq_ctx_destroy(self.0);
        }
    }
}

/// GGUF dtype -> the library's type id (the same GGML numbering).
pub fn aq_type(dtype: GgmlDType) -> Option<i32> {
    Some(match dtype {
        GgmlDType::Q4_0 => AQ_TYPE_Q4_0,
        GgmlDType::Q5_0 => AQ_TYPE_Q5_0,
        GgmlDType::Q8_0 => AQ_TYPE_Q8_0,
        GgmlDType::Q2K => AQ_TYPE_Q2_K,
        GgmlDType::Q3K => AQ_TYPE_Q3_K,
        GgmlDType::Q4K => AQ_TYPE_Q4_K,
        GgmlDType::Q5K => AQ_TYPE_Q5_K,
        GgmlDType::Q6K => AQ_TYPE_Q6_K,
        _ => return None,
    })
}

/// A quantized weight of n rows (outputs) by k columns in HBM.
pub struct GpuQMatMul {
    ctx: *mut AqCtx,
    pub w: *mut AqQWeight,
    pub ty: i32,
    pub n: usize,
    pub k: usize,
}

unsafe impl Send for GpuQMatMul {}

impl GpuQMatMul {
    /// Raw GGUF blocks of an (n, k) weight, as stored in the file.
    pub fn from_blocks(ctx: &GpuCtx, ty: i32, blocks: &[u8], n: usize, k: usize) -> std::result::Result<Self, String> {
        let mut w = std::ptr::null_mut();
        check(unsafe { aq_qweight_upload(ctx.0, ty, blocks.as_ptr() as _, blocks.len(), n as i64, k as i64, &mut w) },
              "aq_qweight_upload")?;
        Ok(Self { ctx: ctx.0, w, ty, n, k })
    }

    /// After ModelWeights::from_gguf (llama_candle.rs:42): a QTensor's blocks.
    pub fn from_qtensor(ctx: &GpuCtx, qt: &QTensor) -> Result<Self> {
        let Some(ty) = aq_type(qt.dtype()) else { bail!("unsupported dtype {:?}", qt.dtype()) };
        let (n, k) = qt.shape().dims2()?;
        let bytes = qt.data()?;
        Self::from_blocks(ctx, ty, &bytes, n, k).map_err(candle_core::Error::Msg)
    }

    /// Same contract as QMatMul::forward on the CPU: xs is f32 [.., k],
    /// rank >= 2; returns f32 [.., n] on the same device.
    pub fn forward(&self, xs: &Tensor) -> Result<Tensor> {
        let dims = xs.dims();
        if dims.len() < 2 {
            bail!("input tensor has only one dimension {:?}", xs.shape())
        }
        if *dims.last().unwrap() != self.k {
            bail!("input tensor {:?} incompatible with ({}, {})", xs.shape(), self.n, self.k)
        }
        let lhs: Vec<f32> = xs.contiguous()?.flatten_all()?.to_vec1()?;
        let m = lhs.len() / self.k;
        let mut dst = vec![0f32; m * self.n];
        check(unsafe { aq_qmatmul_f32(self.ctx, self.w, lhs.as_ptr(), m as i64, self.k as i64, dst.as_mut_ptr()) },
              "aq_qmatmul_f32")
            .map_err(candle_core::Error::Msg)?;
        let mut out = dims[..dims.len() - 1].to_vec();
        out.push(self.n);
        Tensor::from_vec(dst, out, xs.device())
    }

    /// d_x f32 [m][k] -> d_y f32 [m][n], device pointers, on the context's stream.
    pub fn forward_device(&self, d_x: *const f32, m: usize, d_y: *mut f32) -> std::result::Result<(), String> {
        check(unsafe { aq_qmatmul_f32_device(self.ctx, self.w, d_x, m as i64, self.k as i64, d_y) },
              "aq_qmatmul_f32_device")
    }
}

impl Drop for GpuQMatMul {
    fn drop(&mut self) {
        unsafe {
            aq_qweight_free(self.w);
        }
    }
}
