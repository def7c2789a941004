//! ArmAI.LlamaCandle on one MI355X: the same API as the CPU bridge
//! (native/arm_ai_nif/src/llama_candle.rs) -- `LlamaResource`,
//! `load_model`, `generate_greedy`, `generate_greedy_with`,
//! `GenerateResult` -- so lib.rs's `llama_candle_load_op`,
//! `llama_candle_generate_op` and `llama_candle_stream_op` (lib.rs:1659-1699)
//! keep their bodies when this file is compiled as their `llama_candle`
//! module (feature `gpu_mi355x`).
//!
//! The model stays in HBM: every projection's GGUF blocks are uploaded once
//! (libarm_ai_amd.so repacks them), the f32 tensors (embedding table, norms)
//! are dequantized by candle once at load and copied to the device, and the
//! KV cache is preallocated for `max_seq` positions.  generate runs
//! llama_candle.rs:58-139 with device kernels only:
//!   prefill (:83-104): the prompt at offset 0 through the library's
//!     embedding rows, RMSNorm, QMatMuls, prompt attention (RoPE, KV append,
//!     causal grouped-query attention) and SiLU kernels; the first token by
//!     the device argmax;
//!   decode (:108-128): one forward per token, captured once as a HIP graph
//!     (five launches per layer: the QMatMuls form their own rms_norm /
//!     silu inputs) whose argmax feeds the next replay from device memory.
//! Tokens are read back per replay when a callback wants each token as it is
//! chosen (the stream NIF's `{:llama_token, id}`), or every 16 replays
//! otherwise; tokens after a stop token are dropped, so the output is the
//! same either way and the same as stepping one token at a time.
use crate::aq_sys::*;
use crate::gpu_qmatmul::{aq_type, GpuCtx, GpuQMatMul};
use crate::hip_sys::*;
use candle_core::quantized::gguf_file;
use candle_core::Device;
use std::fs::File;
use std::io::{Read, Seek, SeekFrom};
use std::os::raw::c_void;
use std::path::Path;
use std::sync::Mutex;

/// Replays between token read-backs when no callback asks for every token.
const GENERATE_CHUNK: usize = 16;
/// KV-cache positions (prompt + generated tokens) a loaded model can hold.
pub const DEFAULT_MAX_SEQ: usize = 4096;

pub struct Config {
    pub n_layer: usize,
    pub hidden: usize,
    pub ffn: usize,
    pub n_head: usize,
    pub n_kv: usize,
    pub vocab: usize,
    pub max_seq: usize,
    pub eps: f32,
    pub rope_base: f32,
}

impl Config {
    pub fn head_dim(&self) -> usize {
        self.hidden / self.n_head
    }
}

/// Two projections of the same input: one weight with the rows of both
/// (same GGUF type), or two.
enum Pair {
    Merged(GpuQMatMul),
    /// w1|w3 as gate and up rows in pairs of four (see upload_pair)
    Paired(GpuQMatMul),
    Split(GpuQMatMul, GpuQMatMul),
}

struct Layer {
    wqk: Pair,
    wv: GpuQMatMul,
    wo: GpuQMatMul,
    w13: Pair,
    w2: GpuQMatMul,
    attn_norm: DeviceBuf,
    ffn_norm: DeviceBuf,
}

/// The decode step's device state (fixed addresses: the graph is captured over them).
struct Step {
    pos: DeviceBuf,
    tok: DeviceBuf,
    hist: DeviceBuf,
    ra: DeviceBuf,
    rb: DeviceBuf,
    qk: DeviceBuf,
    v: DeviceBuf,
    att: DeviceBuf,
    o: DeviceBuf,
    gu: DeviceBuf,
    d: DeviceBuf,
    logits: DeviceBuf,
    graph: hipGraphExec_t,
}

/// The prompt's buffers, for `rows` positions (grown on demand).
struct PromptBufs {
    rows: usize,
    tok: DeviceBuf,
    x: DeviceBuf,
    h: DeviceBuf,
    qk: DeviceBuf,
    v: DeviceBuf,
    y: DeviceBuf,
    o: DeviceBuf,
    gu: DeviceBuf,
    a: DeviceBuf,
    d: DeviceBuf,
    last: DeviceBuf,
}

pub struct GpuLlama {
    cfg: Config,
    layers: Vec<Layer>,
    output: GpuQMatMul,
    tok_emb: DeviceBuf,
    norm: DeviceBuf,
    cos: DeviceBuf,
    sin: DeviceBuf,
    kcache: DeviceBuf,
    vcache: DeviceBuf,
    step: Option<Step>,
    prompt: Option<PromptBufs>,
    pinned: PinnedBuf,
    stream: hipStream_t,
    ctx: GpuCtx, // last: the library context outlives every weight and buffer above
}

unsafe impl Send for GpuLlama {}

/// Wraps the loaded model; the Mutex serialises calls (llama_candle.rs:27-29).
pub struct LlamaResource {
    pub model: Mutex<GpuLlama>,
}

unsafe impl Send for LlamaResource {}
unsafe impl Sync for LlamaResource {}

pub struct GenerateResult {
    pub tokens: Vec<u32>,
    pub prefill_us: u64,
    pub decode_us: u64,
}

// ------------------------------------------------------------------ load
struct Gguf {
    file: File,
    content: gguf_file::Content,
}

impl Gguf {
    fn u(&self, key: &str) -> Result<usize, String> {
        let v = self.content.metadata.get(key).ok_or_else(|| format!("gguf: missing {key}"))?;
        v.to_u32().map(|x| x as usize).map_err(|e| format!("gguf {key}: {e}"))
    }
    fn f(&self, key: &str) -> Option<f32> {
        self.content.metadata.get(key).and_then(|v| v.to_f32().ok())
    }
    fn has(&self, name: &str) -> bool {
        self.content.tensor_infos.contains_key(name)
    }
    /// (dtype, (rows, cols), the tensor's bytes as stored)
    fn raw(&mut self, name: &str) -> Result<(candle_core::quantized::GgmlDType, (usize, usize), Vec<u8>), String> {
        let ti = self.content.tensor_infos.get(name).ok_or_else(|| format!("gguf: no tensor {name}"))?;
        let dims = ti.shape.dims();
        if dims.len() != 2 {
            return Err(format!("{name}: expected a 2-d tensor, got {dims:?}"));
        }
        let bytes = ti.shape.elem_count() / ti.ggml_dtype.block_size() * ti.ggml_dtype.type_size();
        let mut buf = vec![0u8; bytes];
        self.file
            .seek(SeekFrom::Start(self.content.tensor_data_offset + ti.offset))
            .and_then(|_| self.file.read_exact(&mut buf))
            .map_err(|e| format!("{name}: {e}"))?;
        Ok((ti.ggml_dtype, (dims[0], dims[1]), buf))
    }
    /// A tensor dequantized to f32 by candle (embedding table, norm weights).
    fn f32(&mut self, name: &str) -> Result<Vec<f32>, String> {
        let qt = self.content.tensor(&mut self.file, name, &Device::Cpu).map_err(|e| format!("{name}: {e}"))?;
        qt.dequantize(&Device::Cpu)
            .and_then(|t| t.flatten_all())
            .and_then(|t| t.to_vec1::<f32>())
            .map_err(|e| format!("{name}: {e}"))
    }
}

fn upload(ctx: &GpuCtx, g: &mut Gguf, name: &str) -> Result<GpuQMatMul, String> {
    let (dt, (n, k), bytes) = g.raw(name)?;
    let ty = aq_type(dt).ok_or_else(|| format!("{name}: unsupported dtype {dt:?}"))?;
    GpuQMatMul::from_blocks(ctx, ty, &bytes, n, k)
}

/// wq|wk, w1|w3: one weight of both tensors' rows when they share a type,
/// concatenated -- except w1|w3 (`swiglu`) where the decode matvec forms
/// silu(g) * u in its own launch (aq_swiglu_fused): there one weight of gate
/// and up rows in pairs of four (row 8b + j is gate row 4b + j for j < 4, up
/// row 4b + j - 4 after; aq_qmatmul_rmsnorm_swiglu_f32_device,
/// aq_llama_swiglu_pairs), as arm_ai_amd.llama.swiglu_pair_rows builds it.
fn upload_pair(ctx: &GpuCtx, g: &mut Gguf, a: &str, b: &str, swiglu: bool) -> Result<Pair, String> {
    let (da, (na, ka), mut ba) = g.raw(a)?;
    let (db, (nb, kb), bb) = g.raw(b)?;
    let ta = aq_type(da).ok_or_else(|| format!("{a}: unsupported dtype {da:?}"))?;
    let tb = aq_type(db).ok_or_else(|| format!("{b}: unsupported dtype {db:?}"))?;
    if ta != tb || ka != kb {
        return Ok(Pair::Split(GpuQMatMul::from_blocks(ctx, ta, &ba, na, ka)?,
                              GpuQMatMul::from_blocks(ctx, tb, &bb, nb, kb)?));
    }
    if swiglu && na == nb && na % 4 == 0 && unsafe { aq_swiglu_fused(ta, (na + nb) as i64, ka as i64) } == 1 {
        let four = ba.len() / na * 4;  // the bytes of four rows
        let mut out = Vec::with_capacity(ba.len() + bb.len());
        for (x, y) in ba.chunks(four).zip(bb.chunks(four)) {
            out.extend_from_slice(x);
            out.extend_from_slice(y);
        }
        return Ok(Pair::Paired(GpuQMatMul::from_blocks(ctx, ta, &out, na + nb, ka)?));
    }
    ba.extend_from_slice(&bb);
    Ok(Pair::Merged(GpuQMatMul::from_blocks(ctx, ta, &ba, na + nb, ka)?))
}

/// Load a GGUF Llama-family model (llama_candle.rs:35-48) onto GPU 0.
pub fn load_model(path: &str) -> Result<LlamaResource, String> {
    load_model_on(path, 0, DEFAULT_MAX_SEQ)
}

pub fn load_model_on(path: &str, device: i32, max_seq: usize) -> Result<LlamaResource, String> {
    let mut file = File::open(Path::new(path)).map_err(|e| format!("open {} failed: {}", path, e))?;
    let content = gguf_file::Content::read(&mut file).map_err(|e| format!("gguf read failed: {}", e))?;
    let mut g = Gguf { file, content };
    let n_head = g.u("llama.attention.head_count")?;
    let n_kv = if g.content.metadata.contains_key("llama.attention.head_count_kv") {
        g.u("llama.attention.head_count_kv")?
    } else {
        n_head
    };
    let emb = g.content.tensor_infos.get("token_embd.weight").ok_or("gguf: no token_embd.weight")?;
    let (vocab, hidden) = (emb.shape.dims()[0], emb.shape.dims()[1]);
    let ffn = g.content.tensor_infos.get("blk.0.ffn_gate.weight").ok_or("gguf: no blk.0.ffn_gate.weight")?.shape.dims()[0];
    let cfg = Config {
        n_layer: g.u("llama.block_count")?,
        hidden,
        ffn,
        n_head,
        n_kv,
        vocab,
        max_seq,
        eps: g.f("llama.attention.layer_norm_rms_epsilon").ok_or("gguf: missing llama.attention.layer_norm_rms_epsilon")?,
        rope_base: g.f("llama.rope.freq_base").unwrap_or(10000.0),
    };
    if g.u("llama.embedding_length")? != hidden || hidden % n_head != 0 || n_head % n_kv != 0 {
        return Err(format!("inconsistent llama shape: hidden {hidden}, heads {n_head} / {n_kv}"));
    }

    let ctx = GpuCtx::new(device)?;
    let stream = ctx.stream()?;
    let mut layers = Vec::with_capacity(cfg.n_layer);
    for i in 0..cfg.n_layer {
        let p = |s: &str| format!("blk.{i}.{s}.weight");
        layers.push(Layer {
            wqk: upload_pair(&ctx, &mut g, &p("attn_q"), &p("attn_k"), false)?,
            wv: upload(&ctx, &mut g, &p("attn_v"))?,
            wo: upload(&ctx, &mut g, &p("attn_output"))?,
            w13: upload_pair(&ctx, &mut g, &p("ffn_gate"), &p("ffn_up"), true)?,
            w2: upload(&ctx, &mut g, &p("ffn_down"))?,
            attn_norm: DeviceBuf::from_slice(&g.f32(&p("attn_norm"))?, stream)?,
            ffn_norm: DeviceBuf::from_slice(&g.f32(&p("ffn_norm"))?, stream)?,
        });
    }
    // candle ties the output head to the embedding when output.weight is absent
    let output = if g.has("output.weight") { upload(&ctx, &mut g, "output.weight")? } else { upload(&ctx, &mut g, "token_embd.weight")? };
    let tok_emb = DeviceBuf::from_slice(&g.f32("token_embd.weight")?, stream)?;
    let norm = DeviceBuf::from_slice(&g.f32("output_norm.weight")?, stream)?;

    // precompute_freqs_cis: theta_i = base^(-2i/hd), cos / sin [max_seq][hd/2], f32
    let hd = cfg.head_dim();
    let theta: Vec<f32> = (0..hd).step_by(2).map(|i| 1f32 / cfg.rope_base.powf(i as f32 / hd as f32)).collect();
    let mut cos = Vec::with_capacity(max_seq * hd / 2);
    let mut sin = Vec::with_capacity(max_seq * hd / 2);
    for p in 0..max_seq {
        for t in &theta {
            let a = p as f32 * t;
            cos.push(a.cos());
            sin.push(a.sin());
        }
    }
    let cache_bytes = cfg.n_layer * cfg.n_kv * max_seq * hd * 4;
    let mut model = GpuLlama {
        layers,
        output,
        tok_emb,
        norm,
        cos: DeviceBuf::from_slice(&cos, stream)?,
        sin: DeviceBuf::from_slice(&sin, stream)?,
        kcache: DeviceBuf::new(cache_bytes)?,
        vcache: DeviceBuf::new(cache_bytes)?,
        step: None,
        prompt: None,
        pinned: PinnedBuf::new(8 * max_seq)?,
        stream,
        cfg,
        ctx,
    };
    // a prompt's buffers up front (llama.cpp reserves its compute buffers at
    // context creation), so that the first prompt of up to 512 tokens does
    // not allocate
    let reserve = model.cfg.max_seq.min(512);
    model.prompt_bufs(reserve)?;
    Ok(LlamaResource { model: Mutex::new(model) })
}

// ------------------------------------------------------------------ forward
fn is_norm2(w: &GpuQMatMul) -> bool {
    w.ty == AQ_TYPE_Q4_K || w.ty == AQ_TYPE_Q6_K
}

impl GpuLlama {
    fn c(&self) -> *mut AqCtx {
        self.ctx.0
    }

    fn cache_at(&self, buf: &DeviceBuf, layer: usize) -> *mut f32 {
        buf.f32_at(layer * self.cfg.n_kv * self.cfg.max_seq * self.cfg.head_dim())
    }

    fn h2d_i64(&self, dst: *mut i64, v: i64) -> Result<(), String> {
        // through pinned memory, finished before the pinned word is reused
        unsafe { *(self.pinned.ptr as *mut i64) = v };
        hip_check(unsafe { hipMemcpyAsync(dst as *mut c_void, self.pinned.ptr, 8, hipMemcpyHostToDevice, self.stream) },
                  "hipMemcpyAsync")?;
        hip_check(unsafe { hipStreamSynchronize(self.stream) }, "hipStreamSynchronize")
    }

    fn d2h_i64(&self, src: *const i64, n: usize) -> Result<Vec<i64>, String> {
        hip_check(unsafe { hipMemcpyAsync(self.pinned.ptr, src as *const c_void, 8 * n, hipMemcpyDeviceToHost,
                                          self.stream) }, "hipMemcpyAsync")?;
        hip_check(unsafe { hipStreamSynchronize(self.stream) }, "hipStreamSynchronize")?;
        Ok(self.pinned.i64_slice(n).to_vec())
    }

    fn prompt_bufs(&mut self, rows: usize) -> Result<(), String> {
        if self.prompt.as_ref().map_or(false, |p| p.rows >= rows) {
            return Ok(());
        }
        let c = &self.cfg;
        let (hd, f) = (c.head_dim(), 4);
        let nb = |w: usize| DeviceBuf::new(rows * w * f);
        self.prompt = Some(PromptBufs {
            rows,
            tok: DeviceBuf::new(rows * 8)?,
            x: nb(c.hidden)?,
            h: nb(c.hidden)?,
            qk: nb((c.n_head + c.n_kv) * hd)?,
            v: nb(c.n_kv * hd)?,
            y: nb(c.n_head * hd)?,
            o: nb(c.hidden)?,
            gu: nb(2 * c.ffn)?,
            a: nb(c.ffn)?,
            d: nb(c.hidden)?,
            last: DeviceBuf::new(c.hidden * f)?,
        });
        Ok(())
    }

    /// ModelWeights::forward(&tokens[1, n], index_pos) on the device; the
    /// logits of the last position go to `logits` (device, vocab f32).
    fn forward_prompt(&mut self, tokens: &[u32], index_pos: usize, logits: *mut f32) -> Result<(), String> {
        let n = tokens.len();
        self.prompt_bufs(n)?;
        let cfg = &self.cfg;
        let (h_, kv, hd) = (cfg.n_head, cfg.n_kv, cfg.head_dim());
        let c = self.c();
        let p = self.prompt.as_ref().unwrap();
        let ids: Vec<i64> = tokens.iter().map(|&t| t as i64).collect();
        hip_check(unsafe { hipMemcpyAsync(p.tok.ptr, ids.as_ptr() as *const c_void, 8 * n, hipMemcpyHostToDevice,
                                          self.stream) }, "hipMemcpyAsync")?;
        hip_check(unsafe { hipStreamSynchronize(self.stream) }, "hipStreamSynchronize")?;
        let (n64, hid) = (n as i64, cfg.hidden as i64);
        check(unsafe { aq_llama_embed_rows(c, self.tok_emb.f32(), cfg.vocab as i64, p.tok.i64(), n64, hid, p.x.f32()) },
              "embed")?;
        let mut delta: *const f32 = std::ptr::null();
        for (li, l) in self.layers.iter().enumerate() {
            check(unsafe { aq_llama_rmsnorm(c, p.x.f32(), delta, l.attn_norm.f32(), n64, hid, cfg.eps, p.h.f32()) },
                  "rmsnorm")?;
            let (q, ldq, k, ldk) = match &l.wqk {
                Pair::Merged(w) | Pair::Paired(w) => {  // (wq|wk is never paired)
                    w.forward_device(p.h.f32(), n, p.qk.f32())?;
                    (p.qk.f32(), (h_ + kv) * hd, p.qk.f32_at(h_ * hd), (h_ + kv) * hd)
                }
                Pair::Split(wq, wk) => {
                    wq.forward_device(p.h.f32(), n, p.qk.f32())?;
                    wk.forward_device(p.h.f32(), n, p.qk.f32_at(n * h_ * hd))?;
                    (p.qk.f32(), h_ * hd, p.qk.f32_at(n * h_ * hd), kv * hd)
                }
            };
            l.wv.forward_device(p.h.f32(), n, p.v.f32())?;
            check(unsafe {
                aq_llama_attn_prefill(c, q, ldq as i64, k, ldk as i64, p.v.f32(), (kv * hd) as i64, self.cos.f32(),
                                      self.sin.f32(), index_pos as i64, n64, self.cache_at(&self.kcache, li),
                                      self.cache_at(&self.vcache, li), h_ as i64, kv as i64, hd as i64,
                                      cfg.max_seq as i64, p.y.f32())
            }, "attn_prefill")?;
            l.wo.forward_device(p.y.f32(), n, p.o.f32())?;
            check(unsafe { aq_llama_rmsnorm(c, p.x.f32(), p.o.f32(), l.ffn_norm.f32(), n64, hid, cfg.eps, p.h.f32()) },
                  "rmsnorm")?;
            match &l.w13 {
                Pair::Paired(w) => {  // gate and up rows in pairs of four
                    w.forward_device(p.h.f32(), n, p.gu.f32())?;
                    check(unsafe { aq_llama_swiglu_pairs(c, p.gu.f32(), (2 * cfg.ffn) as i64, n64, cfg.ffn as i64,
                                                         p.a.f32()) }, "swiglu_pairs")?;
                }
                Pair::Merged(w) => {
                    w.forward_device(p.h.f32(), n, p.gu.f32())?;
                    check(unsafe { aq_llama_silu_mul_rows(c, p.gu.f32(), p.gu.f32_at(cfg.ffn), (2 * cfg.ffn) as i64,
                                                          n64, cfg.ffn as i64, p.a.f32()) }, "silu_mul")?;
                }
                Pair::Split(w1, w3) => {
                    w1.forward_device(p.h.f32(), n, p.gu.f32())?;
                    w3.forward_device(p.h.f32(), n, p.gu.f32_at(n * cfg.ffn))?;
                    check(unsafe { aq_llama_silu_mul_rows(c, p.gu.f32(), p.gu.f32_at(n * cfg.ffn), cfg.ffn as i64,
                                                          n64, cfg.ffn as i64, p.a.f32()) }, "silu_mul")?;
                }
            }
            l.w2.forward_device(p.a.f32(), n, p.d.f32())?;
            delta = p.d.f32();
        }
        let last = (n - 1) * cfg.hidden;
        check(unsafe { aq_llama_rmsnorm(c, p.x.f32_at(last), p.d.f32_at(last), self.norm.f32(), 1, hid, cfg.eps,
                                        p.last.f32()) }, "rmsnorm")?;
        self.output.forward_device(p.last.f32(), 1, logits)
    }

    fn alloc_step(&mut self) -> Result<(), String> {
        if self.step.is_some() {
            return Ok(());
        }
        let c = &self.cfg;
        let hd = c.head_dim();
        let f = |n: usize| DeviceBuf::new(n * 4);
        self.step = Some(Step {
            pos: DeviceBuf::new(8)?,
            tok: DeviceBuf::new(8)?,
            hist: DeviceBuf::new(8 * c.max_seq)?,
            ra: f(c.hidden)?,
            rb: f(c.hidden)?,
            qk: f((c.n_head + c.n_kv) * hd)?,
            v: f(c.n_kv * hd)?,
            att: f(c.n_head * hd)?,
            o: f(c.hidden)?,
            gu: f(2 * c.ffn)?,
            d: f(c.hidden)?,
            logits: f(c.vocab)?,
            graph: std::ptr::null_mut(),
        });
        Ok(())
    }

    /// One decode step for the token at step.tok, position step.pos (both in
    /// device memory): logits, then the next token into step.tok and
    /// step.hist[pos], and pos + 1.  Enqueues only; capturable.
    fn decode_step(&self) -> Result<(), String> {
        let cfg = &self.cfg;
        let s = self.step.as_ref().unwrap();
        let c = self.c();
        let (h_, kv, hd) = (cfg.n_head, cfg.n_kv, cfg.head_dim());
        let hid = cfg.hidden as i64;
        let mm_norm = |w: &GpuQMatMul, x: *const f32, delta: *const f32, norm: *const f32, out: *mut f32,
                       h_out: *mut f32| {
            check(unsafe { aq_qmatmul_rmsnorm_f32_device(c, w.w, x, delta, norm, cfg.eps, w.k as i64, h_out, out) },
                  "qmatmul rmsnorm")
        };
        let (cur, other) = (s.ra.f32(), s.rb.f32());
        let mut delta: *const f32 = std::ptr::null();
        for (li, l) in self.layers.iter().enumerate() {
            let an = l.attn_norm.f32();
            match &l.wqk {
                Pair::Merged(w) if is_norm2(w) && is_norm2(&l.wv) => check(unsafe {
                    aq_qmatmul2_rmsnorm_f32_device(c, w.w, l.wv.w, cur, delta, an, cfg.eps, hid, other, s.qk.f32(),
                                                   s.v.f32())
                }, "qmatmul2 rmsnorm")?,
                Pair::Merged(w) | Pair::Paired(w) => {  // (wq|wk is never paired)
                    mm_norm(w, cur, delta, an, s.qk.f32(), other)?;
                    mm_norm(&l.wv, cur, delta, an, s.v.f32(), std::ptr::null_mut())?;
                }
                Pair::Split(wq, wk) => {
                    mm_norm(wq, cur, delta, an, s.qk.f32(), other)?;
                    mm_norm(wk, cur, delta, an, s.qk.f32_at(h_ * hd), std::ptr::null_mut())?;
                    mm_norm(&l.wv, cur, delta, an, s.v.f32(), std::ptr::null_mut())?;
                }
            }
            check(unsafe {
                aq_llama_attn_decode(c, s.qk.f32(), s.v.f32(), self.cos.f32(), self.sin.f32(), s.pos.i64(),
                                     self.cache_at(&self.kcache, li), self.cache_at(&self.vcache, li), h_ as i64,
                                     kv as i64, hd as i64, cfg.max_seq as i64, s.att.f32())
            }, "attn_decode")?;
            l.wo.forward_device(s.att.f32(), 1, s.o.f32())?;
            let fnm = l.ffn_norm.f32();
            match &l.w13 {
                Pair::Paired(w) => {  // silu(g) * u formed by the w1|w3 launch, w2 on it
                    check(unsafe { aq_qmatmul_rmsnorm_swiglu_f32_device(c, w.w, other, s.o.f32(), fnm, cfg.eps,
                                                                        cfg.hidden as i64, cur, s.gu.f32()) },
                          "qmatmul rmsnorm swiglu")?;
                    l.w2.forward_device(s.gu.f32(), 1, s.d.f32())?;
                }
                _ => {  // [g | u], silu(g) * u formed by the w2 launch
                    match &l.w13 {
                        Pair::Split(w1, w3) => {
                            mm_norm(w1, other, s.o.f32(), fnm, s.gu.f32(), cur)?;
                            mm_norm(w3, other, s.o.f32(), fnm, s.gu.f32_at(cfg.ffn), std::ptr::null_mut())?;
                        }
                        Pair::Merged(w) | Pair::Paired(w) => mm_norm(w, other, s.o.f32(), fnm, s.gu.f32(), cur)?,
                    }
                    check(unsafe { aq_qmatmul_silu_mul_f32_device(c, l.w2.w, s.gu.f32(), cfg.ffn as i64, s.d.f32()) },
                          "qmatmul silu")?;
                }
            }
            // the residual x + wo + w2 is now cur + d: the next layer's norm
            // input, with `other` again receiving the sum
            delta = s.d.f32();
        }
        // the head, the greedy pick (token, history, position) and the picked
        // token's embedding row into `ra`, the next step's input
        check(unsafe {
            aq_llama_head_argmax_embed(c, self.output.w, cur, delta, self.norm.f32(), cfg.eps, hid, s.logits.f32(),
                                       s.tok.i64(), s.pos.i64(), s.hist.i64(), cfg.max_seq as i64,
                                       self.tok_emb.f32(), hid, s.ra.f32())
        }, "head argmax embed")
    }

    /// Capture the decode step once (after one eager run at the last cache
    /// slot: first-call set-up stays out of the graph; a step writes only its
    /// own position's k, v).
    fn ensure_graph(&mut self) -> Result<hipGraphExec_t, String> {
        self.alloc_step()?;
        if !self.step.as_ref().unwrap().graph.is_null() {
            return Ok(self.step.as_ref().unwrap().graph);
        }
        self.h2d_i64(self.step.as_ref().unwrap().pos.i64(), self.cfg.max_seq as i64 - 1)?;
        self.decode_step()?;
        self.ctx.synchronize()?;
        hip_check(unsafe { hipStreamBeginCapture(self.stream, hipStreamCaptureModeThreadLocal) }, "begin capture")?;
        let r = self.decode_step();
        let mut graph: hipGraph_t = std::ptr::null_mut();
        let e = unsafe { hipStreamEndCapture(self.stream, &mut graph) };
        r?;
        hip_check(e, "end capture")?;
        let mut exec: hipGraphExec_t = std::ptr::null_mut();
        let e = unsafe { hipGraphInstantiate(&mut exec, graph, std::ptr::null_mut(), std::ptr::null_mut(), 0) };
        unsafe { hipGraphDestroy(graph) };
        hip_check(e, "graph instantiate")?;
        self.step.as_mut().unwrap().graph = exec;
        Ok(exec)
    }
}

impl Drop for GpuLlama {
    fn drop(&mut self) {
        let _ = self.ctx.synchronize();
        if let Some(s) = &self.step {
            if !s.graph.is_null() {
                unsafe { hipGraphExecDestroy(s.graph) };
            }
        }
    }
}

// ------------------------------------------------------------------ generate
/// Greedy decode (llama_candle.rs:51-65): up to `max_new` tokens after the
/// prompt, stopping after a token in `stop_tokens` (kept in the output).
pub fn generate_greedy(res: &LlamaResource, prompt: &[u32], max_new: usize, stop_tokens: &[u32])
                       -> Result<GenerateResult, String> {
    generate_chunked(res, prompt, max_new, stop_tokens, &mut |_| {}, GENERATE_CHUNK)
}

/// Like `generate_greedy`, calling `on_token` with each token as soon as it is
/// chosen (llama_candle.rs:67-139): one token read back per replay.
pub fn generate_greedy_with(res: &LlamaResource, prompt: &[u32], max_new: usize, stop_tokens: &[u32],
                            on_token: &mut dyn FnMut(u32)) -> Result<GenerateResult, String> {
    generate_chunked(res, prompt, max_new, stop_tokens, on_token, 1)
}

fn generate_chunked(res: &LlamaResource, prompt: &[u32], max_new: usize, stop_tokens: &[u32],
                    on_token: &mut dyn FnMut(u32), chunk: usize) -> Result<GenerateResult, String> {
    if max_new == 0 || prompt.is_empty() {
        return Ok(GenerateResult { tokens: Vec::new(), prefill_us: 0, decode_us: 0 });
    }
    let mut model = res.model.lock().map_err(|e| format!("lock: {}", e))?;
    let max_seq = model.cfg.max_seq;
    if prompt.len() + max_new - 1 > max_seq {
        return Err(format!("prompt ({}) + max_new ({}) exceeds the {} cached positions", prompt.len(), max_new, max_seq));
    }
    let graph = model.ensure_graph()?;
    let (tok, pos, hist, logits, ra) = {
        let s = model.step.as_ref().unwrap();
        (s.tok.i64(), s.pos.i64(), s.hist.i64(), s.logits.f32(), s.ra.f32())
    };

    let prefill_start = std::time::Instant::now();
    model.forward_prompt(prompt, 0, logits)?;
    // the first new token by the device argmax: hist[len - 1], then pos = len
    model.h2d_i64(pos, prompt.len() as i64 - 1)?;
    check(unsafe { aq_llama_argmax(model.c(), logits, model.cfg.vocab as i64, tok, pos, hist, max_seq as i64) },
          "argmax")?;
    // the step's input: the token's embedding row (each replay then leaves the next one's)
    check(unsafe { aq_llama_embed(model.c(), model.tok_emb.f32(), model.cfg.vocab as i64, tok,
                                  model.cfg.hidden as i64, ra) }, "embed")?;
    let mut next = model.d2h_i64(tok, 1)?[0] as u32;
    let prefill_us = prefill_start.elapsed().as_micros() as u64;
    let mut generated = vec![next];
    on_token(next);

    let decode_start = std::time::Instant::now();
    let mut offset = prompt.len();
    let mut done = stop_tokens.contains(&next);
    while !done && generated.len() < max_new {
        let n = chunk.min(max_new - generated.len());
        for _ in 0..n {
            hip_check(unsafe { hipGraphLaunch(graph, model.stream) }, "hipGraphLaunch")?;
        }
        let toks = model.d2h_i64(unsafe { hist.add(offset) }, n)?;
        for t in toks {
            next = t as u32;
            generated.push(next);
            on_token(next);
            if stop_tokens.contains(&next) {
                done = true;
                break;
            }
        }
        offset += n;
    }
    let decode_us = decode_start.elapsed().as_micros() as u64;
    Ok(GenerateResult { tokens: generated, prefill_us, decode_us })
}
