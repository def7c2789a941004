"""The call sites of the quantized matmuls: a Llama decoder driven like ArmAI.LlamaCandle.

In the reference, ``llama_candle_generate_op`` (native/arm_ai_nif/src/llama_candle.rs:58-139)
runs candle-transformers' ``quantized_llama::ModelWeights::forward`` once over the
prompt at offset 0 (prefill, :93) and then once per generated token (decode,
:119), picking each next token by a first-maximum argmax (:154-176).  Each
forward makes 7 ``QMatMul::forward`` calls per layer (wq, wk, wv, wo, w1, w3,
w2) plus the output head: for TinyLlama-1.1B that is 155 quantized matmuls per
token, which is where the time goes.

Here those 155 calls are this library's GPU QMatMuls (the product, through the
C ABI, device pointers, on the context's HIP stream).  The operations between
them (token embedding, RMSNorm, interleaved RoPE, grouped-query attention with
a KV cache, SiLU gate, residual adds, argmax) are the library's f32 glue
kernels on the same stream (k_decode.hip, k_attn.hip), so the whole forward
stays on the GPU; torch only allocates the device buffers.  They follow
candle-transformers 0.8.4
``quantized_llama`` (a registry dependency of native/arm_ai_nif/Cargo.lock, not
vendored in the reference):

* ``forward(x, index_pos)``: embedding; per layer
  ``h = x + wo(attn(rms_norm(x)))``, ``x = h + w2(silu(w1(n)) * w3(n))`` with
  ``n = rms_norm(h)``; final ``rms_norm``; the output head on the last position
  only.
* attention: q, k, v reshaped to heads, ``rope_i`` (interleaved pairs) with
  ``theta_i = base^(-2i/head_dim)`` at positions ``index_pos ..``, the new k, v
  appended to the cache, k, v repeated ``n_head / n_kv_head`` times,
  ``softmax(q k^T / sqrt(head_dim))`` with the causal mask ``j > i`` when more
  than one position is fed, ``att v``, heads merged, wo.
* ``rms_norm(x) = x / sqrt(mean(x^2) + eps) * w``; ``silu(x) = x / (1 + e^-x)``.

The decode step (one token at a given position) can be captured once into a
HIP graph and replayed per token (``Llama.generate(..., graph=True)``).  That
step uses the decode forms of the glue kernels (embedding, residual add +
RMSNorm, RoPE + KV-cache write + grouped-query attention with the context
split over workgroups in one launch, and a first-maximum argmax that writes
the next token and advances the device-side position) around the GPU
QMatMuls, whose matvec forms its own input where that input is
rms_norm(x + delta) or silu(g) * u: 5 launches per layer (wq|wk and wv share one).  Projections that share an input and a
type are uploaded as one weight (wq|wk, w1|w3: rows concatenated), so each
pair is one matmul launch.  The KV cache, the RoPE tables and every
intermediate buffer are preallocated for ``max_seq`` positions, so every
replay has the same shapes, and because the step feeds its own next token and
position, several steps can be replayed back to back without a host round
trip.
"""
from __future__ import annotations

import contextlib
import ctypes
import time
from dataclasses import dataclass, field

import numpy as np

from . import synth
from .qmatmul import Context, GgmlDType, QMatMul, QTensor



@dataclass
class LlamaConfig:
    """Hyper-parameters read from GGUF ``llama.*`` metadata in the reference."""

    n_layer: int = 22
    hidden: int = 2048
    ffn: int = 5632
    n_head: int = 32
    n_kv_head: int = 4
    vocab: int = 32000
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    max_seq: int = 1024

    @property
    def head_dim(self) -> int:
        return self.hidden // self.n_head


# TinyLlama-1.1B Q4_K_M tensor types (config 2): Q4_K everywhere except attn_v,
# ffn_down in every other layer (11 of 22) and the output head, which are Q6_K.
def tinyllama_q4km_types(cfg: LlamaConfig, layer: int) -> dict[str, int]:
    return {
        "wq": synth.TYPE_Q4_K,
        "wk": synth.TYPE_Q4_K,
        "wv": synth.TYPE_Q6_K,
        "wo": synth.TYPE_Q4_K,
        "w1": synth.TYPE_Q4_K,
        "w3": synth.TYPE_Q4_K,
        "w2": synth.TYPE_Q6_K if layer % 2 == 1 else synth.TYPE_Q4_K,
    }


# The Q5_K_M files of the same models: Q5_K where Q4_K_M has Q4_K.
def tinyllama_q5km_types(cfg: LlamaConfig, layer: int) -> dict[str, int]:
    return {name: (synth.TYPE_Q5_K if t == synth.TYPE_Q4_K else t)
            for name, t in tinyllama_q4km_types(cfg, layer).items()}


def smollm_135m_config(max_seq: int = 1024) -> LlamaConfig:
    """SmolLM-135M's shape (one of the models the reference's chatbot loads,
    examples/chatbot/README.md:36-37): 30 layers, hidden 576, FFN 1536, 9
    query heads over 3 kv heads (head_dim 64), vocabulary 49152, output head
    tied to the token embedding."""
    return LlamaConfig(n_layer=30, hidden=576, ffn=1536, n_head=9, n_kv_head=3, vocab=49152, max_seq=max_seq)


def gguf_fallback_type(t: int, k: int) -> int:
    """The type llama.cpp's quantizer writes for a tensor whose rows (k) are
    not a multiple of 256, which no K-quant block can hold: Q4_K -> Q5_0,
    Q6_K -> Q8_0 (Q2_K / Q3_K -> IQ4_NL and Q5_K -> Q5_1 have no kernels
    here and are not produced by the mixes below)."""
    if k % 256 == 0:
        return t
    fb = {synth.TYPE_Q4_K: synth.TYPE_Q5_0, synth.TYPE_Q6_K: synth.TYPE_Q8_0}
    if t not in fb:
        raise ValueError(f"no fallback type for GGML type {t} at k={k}")
    return fb[t]


# The Q4_K_M mix of a model whose hidden width is not a multiple of 256
# (SmolLM-135M: 576): every projection that reads the hidden state (wq, wk,
# wv, wo, w1, w3) takes its fallback type, w2 (k = ffn = 1536) keeps its
# K-quant.
def fallback_q4km_types(cfg: LlamaConfig, layer: int) -> dict[str, int]:
    shapes = weight_shapes(cfg)
    return {name: gguf_fallback_type(t, shapes[name][1]) for name, t in tinyllama_q4km_types(cfg, layer).items()}


def weight_shapes(cfg: LlamaConfig) -> dict[str, tuple[int, int]]:
    """(n, k) of each per-layer projection (candle's (out, in))."""
    hd = cfg.head_dim
    return {
        "wq": (cfg.n_head * hd, cfg.hidden),
        "wk": (cfg.n_kv_head * hd, cfg.hidden),
        "wv": (cfg.n_kv_head * hd, cfg.hidden),
        "wo": (cfg.hidden, cfg.n_head * hd),
        "w1": (cfg.ffn, cfg.hidden),
        "w3": (cfg.ffn, cfg.hidden),
        "w2": (cfg.hidden, cfg.ffn),
    }


@dataclass
class HostWeights:
    """A model's weights in host memory: GGUF blocks for the projections,
    f32 for the embedding table and the norm weights."""

    cfg: LlamaConfig
    layers: list[dict[str, QTensor]] = field(default_factory=list)
    attn_norm: list[np.ndarray] = field(default_factory=list)
    ffn_norm: list[np.ndarray] = field(default_factory=list)
    tok_embeddings: np.ndarray | None = None
    norm: np.ndarray | None = None
    output: QTensor | None = None


def synthetic_weights(cfg: LlamaConfig, seed: int = 0, types=tinyllama_q4km_types,
                      output_type: int = synth.TYPE_Q6_K, unit: bool = False) -> HostWeights:
    """Random weights of the given architecture (block value distributions of
    arm_ai_amd.synth.make_weight, or with unit=True synth.make_weight_unit,
    whose values are centred and scaled by 1/sqrt(k) so activations stay of
    order one through every layer; embedding ~ N(0, 1); norm weights ~
    1 + N(0, 0.05))."""
    rng = np.random.default_rng(seed)
    hw = HostWeights(cfg)
    shapes = weight_shapes(cfg)
    make = synth.make_weight_unit if unit else synth.make_weight
    for layer in range(cfg.n_layer):
        t = types(cfg, layer)
        qt = {}
        for name, (n, k) in shapes.items():
            w = make(t[name], n, k, rng=rng)
            qt[name] = QTensor(t[name], (n, k), w.blocks)
        hw.layers.append(qt)
        hw.attn_norm.append((1.0 + 0.05 * rng.standard_normal(cfg.hidden)).astype(np.float32))
        hw.ffn_norm.append((1.0 + 0.05 * rng.standard_normal(cfg.hidden)).astype(np.float32))
    hw.tok_embeddings = rng.standard_normal((cfg.vocab, cfg.hidden), dtype=np.float32)
    hw.norm = (1.0 + 0.05 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    w = make(output_type, cfg.vocab, cfg.hidden, rng=rng)
    hw.output = QTensor(output_type, (cfg.vocab, cfg.hidden), w.blocks)
    return hw


def swiglu_pair_rows(w1: QTensor, w3: QTensor) -> QTensor:
    """The gate (w1) and up (w3) projections as one weight of gate and up rows
    in pairs of four: row 8b + j is w1 row 4b + j for j < 4, w3 row 4b + j - 4
    for j >= 4.  One matmul then gives both, and silu(g) * u of index i sits
    in output columns 8(i / 4) + i % 4 and four on (aq_llama_swiglu_pairs), so
    a matvec kernel can close each 8-row block with its four SwiGLU values
    (aq_qmatmul_rmsnorm_swiglu_f32_device).  The rows are the quantized
    blocks of the two tensors, unchanged."""
    if w1.dtype != w3.dtype or w1.shape != w3.shape or w1.shape[0] % 4:
        raise ValueError("w1 and w3 need one type, one shape and rows in whole fours")
    ffn = w1.shape[0]
    rb = w1.data.size // ffn  # bytes per row
    a = np.asarray(w1.data).reshape(ffn // 4, 1, 4 * rb)
    b = np.asarray(w3.data).reshape(ffn // 4, 1, 4 * rb)
    return QTensor(w1.dtype, (2 * ffn, w1.shape[1]), np.concatenate([a, b], axis=1).reshape(-1))


def rope_tables(cfg: LlamaConfig, n_pos: int) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin [n_pos][head_dim/2] as candle's precompute_freqs_cis (f32)."""
    hd = cfg.head_dim
    theta = np.array([1.0 / (cfg.rope_theta ** (i / hd)) for i in range(0, hd, 2)], dtype=np.float32)
    idx = np.arange(n_pos, dtype=np.float32)[:, None] * theta[None, :]
    return np.cos(idx).astype(np.float32), np.sin(idx).astype(np.float32)


class GenerateResult:
    def __init__(self, tokens: list[int], prefill_us: int, decode_us: int):
        self.tokens = tokens
        self.prefill_us = prefill_us
        self.decode_us = decode_us

    def stats(self, n_prompt: int) -> dict:
        """The statistics ArmAI.LlamaCandle.generate reports (llama_candle.ex:92-101)."""
        n_new = len(self.tokens)
        return {
            "n_prompt": n_prompt,
            "n_new": n_new,
            "prefill_ms": self.prefill_us / 1000.0,
            "decode_total_ms": self.decode_us / 1000.0,
            "decode_ms_per_tok": self.decode_us / 1000.0 / (n_new - 1) if n_new > 1 else None,
            "prefill_tokens_per_sec": n_prompt * 1.0e6 / max(self.prefill_us, 1),
        }


class Llama:
    """ModelWeights on one MI355X: quantized projections in HBM (this library),
    f32 embedding / norms / KV cache as torch tensors on the same device."""

    RESERVE_TOKENS = 512  # the prompt length whose buffers a new model reserves (llama.cpp's default micro-batch)

    def __init__(self, ctx: Context, hw: HostWeights, reserve: int | None = None):
        """reserve: prompt length whose buffers are reserved here (see
        reserve()); None takes min(max_seq, RESERVE_TOKENS), 0 none."""
        import torch

        self.torch = torch
        self.ctx = ctx
        self.cfg = cfg = hw.cfg
        if cfg.hidden % cfg.n_head or cfg.n_head % cfg.n_kv_head:
            raise ValueError("hidden must divide into n_head heads and n_head into n_kv_head groups")
        if not torch.cuda.is_available():
            raise RuntimeError(
                "torch sees no GPU: import torch before the first arm_ai_amd call in this process "
                "(torch loads its own HIP runtime, and a process can use only one)")
        self.dev = torch.device("cuda", ctx.device)
        self.stream = torch.cuda.ExternalStream(ctx.stream, device=self.dev)
        f32 = dict(dtype=torch.float32, device=self.dev)
        with torch.cuda.stream(self.stream):
            self.layers = [self._upload_layer(layer) for layer in hw.layers]
            self.attn_norm = [torch.tensor(w, **f32) for w in hw.attn_norm]
            self.ffn_norm = [torch.tensor(w, **f32) for w in hw.ffn_norm]
            self.tok_embeddings = torch.tensor(hw.tok_embeddings, **f32)
            self.norm = torch.tensor(hw.norm, **f32)
            self.output = QMatMul.from_qtensor(hw.output, ctx)
            cos, sin = rope_tables(cfg, cfg.max_seq)
            self.cos = torch.tensor(cos, **f32)
            self.sin = torch.tensor(sin, **f32)
            hd = cfg.head_dim
            self.k_cache = torch.zeros((cfg.n_layer, cfg.n_kv_head, cfg.max_seq, hd), **f32)
            self.v_cache = torch.zeros((cfg.n_layer, cfg.n_kv_head, cfg.max_seq, hd), **f32)
        self.ctx.synchronize()
        self._n_second = {"wqk": cfg.n_kv_head * cfg.head_dim, "w13": cfg.ffn}
        # The prompt quantises each norm / SwiGLU output once, in the launch
        # that forms it (aq_llama_rmsnorm_act, aq_llama_swiglu_pairs_act), and
        # feeds the planes to every GEMM that reads it: when every layer's
        # projections after the norms take Q8_K activations, w1|w3 is paired
        # and the widths are whole Q8_K blocks.
        q8k = lambda w: w.act_type == GgmlDType.Q8K
        self._prompt_act = cfg.hidden % 256 == 0 and cfg.ffn % 256 == 0 and cfg.hidden <= 8192 and \
            cfg.ffn <= 16384 and all(
                "w13p" in lw and all(q8k(w) for name, w in lw.items() if name != "wo") for lw in self.layers)
        self._graph = None
        self._trace = None  # (rows, full layers, records) while trace_matmuls is active
        self._trace_layer = -1
        self._hidden = None  # {layer index: residual input} while capture_hidden is active
        self.reserve(min(cfg.max_seq, self.RESERVE_TOKENS) if reserve is None else reserve)

    def reserve(self, n: int) -> None:
        """Make the buffers of a prompt of up to n tokens exist before the
        first real one, as llama.cpp reserves its compute buffers when a
        context is created: one forward of n tokens at offset 0 (torch keeps
        the blocks it allocates on this stream, the context keeps its grown
        scratch), then the KV cache is cleared.  Without it the first prompt
        of a new length pays for those allocations (torch's new segments,
        and the scratch's synchronise, free and larger allocation)."""
        n = min(int(n), self.cfg.max_seq)
        if n <= 0:
            return
        self.forward([0] * n, 0)
        with self.torch.cuda.stream(self.stream):
            self.k_cache.zero_()
            self.v_cache.zero_()
        self.ctx.synchronize()

    def _upload_layer(self, layer: dict[str, QTensor]) -> dict[str, QMatMul]:
        """The layer's projections in HBM; when a pair has one type, one weight
        serves both: wq|wk with its rows concatenated ("wqk"), w1|w3 as gate
        and up rows in pairs of four ("w13p", swiglu_pair_rows) where the
        decode matvec then forms silu(g) * u in the same launch
        (aq_swiglu_fused), else concatenated ("w13")."""
        from . import _lib

        out = {}
        qa, qb = layer["wq"], layer["wk"]
        if qa.dtype == qb.dtype and qa.shape[1] == qb.shape[1]:
            cat = QTensor(qa.dtype, (qa.shape[0] + qb.shape[0], qa.shape[1]),
                          np.concatenate([qa.data.reshape(-1), qb.data.reshape(-1)]))
            out["wqk"] = QMatMul.from_qtensor(cat, self.ctx)
        else:
            out["wq"] = QMatMul.from_qtensor(qa, self.ctx)
            out["wk"] = QMatMul.from_qtensor(qb, self.ctx)
        qa, qb = layer["w1"], layer["w3"]
        if qa.dtype == qb.dtype and qa.shape == qb.shape and qa.shape[0] % 4 == 0 and \
                _lib.load().aq_swiglu_fused(int(qa.dtype), 2 * qa.shape[0], qa.shape[1]):
            out["w13p"] = QMatMul.from_qtensor(swiglu_pair_rows(qa, qb), self.ctx)
        elif qa.dtype == qb.dtype and qa.shape[1] == qb.shape[1]:
            cat = QTensor(qa.dtype, (qa.shape[0] + qb.shape[0], qa.shape[1]),
                          np.concatenate([qa.data.reshape(-1), qb.data.reshape(-1)]))
            out["w13"] = QMatMul.from_qtensor(cat, self.ctx)
        else:
            out["w1"] = QMatMul.from_qtensor(qa, self.ctx)
            out["w3"] = QMatMul.from_qtensor(qb, self.ctx)
        for name in ("wv", "wo", "w2"):
            out[name] = QMatMul.from_qtensor(layer[name], self.ctx)
        return out

    def _pair_act(self, lw, act, m, x):
        """q and k from the quantised norm output: one GEMM on wq|wk, or two."""
        if "wqk" in lw:
            y = self._mm_act(lw["wqk"], act, m, x)
            na = y.shape[1] - self._n_second["wqk"]
            return y[:, :na], y[:, na:]
        return self._mm_act(lw["wq"], act, m, x), self._mm_act(lw["wk"], act, m, x)

    def _qkv_act(self, lw, act, m, x):
        """q, k and v from the quantised norm output: wq|wk and wv in one
        call (aq_qmatmul2_preq_device: one launch where their types allow)."""
        from . import _lib

        if "wqk" not in lw:
            q, k = self._pair_act(lw, act, m, x)
            return q, k, self._mm_act(lw["wv"], act, m, x)
        w1, w2 = lw["wqk"], lw["wv"]
        f32 = dict(dtype=self.torch.float32, device=self.dev)
        y1, y2 = self.torch.empty((m, w1.n), **f32), self.torch.empty((m, w2.n), **f32)
        _lib.check(_lib.load().aq_qmatmul2_preq_device(self.ctx.handle, w1.handle, w2.handle, act.data_ptr(), m, w1.k,
                                                       y1.data_ptr(), y2.data_ptr()))
        self._record_mm(w1, x, y1)
        self._record_mm(w2, x, y2)
        na = w1.n - self._n_second["wqk"]
        return y1[:, :na], y1[:, na:], y2

    def _pair(self, lw, merged, a, b, x):
        """Outputs of projections a and b of x: one launch on the merged weight, or two."""
        if merged in lw:
            y = self._mm(lw[merged], x)
            na = y.shape[1] - self._n_second[merged]
            return y[:, :na], y[:, na:]
        return self._mm(lw[a], x), self._mm(lw[b], x)

    @classmethod
    def from_gguf(cls, ctx: Context, path: str, max_seq: int = 4096) -> "Llama":
        """ArmAI.LlamaCandle.load (llama_candle.rs:35-48): read a llama GGUF file
        (arm_ai_amd.gguf) and upload its projections to HBM."""
        from .gguf import load_llama

        _, hw = load_llama(path, max_seq=max_seq)
        return cls(ctx, hw)

    # ------------------------------------------------------------ pieces
    # The work runs on the library's stream; the caller's current stream waits
    # for it on the way out (and it for the caller's on the way in), so tensors
    # handed back can be used on the caller's stream directly.
    def _enter(self):
        self.stream.wait_stream(self.torch.cuda.current_stream(self.dev))

    def _leave(self):
        self.torch.cuda.current_stream(self.dev).wait_stream(self.stream)

    def _mm(self, w: QMatMul, x):
        """QMatMul::forward on device memory: x f32 [m, k] -> f32 [m, n]."""
        torch = self.torch
        x = x.contiguous()
        y = torch.empty((x.shape[0], w.n), dtype=torch.float32, device=self.dev)
        w.forward_device(x.data_ptr(), x.shape[0], y.data_ptr())
        self._record_mm(w, x, y)
        return y

    def _mm_act(self, w: QMatMul, act, m: int, x=None):
        """QMatMul::forward on activation planes already quantised (act, from
        aq_llama_rmsnorm_act / aq_llama_swiglu_pairs_act); x, the f32 values
        they were quantised from, only for trace_matmuls."""
        from . import _lib

        y = self.torch.empty((m, w.n), dtype=self.torch.float32, device=self.dev)
        _lib.check(_lib.load().aq_qmatmul_preq_device(self.ctx.handle, w.handle, act.data_ptr(), m, w.k,
                                                      y.data_ptr()))
        self._record_mm(w, x, y)
        return y

    def _record_mm(self, w, x, y):
        if self._trace is not None:
            rows, full, records = self._trace
            if self._trace_layer in full:
                sel = list(range(x.shape[0]))
            else:
                sel = [r for r in rows if r < x.shape[0]] or [0]
            records.append((self._trace_layer, w, x[sel].cpu().numpy(), y[sel].cpu().numpy(), sel))

    @contextlib.contextmanager
    def capture_hidden(self, layers):
        """Record the residual stream [L, hidden] that forward() feeds to each
        of the given layers (index n_layer: the stream after the last layer),
        copied to the host: a test aid."""
        rec = {"layers": set(layers), "x": {}}
        self._hidden = rec
        try:
            yield rec["x"]
        finally:
            self._hidden = None

    def _record_hidden(self, li, x, delta=None):
        if self._hidden is not None and li in self._hidden["layers"]:
            self._hidden["x"][li] = (x + delta if delta is not None else x).cpu().numpy()

    @contextlib.contextmanager
    def trace_matmuls(self, rows=(0,), full_layers=()):
        """Record every QMatMul::forward made by forward() inside the block:
        yields a list that receives (layer, QMatMul, x rows, y rows, row
        indices) per call (layer n_layer: the output head), for the rows
        given (those below the call's m; row 0 when none is), or every row
        for the layers in full_layers.  A test aid: each record is copied to
        the host as it is made, which synchronises the stream."""
        records = []
        self._trace = (tuple(rows), set(full_layers), records)
        try:
            yield records
        finally:
            self._trace = None

    # ------------------------------------------------------------ forward
    def forward(self, tokens, index_pos: int):
        """ModelWeights::forward(&x[1, L], index_pos) -> logits f32 [vocab] of the last position.

        tokens: a torch int64 tensor [L] on the device, or a sequence of ints.
        Every step is a library kernel on the context's stream (torch only
        allocates): the embedding rows; per layer rms_norm (with the pending
        residual add of the previous layer's w2 output, written back to the
        stream), wq|wk and wv, rotary embedding + KV append + causal
        grouped-query attention (aq_llama_attn_prefill), wo, the residual add
        and rms_norm, w1|w3, silu(g) * u, w2; the final rms_norm of the last
        row and the output head."""
        from . import _lib

        torch = self.torch
        cfg = self.cfg
        L = _lib.load()
        c = self.ctx.handle
        chk = _lib.check
        eps = ctypes.c_float(cfg.rms_eps)
        ptr = lambda t: t.data_ptr()
        self._enter()
        with torch.cuda.stream(self.stream):
            if not torch.is_tensor(tokens):
                tokens = torch.tensor(list(tokens), dtype=torch.int64, device=self.dev)
            tokens = tokens.contiguous()
            n = int(tokens.shape[0])
            if n == 0 or index_pos < 0 or index_pos + n > cfg.max_seq:
                raise ValueError(f"positions {index_pos}..{index_pos + n} outside 0..{cfg.max_seq}")
            H, Hkv, D = cfg.n_head, cfg.n_kv_head, cfg.head_dim
            f32 = dict(dtype=torch.float32, device=self.dev)
            x = torch.empty((n, cfg.hidden), **f32)  # the residual stream (x + delta once delta is set)
            h = torch.empty((n, cfg.hidden), **f32)  # normed input of the next projections
            y = torch.empty((n, H * D), **f32)       # attention output
            a = torch.empty((n, cfg.ffn), **f32)     # silu(g) * u
            chk(L.aq_llama_embed_rows(c, ptr(self.tok_embeddings), cfg.vocab, ptr(tokens), n, cfg.hidden, ptr(x)))
            delta = None
            fused = self._prompt_act and n > 8  # GEMM-sized prompts (fewer rows: fused-quantisation matvecs)
            if fused:  # the quantised norm / SwiGLU outputs (their f32 values only while tracing)
                u8 = dict(dtype=torch.uint8, device=self.dev)
                act_h = torch.empty(int(L.aq_act_bytes(int(GgmlDType.Q8K), n, cfg.hidden)), **u8)
                act_a = torch.empty(int(L.aq_act_bytes(int(GgmlDType.Q8K), n, cfg.ffn)), **u8)
                keep = self._trace is not None
            for li, lw in enumerate(self.layers):
                self._trace_layer = li
                self._record_hidden(li, x, delta)
                if fused:
                    chk(L.aq_llama_rmsnorm_act(c, ptr(x), ptr(delta) if delta is not None else None,
                                               ptr(self.attn_norm[li]), n, cfg.hidden, eps, ptr(h) if keep else None,
                                               ptr(act_h)))
                    q, k, v = self._qkv_act(lw, act_h, n, h)
                    chk(L.aq_llama_attn_prefill(c, ptr(q), q.stride(0), ptr(k), k.stride(0), ptr(v), v.stride(0),
                                                ptr(self.cos), ptr(self.sin), index_pos, n, ptr(self.k_cache[li]),
                                                ptr(self.v_cache[li]), H, Hkv, D, cfg.max_seq, ptr(y)))
                    o = self._mm(lw["wo"], y)
                    chk(L.aq_llama_rmsnorm_act(c, ptr(x), ptr(o), ptr(self.ffn_norm[li]), n, cfg.hidden, eps,
                                               ptr(h) if keep else None, ptr(act_h)))
                    gu = self._mm_act(lw["w13p"], act_h, n, h)
                    chk(L.aq_llama_swiglu_pairs_act(c, ptr(gu), gu.stride(0), n, cfg.ffn, ptr(a) if keep else None,
                                                    ptr(act_a)))
                    delta = self._mm_act(lw["w2"], act_a, n, a)
                    continue
                chk(L.aq_llama_rmsnorm(c, ptr(x), ptr(delta) if delta is not None else None, ptr(self.attn_norm[li]),
                                       n, cfg.hidden, eps, ptr(h)))
                q, k = self._pair(lw, "wqk", "wq", "wk", h)
                v = self._mm(lw["wv"], h)
                chk(L.aq_llama_attn_prefill(c, ptr(q), q.stride(0), ptr(k), k.stride(0), ptr(v), v.stride(0),
                                            ptr(self.cos), ptr(self.sin), index_pos, n, ptr(self.k_cache[li]),
                                            ptr(self.v_cache[li]), H, Hkv, D, cfg.max_seq, ptr(y)))
                o = self._mm(lw["wo"], y)
                chk(L.aq_llama_rmsnorm(c, ptr(x), ptr(o), ptr(self.ffn_norm[li]), n, cfg.hidden, eps, ptr(h)))
                if "w13p" in lw:  # gate and up rows in pairs of four
                    gu = self._mm(lw["w13p"], h)
                    chk(L.aq_llama_swiglu_pairs(c, ptr(gu), gu.stride(0), n, cfg.ffn, ptr(a)))
                else:
                    g, u = self._pair(lw, "w13", "w1", "w3", h)
                    chk(L.aq_llama_silu_mul_rows(c, ptr(g), ptr(u), g.stride(0), n, cfg.ffn, ptr(a)))
                delta = self._mm(lw["w2"], a)
            self._trace_layer = len(self.layers)
            self._record_hidden(len(self.layers), x, delta)
            last = torch.empty((1, cfg.hidden), **f32)
            chk(L.aq_llama_rmsnorm(c, ptr(x[n - 1:]), ptr(delta[n - 1:]), ptr(self.norm), 1, cfg.hidden, eps,
                                   ptr(last)))
            logits = self._mm(self.output, last)[0]
        self._leave()
        return logits

    # ------------------------------------------------------------ graph-captured decode step
    def _decode_buffers(self):
        torch = self.torch
        cfg = self.cfg
        hd = cfg.head_dim
        f32 = dict(dtype=torch.float32, device=self.dev)
        i64 = dict(dtype=torch.int64, device=self.dev)
        self._pos = torch.zeros(1, **i64)
        self._tok = torch.zeros(1, **i64)
        self._hist = torch.zeros(cfg.max_seq, **i64)  # token generated at each position
        self._ra = torch.zeros(cfg.hidden, **f32)      # residual stream, two buffers in turn
        self._rb = torch.zeros(cfg.hidden, **f32)
        self._qk = torch.zeros((cfg.n_head + cfg.n_kv_head) * hd, **f32)
        self._v = torch.zeros(cfg.n_kv_head * hd, **f32)
        self._att = torch.zeros(cfg.n_head * hd, **f32)
        self._o = torch.zeros(cfg.hidden, **f32)       # wo output
        self._gu = torch.zeros(2 * cfg.ffn, **f32)
        self._a = torch.zeros(cfg.ffn, **f32)         # silu(g) * u
        self._d = torch.zeros(cfg.hidden, **f32)       # w2 output (the pending residual delta)
        self._logits = torch.zeros(cfg.vocab, **f32)

    def _decode_step_static(self):
        """One decode step for the token in self._tok at the position in self._pos
        (both device memory), whose embedding row is in self._ra; leaves the
        logits in self._logits, the next token in self._tok and in
        self._hist[pos], its embedding row in self._ra, and pos + 1 in
        self._pos.

        Per layer six launches: the QMatMuls of wq|wk and wv, one launch for
        both, take rms_norm(x + delta) as their input (formed inside the
        matvec, which also writes the residual x + delta once), attention
        (RoPE, KV write, GQA: a split launch and a combining launch), wo,
        w1|w3 on rms_norm(h + wo), w2.  silu(g) * u is formed by the w1|w3
        launch where its gate and up rows are paired ("w13p": each 8-row
        block closes with four SwiGLU values), else by the w2 launch's
        prologue from [g | u]."""
        from . import _lib

        L = _lib.load()
        cfg = self.cfg
        c = self.ctx.handle
        hd = cfg.head_dim
        ptr = lambda t: t.data_ptr()
        chk = _lib.check
        eps = ctypes.c_float(cfg.rms_eps)

        def mm_norm(w, x, delta, norm, out, h_out=None):
            chk(L.aq_qmatmul_rmsnorm_f32_device(c, w.handle, ptr(x), delta, ptr(norm), eps, w.k,
                                                ptr(h_out) if h_out is not None else None, out))

        cur, other = self._ra, self._rb  # cur: the token's embedding row, left by the step before (or _set_token)
        delta = None
        for li, lw in enumerate(self.layers):
            an = self.attn_norm[li]
            if "wqk" in lw:
                # wq|wk and wv: one launch for Q4_K / Q6_K and for Q5_0 / Q8_0 pairs
                chk(L.aq_qmatmul2_rmsnorm_f32_device(c, lw["wqk"].handle, lw["wv"].handle, ptr(cur), delta, ptr(an),
                                                     eps, cfg.hidden, ptr(other), ptr(self._qk), ptr(self._v)))
            else:
                mm_norm(lw["wq"], cur, delta, an, ptr(self._qk), h_out=other)
                mm_norm(lw["wk"], cur, delta, an, ptr(self._qk) + 4 * cfg.n_head * hd)
                mm_norm(lw["wv"], cur, delta, an, ptr(self._v))
            chk(L.aq_llama_attn_decode(c, ptr(self._qk), ptr(self._v), ptr(self.cos), ptr(self.sin), ptr(self._pos),
                                       ptr(self.k_cache[li]), ptr(self.v_cache[li]), cfg.n_head, cfg.n_kv_head, hd,
                                       cfg.max_seq, ptr(self._att)))
            lw["wo"].forward_device(ptr(self._att), 1, ptr(self._o))
            fn = self.ffn_norm[li]
            if "w13p" in lw:  # silu(g) * u formed by the w1|w3 launch, w2 on it
                chk(L.aq_qmatmul_rmsnorm_swiglu_f32_device(c, lw["w13p"].handle, ptr(other), ptr(self._o), ptr(fn),
                                                           eps, cfg.hidden, ptr(cur), ptr(self._a)))
                lw["w2"].forward_device(ptr(self._a), 1, ptr(self._d))
            else:  # [g | u], silu(g) * u formed by the w2 launch
                if "w13" in lw:
                    mm_norm(lw["w13"], other, ptr(self._o), fn, ptr(self._gu), h_out=cur)
                else:
                    mm_norm(lw["w1"], other, ptr(self._o), fn, ptr(self._gu), h_out=cur)
                    mm_norm(lw["w3"], other, ptr(self._o), fn, ptr(self._gu) + 4 * cfg.ffn)
                chk(L.aq_qmatmul_silu_mul_f32_device(c, lw["w2"].handle, ptr(self._gu), cfg.ffn, ptr(self._d)))
            delta = ptr(self._d)  # the residual is now x + wo + w2 = cur + d
        # the head, the greedy pick (token, history, position) and the picked
        # token's embedding row into _ra, the next step's input
        chk(L.aq_llama_head_argmax_embed(c, self.output.handle, ptr(cur), delta, ptr(self.norm), eps, cfg.hidden,
                                         ptr(self._logits), ptr(self._tok), ptr(self._pos), ptr(self._hist),
                                         cfg.max_seq, ptr(self.tok_embeddings), cfg.hidden, ptr(self._ra)))

    def _capture(self):
        torch = self.torch
        self._enter()
        with torch.cuda.stream(self.stream):
            self._decode_buffers()
        # Warm up on the capture stream (library first-call set-up) at the last
        # cache slot: a step writes only its own position's k, v, so the cache
        # entries of a sequence in progress stay intact.
        with torch.cuda.stream(self.stream):
            self._set_token(0, self.cfg.max_seq - 1)
            self._decode_step_static()
        self.ctx.synchronize()
        # (capture_begin / capture_end rather than the torch.cuda.graph
        #  context, which empties torch's block cache on entry and so would
        #  release the prompt buffers reserve() set aside)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(self.stream):
            g.capture_begin()
            try:
                self._decode_step_static()
            finally:
                g.capture_end()
        self._graph = g
        self._leave()

    def _set_token(self, token: int, pos: int):
        """The decode step's input on the library stream: the token, its position
        and its embedding row (a replay then feeds the next one itself)."""
        from . import _lib

        self._pos.fill_(pos)
        self._tok.fill_(token)
        _lib.check(_lib.load().aq_llama_embed(self.ctx.handle, self.tok_embeddings.data_ptr(), self.cfg.vocab,
                                              self._tok.data_ptr(), self.cfg.hidden, self._ra.data_ptr()))

    def decode_step_graph(self, token: int, pos: int):
        """Replay the captured decode step for `token` at position `pos`; returns the device logits."""
        if self._graph is None:
            self._capture()
        if not 0 <= pos < self.cfg.max_seq:
            raise ValueError(f"position {pos} outside 0..{self.cfg.max_seq}")
        self._enter()
        with self.torch.cuda.stream(self.stream):
            self._set_token(token, pos)
            self._graph.replay()
        self._leave()
        return self._logits

    # ------------------------------------------------------------ generate
    @staticmethod
    def argmax_first(logits) -> int:
        """First index of the maximum (llama_candle.rs:154-176 folds with a strict >)."""
        return int(logits.argmax().item())

    def generate(self, prompt: list[int], max_new: int, stop_tokens=(), graph: bool = False,
                 chunk: int = 16, on_token=None) -> GenerateResult:
        """generate_greedy (llama_candle.rs:58-139): prefill at offset 0, then one
        forward per new token; stops after emitting a stop token (kept in the output).

        With graph=True the captured step is replayed `chunk` times back to back
        (each replay feeds the next from device memory), then the chunk's tokens
        are read and checked for a stop token; tokens after the first stop token
        are dropped, so the output is the same as stepping one token at a time.

        on_token: called with each token as soon as it is chosen, in order --
        the streaming form (llama_candle_stream_op's {:llama_token, id},
        native/arm_ai_nif/src/lib.rs:1682-1699).  With graph=True it sets the
        chunk to one: one replay, one token read back, the callback, then the
        next replay (native/arm_ai_nif/src/gpu_llama.rs generate_greedy_with)."""
        if max_new == 0 or len(prompt) == 0:
            return GenerateResult([], 0, 0)
        if len(prompt) + max_new - 1 > self.cfg.max_seq:
            raise ValueError("prompt + max_new exceeds max_seq")
        if on_token is not None:
            chunk = 1
        emit = on_token if on_token is not None else (lambda _t: None)
        if graph and self._graph is None:
            self._capture()
        self.ctx.synchronize()
        t0 = time.perf_counter()
        logits = self.forward(prompt, 0)
        nxt = self.argmax_first(logits)  # .item() synchronises
        prefill_us = int((time.perf_counter() - t0) * 1e6)
        generated = [nxt]
        emit(nxt)
        t1 = time.perf_counter()
        offset = len(prompt)
        if graph and max_new > 1 and nxt not in stop_tokens:
            self._enter()
            with self.torch.cuda.stream(self.stream):
                self._set_token(nxt, offset)
            done = False
            while not done and len(generated) < max_new:
                n = min(chunk, max_new - len(generated))
                with self.torch.cuda.stream(self.stream):
                    for _ in range(n):
                        self._graph.replay()
                    toks = self._hist[offset:offset + n].tolist()  # copies on the stream, then synchronises
                for t in toks:
                    generated.append(int(t))
                    emit(int(t))
                    if t in stop_tokens:
                        done = True
                        break
                offset += n
            self._leave()
        else:
            for _ in range(1, max_new):
                if nxt in stop_tokens:
                    break
                nxt = self.argmax_first(self.forward([nxt], offset))
                generated.append(nxt)
                emit(nxt)
                offset += 1
        decode_us = int((time.perf_counter() - t1) * 1e6)
        return GenerateResult(generated, prefill_us, decode_us)

    def free(self) -> None:
        for lw in self.layers:
            for w in lw.values():
                w.free()
        self.output.free()
