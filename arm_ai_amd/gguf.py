"""GGUF files: the reader behind ``load`` of ArmAI.LlamaCandle, and a writer.

In the reference, ``llama_candle_load_op`` opens the model file and reads it
with candle's ``gguf_file::Content::read`` (native/arm_ai_nif/src/llama_candle.rs:35-48),
then ``quantized_llama::ModelWeights::from_gguf`` builds the model from the
``llama.*`` metadata and the ``token_embd`` / ``blk.N.*`` / ``output*``
tensors.  Both are candle 0.8.4 registry code, not vendored in the reference;
this module restates them from the public GGUF format:

* header: magic ``GGUF``, version (2 or 3; version 1 used 32-bit counts and
  string lengths and is rejected), tensor count, metadata count (u64);
* metadata: key (u64-length string), value type (u32), value; arrays are
  (element type u32, count u64, elements);
* tensor infos: name, n_dims (u32), dims (u64 each, fastest first: a 2-D
  weight of n rows by k columns has dims (k, n)), ggml type (u32), offset
  (u64) from the start of the data section;
* the data section starts at the first multiple of ``general.alignment``
  (default 32) after the tensor infos.

``load_llama`` returns the host weights the driver (arm_ai_amd.llama) uploads:
the quantized projections as raw GGUF blocks (memory-mapped, uploaded to HBM
by aq_qweight_upload), the norm weights as f32, and the token embedding
dequantized to f32 as candle does for its embedding table.  Dequantization
follows candle's ``to_float`` f32 formulas (restated from the GGML block
definitions: Q4_K and Q5_K d*sc*q - dmin*m, Q6_K d*sc*(q-32), Q8_0 d*q,
Q4_0 d*(q-8)); the
embedding only feeds the f32 glue, which is tolerance-checked.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass

import numpy as np

from . import synth
from .qmatmul import GgmlDType, QTensor

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}

# ggml tensor types read here: (elements per block, bytes per block)
GGML_F32, GGML_F16 = 0, 1
TYPE_SIZES = {GGML_F32: (1, 4), GGML_F16: (1, 2), synth.TYPE_Q8_0: (32, 34), synth.TYPE_Q4_0: (32, 18), synth.TYPE_Q5_0: (32, 22),
              synth.TYPE_Q4_K: (256, 144), synth.TYPE_Q5_K: (256, 176), synth.TYPE_Q6_K: (256, 210),
              synth.TYPE_Q2_K: (256, 84), synth.TYPE_Q3_K: (256, 110)}
QUANT_TYPES = (synth.TYPE_Q4_K, synth.TYPE_Q5_K, synth.TYPE_Q6_K, synth.TYPE_Q8_0, synth.TYPE_Q4_0, synth.TYPE_Q2_K,
               synth.TYPE_Q3_K, synth.TYPE_Q5_0)


class GGUFError(ValueError):
    """A file that is not a GGUF model this reader can use (candle: `gguf read failed`)."""


@dataclass
class TensorInfo:
    name: str
    dims: tuple[int, ...]  # GGUF order, fastest first
    type: int
    offset: int  # from the start of the data section

    @property
    def shape(self) -> tuple[int, ...]:
        """candle's shape: dims reversed (a weight is (n, k))."""
        return tuple(reversed(self.dims))

    @property
    def n_elements(self) -> int:
        return int(np.prod(self.dims, dtype=np.int64)) if self.dims else 1

    @property
    def nbytes(self) -> int:
        if self.type not in TYPE_SIZES:
            raise GGUFError(f"tensor {self.name}: ggml type {self.type} is not supported")
        be, bb = TYPE_SIZES[self.type]
        if self.n_elements % be:
            raise GGUFError(f"tensor {self.name}: {self.n_elements} elements is not a whole number of blocks")
        return self.n_elements // be * bb


class _Reader:
    def __init__(self, buf, path: str):
        self.buf = buf
        self.pos = 0
        self.path = path

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise GGUFError(f"{self.path}: truncated at byte {self.pos}")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(T_U64)
        if n > len(self.buf):
            raise GGUFError(f"{self.path}: string length {n} past the end of the file")
        return self.take(n).decode("utf-8", errors="replace")

    def value(self, t: int):
        if t in _SCALAR:
            return self.scalar(t)
        if t == T_STR:
            return self.string()
        if t == T_ARR:
            et = self.scalar(T_U32)
            n = self.scalar(T_U64)
            if et in _SCALAR and et != T_BOOL:
                fmt = _SCALAR[et]
                size = struct.calcsize(fmt)
                raw = self.take(size * n)
                return np.frombuffer(raw, dtype=np.dtype(fmt)).copy()
            return [self.value(et) for _ in range(n)]
        raise GGUFError(f"{self.path}: unknown metadata value type {t}")


class GGUFFile:
    """A GGUF file's metadata and tensor infos; tensor data stays memory-mapped."""

    def __init__(self, path: str):
        if not path:
            raise GGUFError("empty path")
        if not os.path.isfile(path):
            raise GGUFError(f"open {path} failed: no such file")
        self.path = path
        self._map = np.memmap(path, dtype=np.uint8, mode="r") if os.path.getsize(path) else np.zeros(0, np.uint8)
        r = _Reader(self._map, path)
        if r.take(4) != GGUF_MAGIC:
            raise GGUFError(f"{path}: not a GGUF file (bad magic)")
        self.version = r.scalar(T_U32)
        if self.version not in (2, 3):
            raise GGUFError(f"{path}: GGUF version {self.version} is not supported")
        n_tensors = r.scalar(T_U64)
        n_kv = r.scalar(T_U64)
        self.metadata: dict[str, object] = {}
        for _ in range(n_kv):
            key = r.string()
            self.metadata[key] = r.value(r.scalar(T_U32))
        self.tensors: dict[str, TensorInfo] = {}
        for _ in range(n_tensors):
            name = r.string()
            nd = r.scalar(T_U32)
            if nd > 4:
                raise GGUFError(f"{path}: tensor {name} has {nd} dimensions")
            dims = tuple(int(r.scalar(T_U64)) for _ in range(nd))
            t = r.scalar(T_U32)
            off = r.scalar(T_U64)
            self.tensors[name] = TensorInfo(name, dims, t, off)
        align = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"{path}: alignment {align} is not a power of two")
        self.data_start = (r.pos + align - 1) // align * align
        for ti in self.tensors.values():
            if ti.type in TYPE_SIZES and self.data_start + ti.offset + ti.nbytes > len(self._map):
                raise GGUFError(f"{path}: tensor {ti.name} lies past the end of the file")

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes (a read-only view of the mapped file)."""
        ti = self.tensor(name)
        o = self.data_start + ti.offset
        return self._map[o:o + ti.nbytes]

    def tensor(self, name: str) -> TensorInfo:
        if name not in self.tensors:
            raise GGUFError(f"{self.path}: cannot find tensor {name}")
        return self.tensors[name]

    def qtensor(self, name: str) -> QTensor:
        """A 2-D quantized weight as candle's QTensor (n rows, k columns)."""
        ti = self.tensor(name)
        if ti.type not in QUANT_TYPES or len(ti.dims) != 2:
            raise GGUFError(f"tensor {name}: a 2-D Q2_K / Q3_K / Q4_K / Q5_K / Q6_K / Q8_0 / Q4_0 / Q5_0 weight is needed, got type {ti.type} "
                            f"with dims {ti.dims}")
        k, n = ti.dims
        return QTensor(GgmlDType(ti.type), (n, k), self.raw(name))

    def f32(self, name: str) -> np.ndarray:
        """The tensor as f32 in candle's shape (F32, F16 or dequantized blocks)."""
        ti = self.tensor(name)
        raw = self.raw(name)
        if ti.type == GGML_F32:
            v = np.frombuffer(raw, dtype="<f4").astype(np.float32)
        elif ti.type == GGML_F16:
            v = np.frombuffer(raw, dtype="<f2").astype(np.float32)
        elif ti.type in QUANT_TYPES:
            v = dequantize(ti.type, raw, ti.n_elements)
        else:
            raise GGUFError(f"tensor {name}: ggml type {ti.type} is not supported")
        return v.reshape(ti.shape)

    def get(self, key: str, default=None):
        return self.metadata.get(key, default)

    def require(self, key: str):
        if key not in self.metadata:
            raise GGUFError(f"{self.path}: cannot find {key} in metadata")
        return self.metadata[key]


# ------------------------------------------------------------------ dequantize
def _f16(b: np.ndarray) -> np.ndarray:
    return b.copy().view("<f2").astype(np.float32)[..., 0]


def dequantize(type_: int, raw: np.ndarray, n_elements: int) -> np.ndarray:
    """GGUF blocks -> f32 [n_elements], candle to_float's f32 operation order."""
    raw = np.asarray(raw, np.uint8)
    if type_ == synth.TYPE_Q4_0:
        b = raw.reshape(-1, 18)
        d = _f16(b[:, 0:2])
        qs = b[:, 2:18]
        q = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.float32) - 8.0  # elements 0..15, 16..31
        return (q * d[:, None]).reshape(-1)[:n_elements]
    if type_ == synth.TYPE_Q5_0:
        b = raw.reshape(-1, 22)
        d = _f16(b[:, 0:2])
        qh = b[:, 2:6].copy().view("<u4")[:, 0].astype(np.int64)
        qs = b[:, 6:22].astype(np.int64)
        q = np.concatenate([qs & 0xF, qs >> 4], axis=1) | (((qh[:, None] >> np.arange(32)[None, :]) & 1) << 4)
        return ((q - 16).astype(np.float32) * d[:, None]).reshape(-1)[:n_elements]
    if type_ == synth.TYPE_Q8_0:
        b = raw.reshape(-1, 34)
        d = _f16(b[:, 0:2])
        q = b[:, 2:34].view(np.int8).astype(np.float32)
        return (q * d[:, None]).reshape(-1)[:n_elements]
    if type_ in (synth.TYPE_Q4_K, synth.TYPE_Q5_K):
        five = type_ == synth.TYPE_Q5_K
        b = raw.reshape(-1, 176 if five else 144)
        d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
        s = b[:, 4:16].astype(np.uint32)
        sc = np.empty((b.shape[0], 8), np.uint32)
        mn = np.empty((b.shape[0], 8), np.uint32)
        sc[:, 0:4] = s[:, 0:4] & 63
        mn[:, 0:4] = s[:, 4:8] & 63
        sc[:, 4:8] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:8] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qs = b[:, 48:176].reshape(-1, 4, 32) if five else b[:, 16:144].reshape(-1, 4, 32)
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.int32)  # [blk][sub][l]
        if five:  # bit s of qh[l] is bit 4 of element 32s + l
            qh = b[:, 16:48].astype(np.int32)
            q = q + 16 * ((qh[:, None, :] >> np.arange(8)[None, :, None]) & 1)
        q = q.astype(np.float32)
        d1 = d[:, None] * sc.astype(np.float32)
        m1 = dmin[:, None] * mn.astype(np.float32)
        return (d1[:, :, None] * q - m1[:, :, None]).reshape(-1)[:n_elements]
    if type_ == synth.TYPE_Q2_K:
        b = raw.reshape(-1, 84)
        d, dmin = _f16(b[:, 80:82]), _f16(b[:, 82:84])
        sc = (b[:, 0:16] & 0xF).astype(np.float32)
        mn = (b[:, 0:16] >> 4).astype(np.float32)
        qs = b[:, 16:80].reshape(-1, 2, 1, 32)
        q = ((qs >> (2 * np.arange(4)[None, None, :, None])) & 3).reshape(-1, 16, 16).astype(np.float32)
        return ((d[:, None] * sc)[:, :, None] * q - (dmin[:, None] * mn)[:, :, None]).reshape(-1)[:n_elements]
    if type_ == synth.TYPE_Q3_K:
        b = raw.reshape(-1, 110)
        hm = b[:, 0:32].astype(np.int32)
        qs = b[:, 32:96].reshape(-1, 2, 1, 32).astype(np.int32)
        sh = np.arange(4)[None, None, :, None]
        q2 = (qs >> (2 * sh)) & 3                                          # [blk][hf][j][l]
        hb = (hm[:, None, None, :] >> (4 * np.arange(2)[None, :, None, None] + sh)) & 1
        q = (q2 - 4 * (1 - hb)).reshape(-1, 16, 16).astype(np.float32)
        a = b[:, 96:108].astype(np.int32)
        s6 = np.empty((b.shape[0], 16), np.int32)
        s6[:, 0:4] = (a[:, 0:4] & 15) | ((a[:, 8:12] & 3) << 4)
        s6[:, 4:8] = (a[:, 4:8] & 15) | (((a[:, 8:12] >> 2) & 3) << 4)
        s6[:, 8:12] = (a[:, 0:4] >> 4) | (((a[:, 8:12] >> 4) & 3) << 4)
        s6[:, 12:16] = (a[:, 4:8] >> 4) | (((a[:, 8:12] >> 6) & 3) << 4)
        d = _f16(b[:, 108:110])
        return ((d[:, None] * (s6 - 32).astype(np.float32))[:, :, None] * q).reshape(-1)[:n_elements]
    if type_ == synth.TYPE_Q6_K:
        b = raw.reshape(-1, 210)
        ql = b[:, 0:128].reshape(-1, 2, 64)
        qh = b[:, 128:192].reshape(-1, 2, 32)
        sc = b[:, 192:208].view(np.int8).astype(np.float32)
        d = _f16(b[:, 208:210])
        lo, hi = ql[:, :, 0:32], ql[:, :, 32:64]
        q = np.empty((b.shape[0], 2, 4, 32), np.int32)
        q[:, :, 0] = (lo & 0xF) | (((qh >> 0) & 3) << 4)
        q[:, :, 1] = (hi & 0xF) | (((qh >> 2) & 3) << 4)
        q[:, :, 2] = (lo >> 4) | (((qh >> 4) & 3) << 4)
        q[:, :, 3] = (hi >> 4) | (((qh >> 6) & 3) << 4)
        q = (q - 32).reshape(-1, 16, 16).astype(np.float32)  # [blk][sub-block][16]
        return ((d[:, None] * sc)[:, :, None] * q).reshape(-1)[:n_elements]
    raise GGUFError(f"cannot dequantize ggml type {type_}")


# ------------------------------------------------------------------ writer
def _w_str(f, s: str) -> None:
    b = s.encode("utf-8")
    f.write(struct.pack("<Q", len(b)))
    f.write(b)


def _w_value(f, v) -> None:
    if isinstance(v, bool):
        f.write(struct.pack("<I?", T_BOOL, v))
    elif isinstance(v, (int, np.integer)):
        f.write(struct.pack("<II", T_U32, int(v)) if 0 <= int(v) < 2 ** 32 else struct.pack("<Iq", T_I64, int(v)))
    elif isinstance(v, (float, np.floating)):
        f.write(struct.pack("<If", T_F32, float(v)))
    elif isinstance(v, str):
        f.write(struct.pack("<I", T_STR))
        _w_str(f, v)
    elif isinstance(v, (list, tuple)):
        if all(isinstance(e, str) for e in v):
            f.write(struct.pack("<IIQ", T_ARR, T_STR, len(v)))
            for e in v:
                _w_str(f, e)
        else:
            a = np.asarray(v)
            t, fmt = (T_F32, "<f4") if a.dtype.kind == "f" else (T_I32, "<i4")
            f.write(struct.pack("<IIQ", T_ARR, t, a.size))
            f.write(a.astype(fmt).tobytes())
    else:
        raise TypeError(f"cannot write metadata value {v!r}")


def write_gguf(path: str, metadata: dict, tensors: list[tuple[str, tuple[int, ...], int, np.ndarray]],
               alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file. tensors: (name, dims fastest first, ggml type, raw bytes)."""
    md = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        md["general.alignment"] = int(alignment)
    offs, off = [], 0
    for _, dims, t, data in tensors:
        offs.append(off)
        off = (off + int(np.asarray(data).nbytes) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(GGUF_MAGIC + struct.pack("<IQQ", 3, len(tensors), len(md)))
        for k, v in md.items():
            _w_str(f, k)
            _w_value(f, v)
        for (name, dims, t, _), o in zip(tensors, offs):
            _w_str(f, name)
            f.write(struct.pack("<I", len(dims)))
            f.write(struct.pack(f"<{len(dims)}Q", *dims))
            f.write(struct.pack("<IQ", t, o))
        start = (f.tell() + alignment - 1) // alignment * alignment
        f.write(b"\0" * (start - f.tell()))
        for (_, _, _, data), o in zip(tensors, offs):
            f.write(b"\0" * (start + o - f.tell()))
            f.write(np.ascontiguousarray(data).tobytes())


# ------------------------------------------------------------------ Llama models
_LAYER_NAMES = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output",
                "w1": "ffn_gate", "w2": "ffn_down", "w3": "ffn_up"}


def load_llama(path: str, max_seq: int = 4096):
    """ModelWeights::from_gguf for a llama-architecture file -> (LlamaConfig, HostWeights).

    Reads llama.attention.head_count(_kv), llama.block_count,
    llama.embedding_length, llama.attention.layer_norm_rms_epsilon and
    llama.rope.freq_base (default 10000); tensors token_embd.weight
    (dequantized to f32), output_norm.weight, output.weight (the embedding
    table's blocks when absent: tied), and blk.N.{attn_q, attn_k, attn_v,
    attn_output, ffn_gate, ffn_down, ffn_up, attn_norm, ffn_norm}."""
    from .llama import HostWeights, LlamaConfig

    g = GGUFFile(path)
    arch = g.get("general.architecture", "llama")
    if arch != "llama":
        raise GGUFError(f"{path}: architecture {arch!r} is not a llama model")
    emb = g.tensor("token_embd.weight")
    vocab, hidden = emb.shape
    cfg = LlamaConfig(
        n_layer=int(g.require("llama.block_count")),
        hidden=int(g.require("llama.embedding_length")),
        ffn=int(g.tensor("blk.0.ffn_gate.weight").shape[0]),
        n_head=int(g.require("llama.attention.head_count")),
        n_kv_head=int(g.get("llama.attention.head_count_kv", g.require("llama.attention.head_count"))),
        vocab=int(vocab),
        rope_theta=float(g.get("llama.rope.freq_base", 10000.0)),
        rms_eps=float(g.require("llama.attention.layer_norm_rms_epsilon")),
        max_seq=int(max_seq),
    )
    if hidden != cfg.hidden:
        raise GGUFError(f"{path}: token_embd width {hidden} != llama.embedding_length {cfg.hidden}")
    hw = HostWeights(cfg)
    for i in range(cfg.n_layer):
        hw.layers.append({k: g.qtensor(f"blk.{i}.{v}.weight") for k, v in _LAYER_NAMES.items()})
        hw.attn_norm.append(g.f32(f"blk.{i}.attn_norm.weight").astype(np.float32))
        hw.ffn_norm.append(g.f32(f"blk.{i}.ffn_norm.weight").astype(np.float32))
    hw.tok_embeddings = g.f32("token_embd.weight").astype(np.float32)
    hw.norm = g.f32("output_norm.weight").astype(np.float32)
    hw.output = g.qtensor("output.weight" if "output.weight" in g.tensors else "token_embd.weight")
    return cfg, hw


def save_llama(path: str, hw, embedding: QTensor | None = None, tie_output: bool = False) -> None:
    """Write host weights as a llama GGUF file (the layout load_llama reads).
    The embedding table is stored as F32, or as the given quantized blocks
    (`embedding`, shape (vocab, hidden)); tie_output leaves output.weight out,
    so a reader uses the embedding's blocks as the output head."""
    cfg = hw.cfg
    md = {
        "general.architecture": "llama",
        "general.name": "arm_ai_amd synthetic",
        "llama.block_count": cfg.n_layer,
        "llama.embedding_length": cfg.hidden,
        "llama.feed_forward_length": cfg.ffn,
        "llama.attention.head_count": cfg.n_head,
        "llama.attention.head_count_kv": cfg.n_kv_head,
        "llama.rope.dimension_count": cfg.head_dim,
        "llama.rope.freq_base": float(cfg.rope_theta),
        "llama.attention.layer_norm_rms_epsilon": float(cfg.rms_eps),
        "llama.context_length": cfg.max_seq,
    }
    ts = []
    if embedding is not None:
        ts.append(("token_embd.weight", (cfg.hidden, cfg.vocab), int(embedding.dtype), embedding.data))
    else:
        ts.append(("token_embd.weight", (cfg.hidden, cfg.vocab), GGML_F32, hw.tok_embeddings.astype("<f4")))
    ts.append(("output_norm.weight", (cfg.hidden,), GGML_F32, hw.norm.astype("<f4")))
    if hw.output is not None and not tie_output:
        n, k = hw.output.shape
        ts.append(("output.weight", (k, n), int(hw.output.dtype), hw.output.data))
    for i, layer in enumerate(hw.layers):
        for key, nm in _LAYER_NAMES.items():
            qt = layer[key]
            n, k = qt.shape
            ts.append((f"blk.{i}.{nm}.weight", (k, n), int(qt.dtype), qt.data))
        ts.append((f"blk.{i}.attn_norm.weight", (cfg.hidden,), GGML_F32, hw.attn_norm[i].astype("<f4")))
        ts.append((f"blk.{i}.ffn_norm.weight", (cfg.hidden,), GGML_F32, hw.ffn_norm[i].astype("<f4")))
    write_gguf(path, md, ts)
