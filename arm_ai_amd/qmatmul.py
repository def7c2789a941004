"""Host-side mirror of candle's QTensor / QMatMul over the C ABI (include/aq.h).

In the reference, ArmAI.LlamaCandle's NIF (native/arm_ai_nif/src/llama_candle.rs)
builds candle `QTensor`s from a GGUF file (:37-43) and every projection is a
`QMatMul` whose `forward(&Tensor)` ends in
`QuantizedType::matmul_t((m, k, n), lhs, dst)` (candle-core 0.8.4).  This module
keeps those names and their argument meaning:

* ``QTensor(dtype, (n, k), blocks)``: raw GGUF blocks of an (n, k) weight.
* ``QMatMul.from_qtensor(qt, ctx)``: uploads the blocks to HBM once.
* ``QMatMul.forward(xs)``: xs is f32 ``[..., k]`` (rank >= 2, C-contiguous),
  returns f32 ``[..., n]``; the activation is quantised to Q8_K (Q8_0 for
  Q8_0 and Q4_0 weights) and the dot products run on the GPU.

candle's checks are kept with the same outcome (an error, never a crash):
a non-contiguous input, rank < 2, or a last dimension different from k.
"""
from __future__ import annotations

import ctypes
from enum import IntEnum

import numpy as np

from . import _lib


class GgmlDType(IntEnum):
    """GGUF/GGML dtype ids, named as in candle's `GgmlDType`."""

    Q4_0 = 2
    Q5_0 = 6
    Q8_0 = 8
    Q2K = 10
    Q3K = 11
    Q4K = 12
    Q5K = 13
    Q6K = 14
    Q8K = 15

    @property
    def block_size(self) -> int:
        return 32 if self in (GgmlDType.Q8_0, GgmlDType.Q4_0, GgmlDType.Q5_0) else 256

    @property
    def type_size(self) -> int:
        return {GgmlDType.Q4_0: 18, GgmlDType.Q5_0: 22, GgmlDType.Q8_0: 34, GgmlDType.Q2K: 84, GgmlDType.Q3K: 110, GgmlDType.Q4K: 144,
                GgmlDType.Q5K: 176, GgmlDType.Q6K: 210, GgmlDType.Q8K: 292}[self]


class QMatMulError(ValueError):
    """Mirrors candle's `Error` for the conditions QTensor::cpu_fwd rejects."""


def device_count() -> int:
    n = ctypes.c_int(0)
    _lib.check(_lib.load().aq_device_count(ctypes.byref(n)))
    return n.value


class Context:
    """One device, one HIP stream, grow-only scratch (aq_ctx)."""

    def __init__(self, device: int = 0):
        L = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(L.aq_ctx_create(device, ctypes.byref(h)))
        self._h = h
        self.device = device

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("context closed")
        return self._h

    @property
    def stream(self) -> int:
        s = ctypes.c_void_p()
        _lib.check(_lib.load().aq_ctx_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    def synchronize(self) -> None:
        _lib.check(_lib.load().aq_ctx_synchronize(self.handle))

    def close(self) -> None:
        if self._h is not None:
            _lib.load().aq_ctx_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QTensor:
    """Raw GGUF blocks of a weight of shape (n, k) (candle: QTensor)."""

    def __init__(self, dtype: GgmlDType | int, shape: tuple[int, int], data: np.ndarray | bytes):
        self.dtype = GgmlDType(dtype)
        n, k = (int(s) for s in shape)
        if k % self.dtype.block_size:
            raise QMatMulError(f"quantized tensor last dim {k} is not divisible by block size {self.dtype.block_size}")
        buf = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) else np.asarray(data, np.uint8)
        buf = np.ascontiguousarray(buf).reshape(-1)
        want = n * (k // self.dtype.block_size) * self.dtype.type_size
        if buf.size != want:
            raise QMatMulError(f"got {buf.size} bytes for a {self.dtype.name} tensor of shape ({n}, {k}), expected {want}")
        self.shape = (n, k)
        self.data = buf

    def storage_size_in_bytes(self) -> int:
        return int(self.data.size)


class QMatMul:
    """candle's `QMatMul::QTensor` variant, executed on one MI355X."""

    def __init__(self, ctx: Context, handle: ctypes.c_void_p, dtype: GgmlDType, shape: tuple[int, int]):
        self.ctx = ctx
        self._h = handle
        self.dtype = dtype
        self.n, self.k = shape

    @classmethod
    def from_qtensor(cls, qt: QTensor, ctx: Context) -> "QMatMul":
        L = _lib.load()
        h = ctypes.c_void_p()
        n, k = qt.shape
        _lib.check(
            L.aq_qweight_upload(ctx.handle, int(qt.dtype), qt.data.ctypes.data, qt.data.size, n, k, ctypes.byref(h))
        )
        return cls(ctx, h, qt.dtype, qt.shape)

    @classmethod
    def from_device_blocks(cls, ctx: Context, dtype: GgmlDType | int, shape, d_ptr: int, nbytes: int) -> "QMatMul":
        L = _lib.load()
        h = ctypes.c_void_p()
        n, k = shape
        _lib.check(L.aq_qweight_upload_device(ctx.handle, int(dtype), d_ptr, nbytes, n, k, ctypes.byref(h)))
        return cls(ctx, h, GgmlDType(dtype), (n, k))

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("weight freed")
        return self._h

    def device_bytes(self) -> int:
        sz = ctypes.c_size_t()
        _lib.check(_lib.load().aq_qweight_info(self.handle, None, None, None, ctypes.byref(sz)))
        return sz.value

    def _check_input(self, xs: np.ndarray) -> np.ndarray:
        if not isinstance(xs, np.ndarray) or xs.dtype != np.float32:
            raise QMatMulError("QMatMul input must be an f32 array")
        if not xs.flags["C_CONTIGUOUS"]:
            raise QMatMulError(f"input tensor is not contiguous {xs.shape}")
        if xs.ndim < 2:
            raise QMatMulError(f"input tensor has only one dimension {xs.shape}")
        if xs.shape[-1] != self.k:
            raise QMatMulError(f"input tensor {xs.shape} incompatible with {(self.n, self.k)}")
        return xs

    def forward(self, xs: np.ndarray) -> np.ndarray:
        xs = self._check_input(xs)
        m = int(np.prod(xs.shape[:-1]))
        dst = np.empty(xs.shape[:-1] + (self.n,), np.float32)
        _lib.check(_lib.load().aq_qmatmul_f32(self.ctx.handle, self.handle, xs.ctypes.data, m, self.k, dst.ctypes.data))
        return dst

    def forward_device(self, d_x: int, m: int, d_y: int) -> None:
        """Device-pointer variant (asynchronous on the context stream)."""
        _lib.check(_lib.load().aq_qmatmul_f32_device(self.ctx.handle, self.handle, d_x, m, self.k, d_y))

    @property
    def act_type(self) -> GgmlDType:
        return GgmlDType.Q8_0 if self.dtype in (GgmlDType.Q8_0, GgmlDType.Q4_0, GgmlDType.Q5_0) else GgmlDType.Q8K

    def forward_preq_device(self, d_act: int, m: int, d_y: int) -> None:
        """Matmul on an activation quantised by quantize_act_device (asynchronous)."""
        _lib.check(_lib.load().aq_qmatmul_preq_device(self.ctx.handle, self.handle, d_act, m, self.k, d_y))

    def block_sums(self, xs: np.ndarray):
        """Per-block integer sums S, Smin ([m, n, nblk] int32) from the GPU kernels."""
        xs = self._check_input(xs)
        m = int(np.prod(xs.shape[:-1]))
        nblk = self.k // self.dtype.block_size
        S = np.empty((m, self.n, nblk), np.int32)
        Sm = np.empty((m, self.n, nblk), np.int32)
        _lib.check(
            _lib.load().aq_qmatmul_block_sums(
                self.ctx.handle, self.handle, xs.ctypes.data, m, self.k, S.ctypes.data, Sm.ctypes.data
            )
        )
        return S, Sm

    def free(self) -> None:
        if self._h is not None:
            _lib.load().aq_qweight_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def act_bytes(act_type: GgmlDType | int, m: int, k: int) -> int:
    return int(_lib.load().aq_act_bytes(int(act_type), m, k))


def quantize_act_device(ctx: Context, act_type: GgmlDType | int, d_x: int, m: int, k: int, d_act: int) -> None:
    """Quantise device f32 [m, k] into a device activation buffer (asynchronous)."""
    _lib.check(_lib.load().aq_quantize_act_device(ctx.handle, int(act_type), d_x, m, k, d_act))


def quantize_q8k(ctx: Context, x: np.ndarray) -> np.ndarray:
    """BlockQ8K::from_float on the GPU: f32 [m, k] -> uint8 [m, k/256*292]."""
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None]
    m, k = x.shape
    out = np.empty((m, (k // 256) * 292), np.uint8)
    _lib.check(_lib.load().aq_quantize_q8k(ctx.handle, x.ctypes.data, m, k, out.ctypes.data))
    return out


def quantize_q8_0(ctx: Context, x: np.ndarray) -> np.ndarray:
    """BlockQ8_0::from_float on the GPU: f32 [m, k] -> uint8 [m, k/32*34]."""
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None]
    m, k = x.shape
    out = np.empty((m, (k // 32) * 34), np.uint8)
    _lib.check(_lib.load().aq_quantize_q8_0(ctx.handle, x.ctypes.data, m, k, out.ctypes.data))
    return out
