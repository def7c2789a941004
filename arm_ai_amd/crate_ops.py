"""Host-side mirror of the NIF crate's int8 / int4 operators over the C ABI.

The reference exposes these as NIFs (native/arm_ai_nif/src/lib.rs:172-532)
over kernels in native/arm_ai_nif/src/shape_ops.rs; each function here keeps
the NIF's name (without the ``_op`` suffix), argument order and meaning,
takes numpy arrays for the binaries and returns numpy arrays, and runs on the
GPU through include/aq.h ("crate kernels").  Shape errors raise
``QMatMulError`` where the crate returns an error string.
"""
from __future__ import annotations

import numpy as np

from . import _lib
from .qmatmul import Context, QMatMulError


def _arr(x, dtype, size, what):
    a = np.ascontiguousarray(x, dtype=dtype).reshape(-1)
    if a.size != size:
        raise QMatMulError(f"{what}: {a.size} elements, expected {size}")
    return a


def _call(fn, *args):
    try:
        _lib.check(fn(*args))
    except _lib.AqError as e:
        if e.code in (_lib.AQ_ERR_SHAPE, _lib.AQ_ERR_INVALID_ARG):
            raise QMatMulError(str(e)) from None
        raise


def int8_matmul_f32(ctx: Context, a, w, w_scales, act_scale: float, m: int, n: int, k: int) -> np.ndarray:
    """out[m, n] = (sum_k a*w) * act_scale * w_scales[n] (shape_ops.rs:1169-1211)."""
    a = _arr(a, np.int8, m * k, "int8_matmul: a")
    w = _arr(w, np.int8, n * k, "int8_matmul: w")
    ws = _arr(w_scales, np.float32, n, "int8_matmul: w_scales")
    out = np.empty((m, n), np.float32)
    _call(_lib.load().aq_int8_matmul_f32, ctx.handle, a.ctypes.data, w.ctypes.data, ws.ctypes.data, float(act_scale),
          m, n, k, out.ctypes.data)
    return out


def int8_matmul_f32_per_token(ctx: Context, a, w, act_scales, w_scales, m: int, n: int, k: int) -> np.ndarray:
    """out[m, n] = (sum_k a*w) * act_scales[m] * w_scales[n] (shape_ops.rs:1222-1264)."""
    a = _arr(a, np.int8, m * k, "int8_matmul_per_token: a")
    w = _arr(w, np.int8, n * k, "int8_matmul_per_token: w")
    as_ = _arr(act_scales, np.float32, m, "int8_matmul_per_token: act_scales")
    ws = _arr(w_scales, np.float32, n, "int8_matmul_per_token: w_scales")
    out = np.empty((m, n), np.float32)
    _call(_lib.load().aq_int8_matmul_f32_per_token, ctx.handle, a.ctypes.data, w.ctypes.data, as_.ctypes.data,
          ws.ctypes.data, m, n, k, out.ctypes.data)
    return out


def quantize_int8_per_token(ctx: Context, a, m: int, k: int):
    """(q i8 [m, k], scales f32 [m]) (shape_ops.rs:1273-1292)."""
    a = _arr(a, np.float32, m * k, "quantize_int8_per_token: a")
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    _call(_lib.load().aq_quantize_int8_per_token, ctx.handle, a.ctypes.data, m, k, q.ctypes.data, s.ctypes.data)
    return q, s


def dequant_matmul_int8_f32(ctx: Context, act, weights, scales, b: int, m: int, n: int, k: int) -> np.ndarray:
    """out[b, m, n] = (sum_k act * w) * scales[n] (shape_ops.rs:1525-1582)."""
    act = _arr(act, np.float32, b * m * k, "dequant_matmul_int8: act")
    w = _arr(weights, np.int8, n * k, "dequant_matmul_int8: weights")
    s = _arr(scales, np.float32, n, "dequant_matmul_int8: scales")
    out = np.empty((b, m, n), np.float32)
    _call(_lib.load().aq_dequant_matmul_int8_f32, ctx.handle, act.ctypes.data, w.ctypes.data, s.ctypes.data, b, m, n,
          k, out.ctypes.data)
    return out


def dequant_matmul_f16_f32(ctx: Context, act, weights_f16, b: int, m: int, n: int, k: int) -> np.ndarray:
    """f16 weights (IEEE binary16 bits or float16 values) (shape_ops.rs:1386-1490)."""
    act = _arr(act, np.float32, b * m * k, "dequant_matmul_f16: act")
    wf = np.asarray(weights_f16)
    w = _arr(wf.view(np.uint16) if wf.dtype == np.float16 else wf, np.uint16, n * k, "dequant_matmul_f16: weights")
    out = np.empty((b, m, n), np.float32)
    _call(_lib.load().aq_dequant_matmul_f16_f32, ctx.handle, act.ctypes.data, w.ctypes.data, b, m, n, k,
          out.ctypes.data)
    return out


def int4_matmul_f32(ctx: Context, a, w_packed, w_scales, m: int, n: int, k: int) -> np.ndarray:
    """Q4_0-style int4 weights (shape_ops.rs:3175-3236)."""
    if k % 32:
        raise QMatMulError(f"int4_matmul: K={k} must be multiple of 32")
    a = _arr(a, np.float32, m * k, "int4_matmul: a")
    wp = _arr(w_packed, np.uint8, n * (k // 2), "int4_matmul: packed")
    ws = _arr(w_scales, np.float32, n * (k // 32), "int4_matmul: scales")
    out = np.empty((m, n), np.float32)
    _call(_lib.load().aq_int4_matmul_f32, ctx.handle, a.ctypes.data, wp.ctypes.data, ws.ctypes.data, m, n, k,
          out.ctypes.data)
    return out


def int4_matmul_gemv_neon(ctx: Context, a, w_packed, w_scales, n: int, k: int) -> np.ndarray:
    """M = 1 form of int4_matmul_f32 (shape_ops.rs:3059-3166)."""
    return int4_matmul_f32(ctx, a, w_packed, w_scales, 1, n, k)[0]


def int4_matmul_gemv_q4_x_q8_neon(ctx: Context, a, w_packed, w_scales, n: int, k: int) -> np.ndarray:
    """Q4_0 weights x Q8-quantised activation GEMV (shape_ops.rs:2923-3028)."""
    if k % 32:
        raise QMatMulError(f"int4_matmul: K={k} must be multiple of 32")
    a = _arr(a, np.float32, k, "q4_x_q8: a")
    wp = _arr(w_packed, np.uint8, n * (k // 2), "q4_x_q8: packed")
    ws = _arr(w_scales, np.float32, n * (k // 32), "q4_x_q8: scales")
    out = np.empty(n, np.float32)
    _call(_lib.load().aq_int4_matmul_gemv_q4_x_q8, ctx.handle, a.ctypes.data, wp.ctypes.data, ws.ctypes.data, n, k,
          out.ctypes.data)
    return out


def quantize_int4_q4_0(ctx: Context, w, n: int, k: int):
    """(packed u8 [n, k/2], scales f32 [n, k/32]) (shape_ops.rs:3242-3275)."""
    if k % 32:
        raise QMatMulError(f"quantize_int4: K={k} must be multiple of 32")
    w = _arr(w, np.float32, n * k, "quantize_int4: w")
    packed = np.empty((n, k // 2), np.uint8)
    scales = np.empty((n, k // 32), np.float32)
    _call(_lib.load().aq_quantize_int4_q4_0, ctx.handle, w.ctypes.data, n, k, packed.ctypes.data, scales.ctypes.data)
    return packed, scales


def dequantize_q6_k(ctx: Context, blocks, n_elements: int) -> np.ndarray:
    """The crate's Q6_K dequantizer, its sub-scale indexing included (shape_ops.rs:2848-2899)."""
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    out = np.empty(n_elements, np.float32)
    _call(_lib.load().aq_dequantize_q6_k, ctx.handle, b.ctypes.data, b.size, n_elements, out.ctypes.data)
    return out


def q4_0_dequant_row(ctx: Context, packed, scales, row: int, k: int) -> np.ndarray:
    """Row `row` of a Q4_0-style table (shape_ops.rs:2780-2808)."""
    p = np.ascontiguousarray(packed, np.uint8).reshape(-1)
    s = np.ascontiguousarray(scales, np.float32).reshape(-1)
    n_rows = p.size // (k // 2) if k % 32 == 0 else 0
    out = np.empty(k, np.float32)
    _call(_lib.load().aq_q4_0_dequant_row, ctx.handle, p.ctypes.data, s.ctypes.data, n_rows, row, k, out.ctypes.data)
    return out


def q8_0_dequant_row(ctx: Context, weights, scales, row: int, k: int) -> np.ndarray:
    """Row `row` of an int8 table with a scale per 32 (shape_ops.rs:2812-2832)."""
    w = np.ascontiguousarray(weights, np.int8).reshape(-1)
    s = np.ascontiguousarray(scales, np.float32).reshape(-1)
    n_rows = w.size // k if k > 0 else 0
    out = np.empty(k, np.float32)
    _call(_lib.load().aq_q8_0_dequant_row, ctx.handle, w.ctypes.data, s.ctypes.data, n_rows, row, k, out.ctypes.data)
    return out
