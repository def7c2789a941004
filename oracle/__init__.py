"""ctypes front end of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  The C code
restates candle-core 0.8.4's quantized matmul (the path behind
native/arm_ai_nif/src/llama_candle.rs:93, :119); see oracle.h for the
per-function reference and how each is pinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
LIB_V3_PATH = os.path.join(HERE, "liboracle_v3.so")  # same source, x86-64-v3

Q2_K, Q3_K, Q4_0, Q5_0, Q4_K, Q5_K, Q6_K, Q8_0, Q8_K = 10, 11, 2, 6, 12, 13, 14, 8, 15
BLOCK_BYTES = {Q2_K: 84, Q3_K: 110, Q4_0: 18, Q5_0: 22, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34, Q8_K: 292}
BLOCK_ELEMS = {Q2_K: 256, Q3_K: 256, Q4_0: 32, Q5_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_0: 32, Q8_K: 256}

_libs: dict = {}


def build() -> str:
    """Compile liboracle.so (and liboracle_v3.so) with the Makefile (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def cpu_has_v3() -> bool:
    """True when this CPU runs x86-64-v3 code (AVX2, FMA, BMI2, F16C, MOVBE)."""
    try:
        flags = next(line for line in open("/proc/cpuinfo") if line.startswith("flags")).split()
    except (OSError, StopIteration):
        return False
    return all(f in flags for f in ("avx2", "fma", "bmi2", "f16c", "movbe", "bmi1"))


def lib(isa: str = "baseline") -> ctypes.CDLL:
    """The oracle library: the x86-64 baseline build, or isa="v3" for the x86-64-v3 build."""
    if isa not in _libs:
        path = LIB_PATH if isa == "baseline" else LIB_V3_PATH
        if isa != "baseline" and not cpu_has_v3():
            raise RuntimeError("this CPU cannot run the x86-64-v3 build")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32_n.argtypes = [P, i64, P]
        L.orc_f16_to_f32_n.restype = None
        L.orc_f32_to_f16_n.argtypes = [P, i64, P]
        L.orc_f32_to_f16_n.restype = None
        for f in ("orc_quantize_row_q8k", "orc_quantize_row_q8_0"):
            getattr(L, f).argtypes = [P, i64, P]
            getattr(L, f).restype = ctypes.c_int
        for f in ("orc_vec_dot_q2k_q8k", "orc_vec_dot_q3k_q8k", "orc_vec_dot_q4k_q8k", "orc_vec_dot_q5k_q8k", "orc_vec_dot_q6k_q8k", "orc_vec_dot_q8_0_q8_0",
                  "orc_vec_dot_q4_0_q8_0", "orc_vec_dot_q5_0_q8_0"):
            getattr(L, f).argtypes = [i64, P, P]
            getattr(L, f).restype = ctypes.c_float
        L.orc_block_sums.argtypes = [ctypes.c_int, i64, P, P, P, P]
        L.orc_block_sums.restype = None
        L.orc_block_sums_mat.argtypes = [ctypes.c_int, i64, i64, i64, P, P, P, P, ctypes.c_int]
        L.orc_block_sums_mat.restype = ctypes.c_int
        L.orc_matmul.argtypes = [ctypes.c_int, i64, i64, i64, P, P, P, ctypes.c_int]
        L.orc_matmul.restype = ctypes.c_int
        L.orc_matmul_preq.argtypes = [ctypes.c_int, i64, i64, i64, P, P, P, ctypes.c_int]
        L.orc_matmul_preq.restype = ctypes.c_int
        L.orc_dequantize_row.argtypes = [ctypes.c_int, P, i64, P]
        L.orc_dequantize_row.restype = ctypes.c_int
        L.orc_max_threads.argtypes = []
        L.orc_max_threads.restype = ctypes.c_int
        _libs[isa] = L
    return _libs[isa]


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, np.uint16).ravel()
    out = np.empty(b.size, np.float32)
    lib().orc_f16_to_f32_n(_p(b), b.size, _p(out))
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(f.size, np.uint16)
    lib().orc_f32_to_f16_n(_p(f), f.size, _p(out))
    return out


def act_type(wtype: int) -> int:
    return Q8_0 if wtype in (Q8_0, Q4_0, Q5_0) else Q8_K


def quantize(x: np.ndarray, atype: int = Q8_K) -> np.ndarray:
    """Quantise f32 rows [m, k] to Q8_K (or Q8_0) block bytes [m, k/blk*bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    blk, nbytes = BLOCK_ELEMS[atype], BLOCK_BYTES[atype]
    if k % blk:
        raise ValueError("k not a multiple of the block size")
    out = np.zeros((m, k // blk * nbytes), np.uint8)
    f = lib().orc_quantize_row_q8k if atype == Q8_K else lib().orc_quantize_row_q8_0
    for r in range(m):
        rc = f(_p(x[r]), k, out[r].ctypes.data)
        assert rc == 0
    return out


def q8k_fields(blocks: np.ndarray):
    """Split Q8_K block bytes [..., nb*292] into (d f32 [..,nb], qs i8 [..,nb,256], bsums i16 [..,nb,16])."""
    b = np.ascontiguousarray(blocks).reshape(*blocks.shape[:-1], -1, 292)
    d = b[..., 0:4].copy().view(np.float32)[..., 0]
    qs = b[..., 4:260].copy().view(np.int8)
    bs = b[..., 260:292].copy().view(np.int16)
    return d, qs, bs


def q8_0_fields(blocks: np.ndarray):
    b = np.ascontiguousarray(blocks).reshape(*blocks.shape[:-1], -1, 34)
    d = b[..., 0:2].copy().view(np.float16)[..., 0]
    qs = b[..., 2:34].copy().view(np.int8)
    return d, qs


def vec_dot(wtype: int, k: int, wrow: np.ndarray, xq_row: np.ndarray) -> float:
    L = lib()
    f = {Q2_K: L.orc_vec_dot_q2k_q8k, Q3_K: L.orc_vec_dot_q3k_q8k, Q4_K: L.orc_vec_dot_q4k_q8k, Q5_K: L.orc_vec_dot_q5k_q8k, Q6_K: L.orc_vec_dot_q6k_q8k,
         Q8_0: L.orc_vec_dot_q8_0_q8_0, Q4_0: L.orc_vec_dot_q4_0_q8_0, Q5_0: L.orc_vec_dot_q5_0_q8_0}[wtype]
    wrow = np.ascontiguousarray(wrow)
    xq_row = np.ascontiguousarray(xq_row)
    return float(f(k, _p(wrow), _p(xq_row)))


def _row_bytes(wtype: int, k: int) -> int:
    if wtype not in BLOCK_ELEMS:
        raise ValueError(f"unsupported GGML type {wtype}")
    if k <= 0 or k % BLOCK_ELEMS[wtype]:
        raise ValueError(f"k={k} is not a multiple of the block size {BLOCK_ELEMS[wtype]}")
    return k // BLOCK_ELEMS[wtype] * BLOCK_BYTES[wtype]


def _rows_of(buf: np.ndarray, row_bytes: int, what: str) -> int:
    """Row count of a buffer of whole rows (any shape); the C code trusts it."""
    if buf.nbytes % row_bytes:
        raise ValueError(f"{what}: {buf.nbytes} bytes is not a whole number of {row_bytes}-byte rows")
    return buf.nbytes // row_bytes


def block_sums(wtype: int, k: int, w: np.ndarray, xq: np.ndarray, nthreads: int = 0):
    """Integer sums per (m, n, block): returns S, Smin int32 [m, n, nb]."""
    w = np.ascontiguousarray(w)
    xq = np.ascontiguousarray(xq)
    n = _rows_of(w, _row_bytes(wtype, k), "weight")
    m = _rows_of(xq, _row_bytes(act_type(wtype), k), "quantised activation")
    nb = k // BLOCK_ELEMS[wtype]
    S = np.zeros((m, n, nb), np.int32)
    Sm = np.zeros((m, n, nb), np.int32)
    rc = lib().orc_block_sums_mat(wtype, m, n, k, _p(w), _p(xq), _p(S), _p(Sm), nthreads)
    if rc != 0:
        raise ValueError(f"orc_block_sums_mat failed: {rc}")
    return S, Sm


def matmul(wtype: int, x: np.ndarray, w: np.ndarray, n: int, k: int, nthreads: int = 0,
           isa: str = "baseline") -> np.ndarray:
    """k_quants::matmul: f32 [m, k] x W[n, k]^T -> f32 [m, n]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m = x.shape[0]
    if x.shape[1] != k:
        raise ValueError(f"x has {x.shape[1]} columns, k={k}")
    w = np.ascontiguousarray(w)
    if w.nbytes != n * _row_bytes(wtype, k):
        raise ValueError(f"weight has {w.nbytes} bytes, {n} rows of k={k} need {n * _row_bytes(wtype, k)}")
    dst = np.zeros((m, n), np.float32)
    rc = lib(isa).orc_matmul(wtype, m, k, n, _p(x), _p(w), _p(dst), nthreads)
    if rc != 0:
        raise ValueError(f"orc_matmul failed: {rc}")
    return dst


def matmul_preq(wtype: int, xq: np.ndarray, w: np.ndarray, n: int, k: int, nthreads: int = 0) -> np.ndarray:
    xq = np.ascontiguousarray(xq)
    w = np.ascontiguousarray(w)
    m = _rows_of(xq, _row_bytes(act_type(wtype), k), "quantised activation")
    if w.nbytes != n * _row_bytes(wtype, k):
        raise ValueError(f"weight has {w.nbytes} bytes, {n} rows of k={k} need {n * _row_bytes(wtype, k)}")
    dst = np.zeros((m, n), np.float32)
    rc = lib().orc_matmul_preq(wtype, m, k, n, _p(xq), _p(dst), _p(w), nthreads)
    if rc != 0:
        raise ValueError(f"orc_matmul_preq failed: {rc}")
    return dst


def dequantize(wtype: int, w: np.ndarray, k: int) -> np.ndarray:
    w = np.ascontiguousarray(w)
    out = np.zeros((w.shape[0], k), np.float32)
    for r in range(w.shape[0]):
        rc = lib().orc_dequantize_row(wtype, w[r].ctypes.data, k, out[r].ctypes.data)
        assert rc == 0
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())


# ---------------------------------------------------------------------------
# The NIF crate's own int8 / int4 kernels (crate_ops.c, restating
# native/arm_ai_nif/src/shape_ops.rs; see the C comments for line numbers).
# ---------------------------------------------------------------------------
def _crate_lib() -> ctypes.CDLL:
    L = lib()
    if getattr(L, "_crate_ready", False):
        return L
    P, i64, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
    sigs = {
        "orc_int8_matmul_f32": [P, P, f32, P, i64, i64, i64, P],
        "orc_int8_matmul_f32_per_token": [P, P, P, P, i64, i64, i64, P],
        "orc_quantize_int8_per_token": [P, i64, i64, P, P],
        "orc_dequant_matmul_int8_f32": [P, P, P, i64, i64, i64, i64, P],
        "orc_dequant_matmul_f16_f32": [P, P, i64, i64, i64, i64, P],
        "orc_int4_matmul_f32": [P, P, P, i64, i64, i64, P],
        "orc_int4_matmul_gemv": [P, P, P, i64, i64, P],
        "orc_quantize_q8_groups": [P, i64, P, P],
        "orc_int4_matmul_gemv_q4_x_q8": [P, P, P, i64, i64, P, P, P],
        "orc_quantize_int4_q4_0": [P, i64, i64, P, P],
        "orc_dequantize_q6_k_crate": [P, i64, P],
        "orc_q4_0_dequant_row": [P, P, i64, i64, P],
        "orc_q8_0_dequant_row": [P, P, i64, i64, P],
    }
    for name, args in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = None
    L._crate_ready = True
    return L


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def int8_matmul_f32(a, w, act_scale, w_scales, m, n, k):
    a, w, ws = _c(a, np.int8), _c(w, np.int8), _c(w_scales, np.float32)
    out = np.zeros((m, n), np.float32)
    _crate_lib().orc_int8_matmul_f32(_p(a), _p(w), float(act_scale), _p(ws), m, n, k, _p(out))
    return out


def int8_matmul_f32_per_token(a, w, act_scales, w_scales, m, n, k):
    a, w = _c(a, np.int8), _c(w, np.int8)
    as_, ws = _c(act_scales, np.float32), _c(w_scales, np.float32)
    out = np.zeros((m, n), np.float32)
    _crate_lib().orc_int8_matmul_f32_per_token(_p(a), _p(w), _p(as_), _p(ws), m, n, k, _p(out))
    return out


def quantize_int8_per_token(a, m, k):
    a = _c(a, np.float32)
    q = np.zeros((m, k), np.int8)
    s = np.zeros(m, np.float32)
    _crate_lib().orc_quantize_int8_per_token(_p(a), m, k, _p(q), _p(s))
    return q, s


def dequant_matmul_int8_f32(act, w, scales, b, m, n, k):
    act, w, s = _c(act, np.float32), _c(w, np.int8), _c(scales, np.float32)
    out = np.zeros((b, m, n), np.float32)
    _crate_lib().orc_dequant_matmul_int8_f32(_p(act), _p(w), _p(s), b, m, n, k, _p(out))
    return out


def dequant_matmul_f16_f32(act, w_f16bits, b, m, n, k):
    act, w = _c(act, np.float32), _c(w_f16bits, np.uint16)
    out = np.zeros((b, m, n), np.float32)
    _crate_lib().orc_dequant_matmul_f16_f32(_p(act), _p(w), b, m, n, k, _p(out))
    return out


def int4_matmul_f32(a, w_packed, w_scales, m, n, k):
    a, wp, ws = _c(a, np.float32), _c(w_packed, np.uint8), _c(w_scales, np.float32)
    out = np.zeros((m, n), np.float32)
    _crate_lib().orc_int4_matmul_f32(_p(a), _p(wp), _p(ws), m, n, k, _p(out))
    return out


def int4_matmul_gemv(a, w_packed, w_scales, n, k):
    a, wp, ws = _c(a, np.float32), _c(w_packed, np.uint8), _c(w_scales, np.float32)
    out = np.zeros(n, np.float32)
    _crate_lib().orc_int4_matmul_gemv(_p(a), _p(wp), _p(ws), n, k, _p(out))
    return out


def quantize_q8_groups(a, k):
    a = _c(a, np.float32)
    q = np.zeros(k, np.int8)
    s = np.zeros(k // 32, np.float32)
    _crate_lib().orc_quantize_q8_groups(_p(a), k, _p(q), _p(s))
    return q, s


def int4_matmul_gemv_q4_x_q8(a, w_packed, w_scales, n, k):
    """Returns (out [n], quantised activation i8 [k], its group scales [k/32])."""
    a, wp, ws = _c(a, np.float32), _c(w_packed, np.uint8), _c(w_scales, np.float32)
    out = np.zeros(n, np.float32)
    q = np.zeros(k, np.int8)
    s = np.zeros(k // 32, np.float32)
    _crate_lib().orc_int4_matmul_gemv_q4_x_q8(_p(a), _p(wp), _p(ws), n, k, _p(out), _p(q), _p(s))
    return out, q, s


def quantize_int4_q4_0(w, n, k):
    w = _c(w, np.float32)
    packed = np.zeros((n, k // 2), np.uint8)
    scales = np.zeros((n, k // 32), np.float32)
    _crate_lib().orc_quantize_int4_q4_0(_p(w), n, k, _p(packed), _p(scales))
    return packed, scales


def dequantize_q6_k_crate(blocks, n_elements):
    b = _c(blocks, np.uint8).ravel()
    nb = n_elements // 256
    out = np.zeros(nb * 256, np.float32)
    _crate_lib().orc_dequantize_q6_k_crate(_p(b), nb, _p(out))
    return out


def q4_0_dequant_row(packed, scales, row, k):
    p, s = _c(packed, np.uint8), _c(scales, np.float32)
    out = np.zeros(k, np.float32)
    _crate_lib().orc_q4_0_dequant_row(_p(p), _p(s), row, k, _p(out))
    return out


def q8_0_dequant_row(w, scales, row, k):
    w, s = _c(w, np.int8), _c(scales, np.float32)
    out = np.zeros(k, np.float32)
    _crate_lib().orc_q8_0_dequant_row(_p(w), _p(s), row, k, _p(out))
    return out
