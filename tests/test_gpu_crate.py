"""GPU parity of the NIF crate's int8 / int4 kernels (include/aq.h, "crate kernels").

Against the CPU restatement (oracle/crate_ops.c, pinned in
tests/test_crate_oracle.py): the int8 x int8 matmuls, the quantizers and the
dequantizers bit-exact; the weight-only f32 matmuls within the path's
tolerance (max relative error 1e-5, 1e-4 for K >= 14336), because their f32
sums are reordered.
"""
import numpy as np
import pytest

import arm_ai_amd as A
import oracle as O
from arm_ai_amd import crate_ops as C
from tests._metrics import tol_for_k

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(77)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("m,n,k", [(1, 300, 256), (3, 65, 37), (8, 128, 1000), (9, 40, 64), (40, 200, 96),
                                   (130, 70, 4096), (64, 4096, 4096), (33, 129, 64), (257, 300, 128),
                                   (512, 384, 1024)])
def test_int8_matmuls_bitexact(ctx, m, n, k):
    a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    ws = RNG.uniform(1e-4, 0.02, n).astype(np.float32)
    as_ = RNG.uniform(1e-4, 0.02, m).astype(np.float32)
    assert np.array_equal(C.int8_matmul_f32(ctx, a, w, ws, 0.0173, m, n, k), O.int8_matmul_f32(a, w, 0.0173, ws, m, n, k))
    assert np.array_equal(C.int8_matmul_f32_per_token(ctx, a, w, as_, ws, m, n, k),
                          O.int8_matmul_f32_per_token(a, w, as_, ws, m, n, k))


def test_int8_matmul_extreme_values(ctx):
    m, n, k = 33, 33, 4096  # |sum| up to 4096 * 127 * 128: exact in i32
    a = np.full((m, k), -128, np.int8)
    a[1::2] = 127
    w = np.full((n, k), -128, np.int8)
    ws = np.ones(n, np.float32)
    assert np.array_equal(C.int8_matmul_f32(ctx, a, w, ws, 1.0, m, n, k), O.int8_matmul_f32(a, w, 1.0, ws, m, n, k))


def test_quantize_int8_per_token_bitexact(ctx):
    x = (RNG.standard_normal((7, 1000)) * RNG.uniform(1e-3, 1e3, (7, 1))).astype(np.float32)
    x[1] = 0.0
    x[2, :8] = [127.0, -63.5, 0.5, 2.5, -2.5, 0.0, 1.49, -126.5]
    x[2, 8:] = 0.0
    x[3, 5] = np.nan
    x[4, ::3] = np.float32(1e-40)
    q, s = C.quantize_int8_per_token(ctx, x, 7, 1000)
    qo, so = O.quantize_int8_per_token(x, 7, 1000)
    assert np.array_equal(s, so) and np.array_equal(q, qo)


@pytest.mark.parametrize("b,m,n,k", [(1, 1, 512, 2048), (2, 3, 100, 100), (1, 9, 64, 37), (1, 2, 64, 14336)])
def test_weight_only_matmuls(ctx, b, m, n, k):
    act = RNG.standard_normal((b, m, k)).astype(np.float32)
    w8 = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    s8 = RNG.uniform(1e-3, 0.02, n).astype(np.float32)
    tol = tol_for_k(k)
    assert _rel(C.dequant_matmul_int8_f32(ctx, act, w8, s8, b, m, n, k), O.dequant_matmul_int8_f32(act, w8, s8, b, m, n, k)) <= tol
    wh = (RNG.standard_normal((n, k)) * 0.05).astype(np.float16)
    assert _rel(C.dequant_matmul_f16_f32(ctx, act, wh, b, m, n, k),
                O.dequant_matmul_f16_f32(act, wh.view(np.uint16), b, m, n, k)) <= tol


@pytest.mark.parametrize("m,n,k", [(1, 2048, 2048), (3, 100, 256), (9, 33, 4096), (1, 64, 14336)])
def test_int4_matmuls(ctx, m, n, k):
    packed = RNG.integers(0, 256, (n, k // 2)).astype(np.uint8)
    scales = RNG.uniform(1e-3, 0.05, (n, k // 32)).astype(np.float32)
    a = RNG.standard_normal((m, k)).astype(np.float32)
    tol = tol_for_k(k)
    assert _rel(C.int4_matmul_f32(ctx, a, packed, scales, m, n, k), O.int4_matmul_f32(a, packed, scales, m, n, k)) <= tol
    assert _rel(C.int4_matmul_gemv_neon(ctx, a[0], packed, scales, n, k), O.int4_matmul_gemv(a[0], packed, scales, n, k)) <= tol
    out = C.int4_matmul_gemv_q4_x_q8_neon(ctx, a[0], packed, scales, n, k)
    want, _, _ = O.int4_matmul_gemv_q4_x_q8(a[0], packed, scales, n, k)
    assert _rel(out, want) <= tol


def test_q4_x_q8_activation_quantisation_bitexact(ctx):
    from arm_ai_amd import hip

    n, k = 100, 1024
    packed = RNG.integers(0, 256, (n, k // 2)).astype(np.uint8)
    scales = RNG.uniform(1e-3, 0.05, (n, k // 32)).astype(np.float32)
    a = (RNG.standard_normal(k) * 4).astype(np.float32)
    a[64:96] = 0.0
    a[3] = np.nan
    a[200:232] = np.linspace(-2.5, 2.5, 32, dtype=np.float32)
    da, dp, ds = hip.to_device(a), hip.to_device(packed), hip.to_device(scales)
    dout = hip.DeviceBuffer(n * 4)
    act = hip.DeviceBuffer(int(A._lib.load().aq_q4_x_q8_act_bytes(k)))
    dq, dqs = hip.DeviceBuffer(k), hip.DeviceBuffer(k // 32 * 4)
    A._lib.check(A._lib.load().aq_int4_matmul_gemv_q4_x_q8_device(
        ctx.handle, da.ptr, dp.ptr, ds.ptr, n, k, dout.ptr, act.ptr, dq.ptr, dqs.ptr))
    ctx.synchronize()
    _, qo, so = O.int4_matmul_gemv_q4_x_q8(a, packed, scales, n, k)
    assert np.array_equal(dq.download(np.int8, (k,)), qo)
    assert np.array_equal(dqs.download(np.float32, (k // 32,)), so)


def test_quantize_int4_q4_0_bitexact(ctx):
    n, k = 37, 512
    w = (RNG.standard_normal((n, k)) * RNG.uniform(1e-3, 10, (n, 1))).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :8] = [7.0, -7.0, 3.5, -3.5, 0.5, -0.5, 2.49, 6.51]
    w[1, 8:32] = 0.0
    p, s = C.quantize_int4_q4_0(ctx, w, n, k)
    po, so = O.quantize_int4_q4_0(w, n, k)
    assert np.array_equal(s, so) and np.array_equal(p, po)


def test_dequantizers_bitexact(ctx):
    from arm_ai_amd import synth as S
    from arm_ai_amd import hip

    W = S.make_weight(S.TYPE_Q6_K, 6, 1024, seed=9)
    assert np.array_equal(C.dequantize_q6_k(ctx, W.blocks, 6 * 1024), O.dequantize_q6_k_crate(W.blocks, 6 * 1024))
    n, k = 5, 256
    packed = RNG.integers(0, 256, (n, k // 2)).astype(np.uint8)
    scales = RNG.uniform(1e-3, 0.05, (n, k // 32)).astype(np.float32)
    w8 = RNG.integers(-128, 128, (n, k)).astype(np.int8)
    for r in range(n):
        assert np.array_equal(C.q4_0_dequant_row(ctx, packed, scales, r, k), O.q4_0_dequant_row(packed, scales, r, k))
        assert np.array_equal(C.q8_0_dequant_row(ctx, w8, scales, r, k), O.q8_0_dequant_row(w8, scales, r, k))
    with pytest.raises(A.QMatMulError):
        C.q4_0_dequant_row(ctx, packed, scales, n, k)  # row out of range
    # batched device lookup; an out-of-range index gives a zero row
    rows = np.array([4, 0, 7, 2, -1], np.int64)
    dt, ds, dr = hip.to_device(packed), hip.to_device(scales), hip.to_device(rows)
    dout = hip.DeviceBuffer(rows.size * k * 4)
    A._lib.check(A._lib.load().aq_dequant_rows_device(ctx.handle, 0, dt.ptr, ds.ptr, n, dr.ptr, rows.size, k, dout.ptr))
    ctx.synchronize()
    got = dout.download(np.float32, (rows.size, k))
    for i, r in enumerate(rows):
        want = O.q4_0_dequant_row(packed, scales, r, k) if 0 <= r < n else np.zeros(k, np.float32)
        assert np.array_equal(got[i], want)


def test_crate_shape_errors(ctx):
    with pytest.raises(A.QMatMulError):
        C.int4_matmul_f32(ctx, np.zeros((1, 40), np.float32), np.zeros(20, np.uint8), np.zeros(1, np.float32), 1, 1, 40)
    with pytest.raises(A.QMatMulError):
        C.int8_matmul_f32(ctx, np.zeros(10, np.int8), np.zeros(10, np.int8), np.ones(1, np.float32), 1.0, 2, 1, 10)
    L = A._lib.load()
    assert L.aq_dequantize_q6_k(ctx.handle, None, 100, 256, None) == A._lib.AQ_ERR_SHAPE
    assert C.int8_matmul_f32(ctx, np.zeros(0, np.int8), np.zeros(16, np.int8), np.ones(1, np.float32), 1.0, 0, 1, 16).shape == (0, 1)
