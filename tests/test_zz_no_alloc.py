"""aq_qmatmul_f32_device_noalloc: the device-pointer matmul without any
allocation (its scratch is a fixed per-GPU array in the library image).

Called through the C ABI and checked against aq_qmatmul_f32_device, the
entry point it mirrors, on two calls in a row on the same weight: the first
with a prefill-sized input (the GEMM path, which needs the scratch), the
second with a smaller one (the array keeps the first call's contents, which
must not leak into the second's result).  The kernels are the same, so the
results must be identical to the bit.  Plus the one-row path, a Q6_K weight
(the f16 GEMM, whose workspace also holds the f16 copy of the quants), and
the size limit.
"""
import numpy as np
import pytest

import arm_ai_amd as A
import oracle as O
from arm_ai_amd import _lib, hip
from arm_ai_amd import synth as S

pytestmark = pytest.mark.gpu


def _both(ctx, mm, x):
    L = _lib.load()
    m, k = x.shape
    dx = hip.to_device(x)
    ya, yb = hip.DeviceBuffer(m * mm.n * 4), hip.DeviceBuffer(m * mm.n * 4)
    _lib.check(L.aq_qmatmul_f32_device(ctx.handle, mm.handle, dx.ptr, m, k, ya.ptr))
    _lib.check(L.aq_qmatmul_f32_device_noalloc(ctx.handle, mm.handle, dx.ptr, m, k, yb.ptr))
    ctx.synchronize()
    return ya.download(np.float32, (m, mm.n)), yb.download(np.float32, (m, mm.n))


@pytest.mark.parametrize("wtype,n,k,ms", [
    (S.TYPE_Q4_K, 2048, 5632, (64, 20, 1)),   # int8 GEMM, then a smaller GEMM, then the matvec
    (S.TYPE_Q6_K, 2048, 2048, (96, 33)),      # f16 GEMM (quants copied to f16 in the scratch)
    (S.TYPE_Q8_0, 1024, 4096, (48, 9)),       # Q8_0 GEMM (Q8_0 activation planes)
    (S.TYPE_Q4_K, 512, 14336, (8, 3)),        # batched matvec in K parts (the parts' sums in the scratch)
])
def test_noalloc_matches_the_allocating_entry(ctx, wtype, n, k, ms):
    W = S.make_weight(wtype, n, k, seed=n + k + wtype)
    mm = A.QMatMul.from_qtensor(A.QTensor(wtype, (n, k), W.blocks), ctx)
    for i, m in enumerate(ms):
        x = S.make_activation(m, k, seed=100 * i + m)
        ya, yb = _both(ctx, mm, x)
        assert np.array_equal(ya, yb), f"m={m}: the fixed-scratch call differs from the allocating one"
        r = O.matmul(wtype, x, W.blocks, n, k)
        tol = 1e-4 if k >= 14336 else 1e-5  # the parity bar for rows of 14336 and more
        assert float(np.abs(yb - r).max()) <= tol * float(np.abs(r).max())
    mm.free()


def test_noalloc_rejects_shapes_beyond_its_scratch(ctx):
    L = _lib.load()
    cap = L.aq_fixed_scratch_bytes()
    assert cap == 32 << 20
    k, n = 14336, 256
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=3)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (n, k), W.blocks), ctx)
    m = 4096  # the quantised activation alone (m * k * ~1.44 bytes) exceeds 32 MiB
    dx, dy = hip.DeviceBuffer(m * k * 4), hip.DeviceBuffer(m * n * 4)
    rc = L.aq_qmatmul_f32_device_noalloc(ctx.handle, mm.handle, dx.ptr, m, k, dy.ptr)
    assert rc == _lib.AQ_ERR_SHAPE
    assert b"fixed" in L.aq_last_error()
    # the same call through the allocating entry point still works afterwards
    x = S.make_activation(16, k, seed=4)
    ya, yb = _both(ctx, mm, x)
    assert np.array_equal(ya, yb)
    mm.free()
