"""Pins of the CPU restatement of the NIF crate's int8 / int4 kernels (oracle/crate_ops.c).

The reference holds no tests or fixtures for these functions (their caller is
an external package), so each is pinned by what the mathematics fixes:
integer dots against numpy's int64 products, f32 accumulations against f64
sums of the same terms, quantizers by known answers (Rust's ties-away
rounding, clamps, the zero-row scale of 1) and invariants, the Q4_0 packing
by a round trip, and the crate's Q6_K dequantizer against the GGML one on
blocks where its sub-scale indexing cannot matter.  Planted mistakes (a
transposed operand, swapped nibbles) must fail.
"""
import numpy as np
import pytest

import oracle as O
from arm_ai_amd import synth as S

RNG = np.random.default_rng(2024)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ------------------------------------------------------------- int8 x int8
@pytest.mark.parametrize("m,n,k", [(1, 7, 16), (3, 5, 37), (4, 9, 128)])
def test_int8_matmuls_integer_part_and_scaling(m, n, k):
    a = RNG.integers(-127, 128, (m, k)).astype(np.int8)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    acc = a.astype(np.int64) @ w.astype(np.int64).T  # exact
    ws = RNG.uniform(0.001, 0.02, n).astype(np.float32)
    as_ = RNG.uniform(0.001, 0.02, m).astype(np.float32)
    got = O.int8_matmul_f32(a, w, 0.0125, ws, m, n, k)
    want = (acc.astype(np.float32) * np.float32(0.0125)) * ws[None, :]
    assert np.array_equal(got, want)
    got2 = O.int8_matmul_f32_per_token(a, w, as_, ws, m, n, k)
    want2 = (acc.astype(np.float32) * as_[:, None]) * ws[None, :]
    assert np.array_equal(got2, want2)
    if m == n:  # a planted transposition must not pass
        assert not np.array_equal(O.int8_matmul_f32(w, a, 0.0125, ws, m, n, k), want)


def test_quantize_int8_per_token_known_answers():
    row = np.array([127.0, -63.5, 0.5, 2.5, -2.5, 0.0, 1.49, -126.5], np.float32)
    q, s = O.quantize_int8_per_token(row, 1, row.size)
    assert s[0] == np.float32(1.0)
    assert q[0].tolist() == [127, -64, 1, 3, -3, 0, 1, -127]  # ties away from zero
    q, s = O.quantize_int8_per_token(np.zeros((2, 5), np.float32), 2, 5)
    assert s.tolist() == [1.0, 1.0] and not q.any()  # zero rows: scale 1
    row = np.array([1.0, np.nan, -1.0, 0.25], np.float32)
    q, s = O.quantize_int8_per_token(row, 1, 4)
    assert s[0] == np.float32(1.0) / np.float32(127.0) and q[0].tolist() == [127, 0, -127, 32]


def test_quantize_int8_per_token_invariants():
    x = (RNG.standard_normal((6, 300)) * RNG.uniform(0.01, 100, (6, 1))).astype(np.float32)
    q, s = O.quantize_int8_per_token(x, 6, 300)
    assert np.all(np.abs(q.astype(int)) <= 127)
    amax = np.max(np.abs(x), axis=1)
    assert np.allclose(s, amax / 127.0, rtol=1e-7)
    assert np.all(np.abs(np.abs(q[np.arange(6), np.argmax(np.abs(x), axis=1)]).astype(int)) == 127)
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert np.all(err <= s[:, None] * 0.5 * (1 + 1e-5))


# ------------------------------------------------------- weight-only f32 paths
@pytest.mark.parametrize("b,m,n,k", [(1, 1, 9, 64), (2, 3, 5, 100)])
def test_dequant_matmuls_against_f64(b, m, n, k):
    act = RNG.standard_normal((b, m, k)).astype(np.float32)
    w = RNG.integers(-127, 128, (n, k)).astype(np.int8)
    s = RNG.uniform(0.001, 0.02, n).astype(np.float32)
    got = O.dequant_matmul_int8_f32(act, w, s, b, m, n, k)
    want = (act.astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64)
    assert _rel(got, want) < 1e-5
    wh = (RNG.standard_normal((n, k)) * 0.05).astype(np.float16)
    got = O.dequant_matmul_f16_f32(act, wh.view(np.uint16), b, m, n, k)
    want = act.astype(np.float64) @ wh.astype(np.float64).T
    assert _rel(got, want) < 1e-5
    # small integers: every partial sum is exact in f32, so the result is exact
    ai = RNG.integers(-8, 9, (b, m, k)).astype(np.float32)
    wi = RNG.integers(-8, 9, (n, k)).astype(np.float16)
    assert np.array_equal(O.dequant_matmul_f16_f32(ai, wi.view(np.uint16), b, m, n, k),
                          (ai.astype(np.int64) @ wi.astype(np.int64).T).astype(np.float32))


def _q4_0(n, k):
    packed = RNG.integers(0, 256, (n, k // 2)).astype(np.uint8)
    scales = RNG.uniform(0.001, 0.05, (n, k // 32)).astype(np.float32)
    lo = (packed & 15).astype(np.int64) - 8
    hi = (packed >> 4).astype(np.int64) - 8
    vals = np.empty((n, k), np.int64)
    vals[:, 0::2], vals[:, 1::2] = lo, hi  # low nibble = even k
    return packed, scales, vals


@pytest.mark.parametrize("m,n,k", [(1, 6, 64), (3, 4, 256)])
def test_int4_matmuls_against_f64(m, n, k):
    packed, scales, vals = _q4_0(n, k)
    deq = vals.astype(np.float64) * np.repeat(scales.astype(np.float64), 32, axis=1)
    a = RNG.standard_normal((m, k)).astype(np.float32)
    want = a.astype(np.float64) @ deq.T
    assert _rel(O.int4_matmul_f32(a, packed, scales, m, n, k), want) < 1e-5
    assert _rel(O.int4_matmul_gemv(a[0], packed, scales, n, k), want[0]) < 1e-5
    # planted mistake: nibble order swapped must not agree
    swapped = ((packed & 15) << 4 | (packed >> 4)).astype(np.uint8)
    assert _rel(O.int4_matmul_f32(a, swapped, scales, m, n, k), want) > 1e-3
    # dequantised rows: the same decode
    for r in range(n):
        assert np.array_equal(O.q4_0_dequant_row(packed, scales, r, k),
                              (vals[r].astype(np.float32) * np.repeat(scales[r], 32)))


def test_int4_q4_x_q8_gemv():
    n, k = 7, 256
    packed, scales, vals = _q4_0(n, k)
    a = (RNG.standard_normal(k) * 3).astype(np.float32)
    a[32:64] = 0.0  # a zero group: scale 1, quants 0
    out, q, s = O.int4_matmul_gemv_q4_x_q8(a, packed, scales, n, k)
    qo, so = O.quantize_q8_groups(a, k)
    assert np.array_equal(q, qo) and np.array_equal(s, so)
    assert s[1] == np.float32(1.0) and not q[32:64].any()
    g = a.reshape(-1, 32)
    assert np.allclose(s, np.where(np.max(np.abs(g), 1) > 0, np.max(np.abs(g), 1) / 127.0, 1.0), rtol=1e-7)
    assert np.all(np.abs(q.astype(np.float64) * np.repeat(s, 32) - a) <= np.repeat(s, 32) * 0.5 * (1 + 1e-5))
    dots = (vals.reshape(n, -1, 32) * q.astype(np.int64).reshape(1, -1, 32)).sum(-1)  # exact group dots
    want = (dots.astype(np.float64) * scales.astype(np.float64) * s.astype(np.float64)).sum(1)
    assert _rel(out, want) < 1e-6


def test_quantize_int4_q4_0_known_answers_and_round_trip():
    grp = np.zeros(32, np.float32)
    grp[:8] = [7.0, -7.0, 3.5, -3.5, 0.5, -0.5, 2.49, 6.51]
    packed, scales = O.quantize_int4_q4_0(grp, 1, 32)
    assert scales[0, 0] == np.float32(1.0)
    lo, hi = (packed[0] & 15).astype(int), (packed[0] >> 4).astype(int)
    q = np.empty(32, int)
    q[0::2], q[1::2] = lo, hi
    assert q[:8].tolist() == [15, 1, 12, 4, 9, 7, 10, 15]  # round(x) + 8, ties away, clamp at 7
    p0, s0 = O.quantize_int4_q4_0(np.zeros((1, 64), np.float32), 1, 64)
    assert s0.tolist() == [[1.0, 1.0]] and np.all(p0 == 0x88)
    w = (RNG.standard_normal((5, 128)) * RNG.uniform(0.01, 2, (5, 1))).astype(np.float32)
    packed, scales = O.quantize_int4_q4_0(w, 5, 128)
    for r in range(5):
        back = O.q4_0_dequant_row(packed, scales, r, 128)
        assert np.all(np.abs(back - w[r]) <= np.repeat(scales[r], 32) * 0.5 * (1 + 1e-5))


def test_q8_0_dequant_row():
    w = RNG.integers(-128, 128, (3, 96)).astype(np.int8)
    s = RNG.uniform(0.001, 0.05, (3, 3)).astype(np.float32)
    for r in range(3):
        assert np.array_equal(O.q8_0_dequant_row(w, s, r, 96), w[r].astype(np.float32) * np.repeat(s[r], 32))


def test_crate_q6k_dequantizer_and_its_subscale_indexing():
    W = S.make_weight(S.TYPE_Q6_K, 4, 512, seed=5)
    ggml = O.dequantize(O.Q6_K, W.blocks, 512).ravel()
    crate = O.dequantize_q6_k_crate(W.blocks, 4 * 512)
    # the crate uses sub-scale 8h + {0,2,4,6} for all 32 elements of a group;
    # GGML uses 8h + l/16 + {0,2,4,6}: they agree wherever the two halves of a
    # group share a sub-scale, so force that and compare exactly
    sc = W.sc.copy()  # [n, nb, 16] int8
    sc[..., 1::2] = sc[..., 0::2]
    W2 = S.pack_q6k(W.d, sc, W.q)
    assert np.array_equal(O.dequantize_q6_k_crate(W2, 4 * 512), O.dequantize(O.Q6_K, W2, 512).ravel())
    # with distinct sub-scales the elements 16..31 of each 32-group differ
    diff = (crate != ggml).reshape(-1, 8, 32)
    assert not diff[..., :16].any() and diff[..., 16:].any()
