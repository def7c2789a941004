"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

The reference holds no golden vectors for this path (its only model test
needs a downloaded GGUF, test/llama_candle_model_test.exs:2-4), and candle's
source is not in this image.  The oracle is therefore pinned by
* library routines (numpy IEEE f16 conversion),
* closed-form known answers built so that the plausible mistakes (ties-to-even
  instead of ties-away, last-max instead of first-max, missing clamp, wrong
  sign of d, unrounded vs f16-rounded Q8_0 d) each give a different byte,
* exact integer sums computed from the generator's element arrays, which never
  go through the oracle's unpacking code (a swapped nibble, scale/min mix-up
  or wrong sub-scale index changes them),
* f64 dequantise-then-dot truth,
* the reference's own Q6_K bit layout (shape_ops.rs:2848-2899), restated.
"""
import numpy as np
import pytest

import oracle as O
from arm_ai_amd import synth as S
from tests._metrics import rel_cond, rel_max


# ------------------------------------------------------------------ f16
def test_f16_to_f32_all_half_values():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    # dense coverage of the f16 range, halfway cases and subnormals
    f16_all = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    f16_all = f16_all[np.isfinite(f16_all)]
    nxt = np.nextafter(f16_all.astype(np.float16), np.float16(np.inf)).astype(np.float32)
    mids = ((f16_all.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    extra = np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, 2.0**-25, 2.0**-24, 3 * 2.0**-26], np.float32)
    x = np.concatenate([bits.view(np.float32), f16_all, mids, np.nextafter(mids, np.float32(0)), extra])
    got = O.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x03FF) != 0)


# --------------------------------------------------------------- Q8_K
def _q8k(x):
    blocks = O.quantize(np.asarray(x, np.float32)[None, :], O.Q8_K)
    d, qs, bs = O.q8k_fields(blocks)
    return d[0], qs[0], bs[0]


def test_q8k_known_answers_rounding_and_scale():
    x = np.zeros(256, np.float32)
    x[0] = -128.0  # max |x| -> max = -128 -> iscale = 1.0, d = 1.0
    x[1], x[2], x[3], x[4], x[5] = 2.5, -2.5, 0.5, 1.5, 127.4
    d, qs, bs = _q8k(x)
    assert d[0] == np.float32(1.0)
    # ties away from zero (Rust f32::round): 2.5 -> 3, -2.5 -> -3, 0.5 -> 1, 1.5 -> 2
    assert list(qs[0, :6]) == [-128, 3, -3, 1, 2, 127]
    assert bs[0, 0] == int(qs[0, :16].astype(np.int32).sum())


def test_q8k_first_max_wins_and_clamp():
    x = np.zeros(256, np.float32)
    x[5], x[9] = 3.0, -3.0  # equal |x|: the first (+3) is `max`
    x[17] = 1.0
    d, qs, bs = _q8k(x)
    iscale = np.float32(-128.0) / np.float32(3.0)
    assert d[0] == np.float32(1.0) / iscale and d[0] < 0
    assert qs[0, 5] == -128
    assert qs[0, 9] == 127  # round(+128) clamped by min(127)
    assert qs[0, 17] == int(np.round(np.float64(iscale * np.float32(1.0))))
    assert bs[0, 0] == -1 and bs[0, 1] == qs[0, 17]


def test_q8k_zero_block_and_nan():
    x = np.zeros(512, np.float32)
    x[256 + 3] = np.nan  # NaN never becomes the max; round(NaN).min(127) -> 127
    x[256 + 7] = -2.0
    d, qs, bs = _q8k(x)
    assert d[0] == 0 and not qs[0].any() and not bs[0].any()
    assert d[1] == np.float32(1.0) / (np.float32(-128.0) / np.float32(-2.0))
    assert qs[1, 3] == 127 and qs[1, 7] == -128


def test_q8k_invariants_random():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 4096), dtype=np.float32) * rng.uniform(0.01, 100, size=(4, 1)).astype(np.float32)
    blocks = O.quantize(x, O.Q8_K)
    d, qs, bs = O.q8k_fields(blocks)
    xb = x.reshape(4, 16, 256)
    assert np.array_equal(bs, qs.reshape(4, 16, 16, 16).astype(np.int32).sum(-1).astype(np.int16))
    first = np.abs(xb).argmax(-1)  # numpy argmax returns the first maximum
    assert np.all(np.take_along_axis(qs, first[..., None], -1) == -128)
    mx = np.take_along_axis(xb, first[..., None], -1)[..., 0]
    assert np.allclose(d, -mx / 128.0, rtol=1e-6)
    err = np.abs(d[..., None].astype(np.float64) * qs - xb)
    clamped = qs == 127
    assert np.all(err[~clamped] <= np.abs(d[..., None].repeat(256, -1))[~clamped] * 0.5 * (1 + 1e-5))
    assert np.all(err[clamped] <= np.abs(d[..., None].repeat(256, -1))[clamped] * 1.5)


# --------------------------------------------------------------- Q8_0
def test_q8_0_known_answers():
    x = np.zeros(64, np.float32)
    x[:4] = [127.0, 63.5, -63.5, 0.5]
    x[32] = 1.0
    x[33] = 0.5
    blocks = O.quantize(x[None], O.Q8_0)
    d, qs = O.q8_0_fields(blocks)
    assert d[0, 0] == np.float16(1.0)
    assert list(qs[0, 0, :4]) == [127, 64, -64, 1]
    # d = 1/127 is stored f16-rounded; q uses the unrounded f32 id = 1/d
    d1 = np.float32(1.0) / np.float32(127.0)
    assert d[0, 1].view(np.uint16) == np.float32(d1).astype(np.float16).view(np.uint16)
    id1 = np.float32(1.0) / d1
    assert qs[0, 1, 0] == 127 and qs[0, 1, 1] == int(np.trunc(np.float64(np.float32(0.5) * id1) + 0.5))


# -------------------------------------------------- weights: layouts and sums
def _int_sums(W, xq, wtype):
    """S, Smin [m, n, nb] from the generator's element arrays (no unpacking)."""
    m = xq.shape[0]
    if wtype in (O.Q8_0, O.Q4_0, O.Q5_0):
        _, qx = O.q8_0_fields(xq)  # [m, nb, 32]
        qw = W.q.astype(np.int64) - {O.Q4_0: 8, O.Q5_0: 16}.get(wtype, 0)
        Sx = np.einsum("nbe,mbe->mnb", qw, qx.astype(np.int64))
        return Sx, np.zeros_like(Sx)
    _, qx, bs = O.q8k_fields(xq)  # [m, nb, 256], [m, nb, 16]
    if wtype == O.Q2_K:
        isum = np.einsum("nbje,mbje->mnbj", W.q.reshape(W.n, -1, 16, 16).astype(np.int64),
                         qx.reshape(m, -1, 16, 16).astype(np.int64))
        Sx = (isum * W.sc.astype(np.int64)[None]).sum(-1)
        Sm = np.einsum("mbg,nbg->mnb", bs.astype(np.int64), W.mn.astype(np.int64))
        return Sx, Sm
    if wtype in (O.Q4_K, O.Q5_K):
        isum = np.einsum("nbje,mbje->mnbj", W.q.reshape(W.n, -1, 8, 32).astype(np.int64),
                         qx.reshape(m, -1, 8, 32).astype(np.int64))
        Sx = (isum * W.sc.astype(np.int64)[None]).sum(-1)
        Sm = np.einsum("mbg,nbg->mnb", bs.astype(np.int64), np.repeat(W.mn.astype(np.int64), 2, axis=-1))
        return Sx, Sm
    isum = np.einsum("nbje,mbje->mnbj", W.q.reshape(W.n, -1, 16, 16).astype(np.int64),
                     qx.reshape(m, -1, 16, 16).astype(np.int64))
    Sx = (isum * W.sc.astype(np.int64)[None]).sum(-1)
    return Sx, np.zeros_like(Sx)


WTYPES = [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0, O.Q4_0, O.Q2_K, O.Q3_K, O.Q5_0]


@pytest.mark.parametrize("wtype", WTYPES)
@pytest.mark.parametrize("k", [256, 2048, 5632])
def test_block_sums_exact(wtype, k):
    W = S.make_weight(wtype, 24, k, seed=k + wtype)
    x = S.make_activation(3, k, seed=7)
    xq = O.quantize(x, O.act_type(wtype))
    got_S, got_Sm = O.block_sums(wtype, k, W.blocks, xq)
    want_S, want_Sm = _int_sums(W, xq, wtype)
    assert np.array_equal(got_S, want_S)
    assert np.array_equal(got_Sm, want_Sm)


@pytest.mark.parametrize("wtype", WTYPES)
def test_dequantize_matches_element_arrays(wtype):
    W = S.make_weight(wtype, 16, 1024, seed=11)
    got = O.dequantize(wtype, W.blocks, 1024).astype(np.float64)
    want = W.dequantize()
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("wtype", WTYPES)
def test_matmul_vs_f64_truth(wtype):
    k = 2048
    W = S.make_weight(wtype, 96, k, seed=5)
    x = S.make_activation(2, k, seed=6)
    xq = O.quantize(x, O.act_type(wtype))
    if wtype in (O.Q8_0, O.Q4_0, O.Q5_0):
        dx, qx = O.q8_0_fields(xq)
    else:
        dx, qx, _ = O.q8k_fields(xq)
    xdeq = (dx.astype(np.float64)[..., None] * qx).reshape(2, k)
    truth = xdeq @ W.dequantize().T
    got = O.matmul(wtype, x, W.blocks, 96, k)
    assert rel_max(got, truth) < 1e-6
    assert rel_cond(got, truth, W, np.abs(xdeq)) < 1e-6


def test_q4k_scale_unpack_two_formulations():
    """GGML get_scale_min_k4 (restated here) must invert the generator's pack for all 64x64 values."""
    sc = np.repeat(np.arange(64, dtype=np.uint8), 64).reshape(-1, 1, 1).repeat(8, axis=2)
    mn = np.tile(np.arange(64, dtype=np.uint8), 64).reshape(-1, 1, 1).repeat(8, axis=2)
    n = sc.shape[0]
    one = np.ones((n, 1), np.float16)
    blocks = S.pack_q4k(one, one, sc, mn, np.zeros((n, 1, 256), np.uint8)).reshape(n, 144)
    q = blocks[:, 4:16].astype(np.int32)
    for j in range(8):
        if j < 4:
            s, m = q[:, j] & 63, q[:, j + 4] & 63
        else:
            s = (q[:, j + 4] & 0xF) | ((q[:, j - 4] >> 6) << 4)
            m = (q[:, j + 4] >> 4) | ((q[:, j] >> 6) << 4)
        assert np.array_equal(s, sc[:, 0, j]) and np.array_equal(m, mn[:, 0, j])


def _ref_dequantize_q6_k(block_bytes: np.ndarray) -> np.ndarray:
    """Restatement of the reference's shape_ops.rs:2848-2899 (dequantize_q6_k),
    including its sub-scale indexing (scales[8n + {0,2,4,6}] for all l)."""
    out = np.zeros(256, np.float64)
    ql, qh, scales = block_bytes[0:128], block_bytes[128:192], block_bytes[192:208].view(np.int8)
    d = float(block_bytes[208:210].view(np.float16)[0])
    for n in range(2):
        for l in range(32):
            qhi = int(qh[32 * n + l])
            a, b = int(ql[64 * n + l]), int(ql[64 * n + l + 32])
            q1 = ((a & 0xF) | (((qhi >> 0) & 3) << 4)) - 32
            q2 = ((b & 0xF) | (((qhi >> 2) & 3) << 4)) - 32
            q3 = (((a >> 4) & 0xF) | (((qhi >> 4) & 3) << 4)) - 32
            q4 = (((b >> 4) & 0xF) | (((qhi >> 6) & 3) << 4)) - 32
            s = [int(scales[8 * n + i]) for i in (0, 2, 4, 6)]
            out[128 * n + l + 0] = d * s[0] * q1
            out[128 * n + l + 32] = d * s[1] * q2
            out[128 * n + l + 64] = d * s[2] * q3
            out[128 * n + l + 96] = d * s[3] * q4
    return out


def test_q6k_layout_vs_reference_dequantizer():
    rng = np.random.default_rng(21)
    W = S.make_weight(O.Q6_K, 4, 512, seed=21)
    # make odd sub-scales equal to the even ones, where the reference's
    # indexing and GGML's agree, then repack
    sc = W.sc.copy()
    sc[..., 1::2] = sc[..., 0::2]
    blocks = S.pack_q6k(W.d, sc, W.q).reshape(4, 2, 210)
    ours = O.dequantize(O.Q6_K, blocks.reshape(4, -1), 512).reshape(4, 2, 256)
    for r in range(4):
        for b in range(2):
            ref = _ref_dequantize_q6_k(blocks[r, b])
            assert np.allclose(ours[r, b], ref, rtol=1e-6, atol=0), (r, b)
    del rng


def test_special_case_reduces_to_int8_dot():
    """sc=1, m=0, d=1, dmin=0 turns Q4_K . Q8_K into d_x * sum q*qx."""
    rng = np.random.default_rng(1)
    n, k = 8, 512
    nb = k // 256
    q = rng.integers(0, 16, (n, nb, 256), dtype=np.uint8)
    blocks = S.pack_q4k(np.ones((n, nb), np.float16), np.zeros((n, nb), np.float16),
                        np.ones((n, nb, 8), np.uint8), np.zeros((n, nb, 8), np.uint8), q)
    x = S.make_activation(1, k, seed=2)
    xq = O.quantize(x, O.Q8_K)
    dx, qx, _ = O.q8k_fields(xq)
    want = (q.astype(np.int64) * qx[0].astype(np.int64)[None]).sum(-1)  # [n, nb]
    want_f = (want * dx[0].astype(np.float64)[None]).sum(-1)
    got = O.matmul_preq(O.Q4_K, xq, blocks, n, k)[0]
    assert np.allclose(got, want_f, rtol=1e-6)


def test_matmul_thread_count_independent_and_rowwise():
    W = S.make_weight(O.Q4_K, 700, 1024, seed=9)
    x = S.make_activation(3, 1024, seed=10)
    a = O.matmul(O.Q4_K, x, W.blocks, 700, 1024, nthreads=1)
    b = O.matmul(O.Q4_K, x, W.blocks, 700, 1024, nthreads=4)
    assert np.array_equal(a, b)
    for r in range(3):
        assert np.array_equal(O.matmul(O.Q4_K, x[r], W.blocks, 700, 1024, nthreads=2)[0], a[r])


def test_matmul_rejects_bad_shapes():
    with pytest.raises(ValueError):
        O.matmul(O.Q4_K, np.zeros((1, 300), np.float32), np.zeros((1, 144), np.uint8), 1, 300)
    with pytest.raises(ValueError):
        O.matmul(99, np.zeros((1, 256), np.float32), np.zeros((1, 144), np.uint8), 1, 256)


def test_planted_mistakes_are_caught():
    """Each check above fails for a plausible oracle mistake, planted here on the CPU."""
    k = 512
    W = S.make_weight(O.Q4_K, 8, k, seed=4)
    x = S.make_activation(1, k, seed=5)
    xq = O.quantize(x, O.Q8_K)
    want_S, want_Sm = _int_sums(W, xq, O.Q4_K)
    # (1) low/high nibble swapped in the unpack
    swapped = W.blocks.reshape(8, 2, 144).copy()
    qs = swapped[..., 16:]
    swapped[..., 16:] = ((qs & 0x0F) << 4) | (qs >> 4)
    S1, _ = O.block_sums(O.Q4_K, k, swapped.reshape(8, -1), xq)
    assert not np.array_equal(S1, want_S)
    # (2) scales and mins exchanged
    sw = S.pack_q4k(W.d, W.dmin, W.mn, W.sc, W.q)
    S2, Sm2 = O.block_sums(O.Q4_K, k, sw, xq)
    assert not np.array_equal(S2, want_S) and not np.array_equal(Sm2, want_Sm)
    # (3) ties-to-even instead of ties-away in Q8_K
    xx = np.zeros(256, np.float32)
    xx[0], xx[1] = -128.0, 2.5
    assert _q8k(xx)[1][0, 1] != int(np.rint(2.5))


def _q5k_block(qh=None, qs=None, sc=1, d=1.0):
    """One Q5_K block built byte by byte (not by the generator's packer):
    d, dmin = 0, every 6-bit scale = sc and min = 0 (the Q4_K packing of a
    constant scale below 16: bytes 0-3 = sc, 4-7 = 0, 8-11 = sc)."""
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[4:8] = sc
    b[12:16] = sc
    if qh is not None:
        b[16:48] = qh
    if qs is not None:
        b[48:176] = qs
    return b


@pytest.mark.parametrize("s,l", [(0, 0), (1, 5), (2, 31), (5, 17), (7, 9)])
def test_q5k_fifth_bit_lands_on_element_32s_plus_l(s, l):
    """GGML dequantize_row_q5_K: chunk c uses qh bit 2c for its low nibbles
    (elements 64c + l) and bit 2c+1 for its high nibbles (64c + 32 + l), i.e.
    bit s of qh[l] is bit 4 of element 32s + l."""
    qh = np.zeros(32, np.uint8)
    qh[l] = 1 << s
    got = O.dequantize(O.Q5_K, _q5k_block(qh=qh)[None], 256)[0]
    want = np.zeros(256)
    want[32 * s + l] = 16.0
    assert np.array_equal(got, want)


@pytest.mark.parametrize("c,l,hi", [(0, 3, False), (0, 3, True), (3, 30, True), (2, 0, False)])
def test_q5k_nibbles_land_like_q4k(c, l, hi):
    qs = np.zeros(128, np.uint8)
    qs[32 * c + l] = 0x50 if hi else 0x05
    got = O.dequantize(O.Q5_K, _q5k_block(qs=qs)[None], 256)[0]
    want = np.zeros(256)
    want[64 * c + 32 * hi + l] = 5.0
    assert np.array_equal(got, want)


def test_q5k_dot_is_plain_int8_dot_for_unit_scales():
    """sc = 1, m = 0, d = 1: Q5_K . Q8_K reduces to d_x * sum q5 * qx."""
    rng = np.random.default_rng(21)
    q = rng.integers(0, 32, 256)
    qs = ((q[np.r_[0:32, 64:96, 128:160, 192:224]] & 15) |
          ((q[np.r_[32:64, 96:128, 160:192, 224:256]] & 15) << 4)).astype(np.uint8)
    qh = np.zeros(32, np.uint8)
    for s in range(8):
        qh |= (((q[32 * s:32 * s + 32] >> 4) & 1) << s).astype(np.uint8)
    w = _q5k_block(qh=qh, qs=qs)[None]
    x = rng.standard_normal((1, 256)).astype(np.float32)
    xq = O.quantize(x, O.Q8_K)
    dx, qx, _ = O.q8k_fields(xq)
    got = O.matmul_preq(O.Q5_K, xq, w, 1, 256)[0, 0]
    # candle's order: eight i32 lanes (element e goes to lane e % 8), each
    # scaled by d = f16(d_w) * d_x in f32, then summed in lane order
    lanes = (q * qx[0, 0].astype(np.int64)).reshape(32, 8).sum(0)
    d = np.float32(1.0) * np.float32(dx[0, 0])
    t = np.float32(0.0)
    for l in range(8):
        t = np.float32(t + np.float32(d * np.float32(lanes[l])))
    assert int(lanes.sum()) == int((q * qx[0, 0].astype(np.int64)).sum())
    assert got == np.float32(np.float32(-0.0) + t)


@pytest.mark.parametrize("j,hi", [(0, False), (0, True), (7, True), (15, False), (15, True)])
def test_q4_0_nibble_lands_on_element_j_or_j_plus_16(j, hi):
    """GGML dequantize_row_q4_0: qs[j] & 15 is element j, qs[j] >> 4 element
    j + 16, value d * (q - 8); the block is built byte by byte."""
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([2.0], np.float16).view(np.uint8)
    b[2:18] = 0x88  # every quant 8 -> value 0
    b[2 + j] = 0x8D if not hi else 0xD8  # q = 13 -> value 2 * 5 = 10
    got = O.dequantize(O.Q4_0, b[None], 32)[0]
    want = np.zeros(32)
    want[j + 16 * hi] = 10.0
    assert np.array_equal(got, want)


# ------------------------------------------ Q2_K / Q3_K: hand-built blocks
def _q2k_block(scales=0x01, qs=None, d=1.0, dmin=0.0):
    """One Q2_K block built byte by byte: scales[16] @0 (low nibble scale,
    high nibble min), qs[64] @16, f16 d @80, f16 dmin @82."""
    b = np.zeros(84, np.uint8)
    b[0:16] = scales
    if qs is not None:
        b[16:80] = qs
    b[80:82] = np.array([d], np.float16).view(np.uint8)
    b[82:84] = np.array([dmin], np.float16).view(np.uint8)
    return b


@pytest.mark.parametrize("hf,j,l", [(0, 0, 0), (0, 3, 31), (1, 1, 7), (1, 2, 16), (0, 2, 15)])
def test_q2k_quant_lands_on_element_128hf_32j_l(hf, j, l):
    """GGML dequantize_row_q2_K: bits 2j..2j+1 of qs[32hf + l] are element
    128hf + 32j + l."""
    qs = np.zeros(64, np.uint8)
    qs[32 * hf + l] = 3 << (2 * j)
    got = O.dequantize(O.Q2_K, _q2k_block(qs=qs)[None], 256)[0]
    want = np.zeros(256)
    want[128 * hf + 32 * j + l] = 3.0
    assert np.array_equal(got, want)


@pytest.mark.parametrize("g", [0, 5, 8, 15])
def test_q2k_scale_and_min_of_group_g(g):
    """scales[g] holds the scale (low nibble) and min (high nibble) of
    elements 16g .. 16g + 15: value d * sc * q - dmin * mn."""
    sc = np.zeros(16, np.uint8)
    sc[g] = 0x75  # scale 5, min 7
    qs = np.full(64, 0x55, np.uint8)  # every quant 1
    got = O.dequantize(O.Q2_K, _q2k_block(scales=sc, qs=qs, d=2.0, dmin=0.5)[None], 256)[0]
    want = np.zeros(256)
    want[16 * g:16 * g + 16] = 2.0 * 5 * 1 - 0.5 * 7
    assert np.array_equal(got, want)


def test_q2k_dot_closed_form():
    """Every quant 3, scale 15, min 15, d = 1, dmin = 1, activation all ones
    (quants -128 after Q8_K: the first max maps to -128): per block
    S = 16 * 15 * (3 * -128 * 16), Smin = 16 * 15 * (-128 * 16)."""
    w = _q2k_block(scales=0xFF, qs=np.full(64, 0xFF, np.uint8), d=1.0, dmin=1.0)[None]
    x = np.ones((1, 256), np.float32)
    xq = O.quantize(x, O.Q8_K)
    S_, Sm = O.block_sums(O.Q2_K, 256, w, xq)
    assert S_[0, 0, 0] == 16 * 15 * 3 * -128 * 16
    assert Sm[0, 0, 0] == 16 * 15 * -128 * 16
    dx = O.q8k_fields(xq)[0][0, 0]
    got = O.matmul_preq(O.Q2_K, xq, w, 1, 256)[0, 0]
    assert got == np.float32(np.float32(dx * np.float32(S_[0, 0, 0])) - np.float32(dx * np.float32(Sm[0, 0, 0])))


def _q3k_block(hmask=0xFF, qs=None, scale_bytes=None, d=1.0):
    """One Q3_K block built byte by byte: hmask[32] @0, qs[64] @32,
    scales[12] @96, f16 d @108.  Default scale bytes give every group the
    6-bit scale 32 (value 0): low nibbles 0, two-bit fields 0b10."""
    b = np.zeros(110, np.uint8)
    b[0:32] = hmask
    if qs is not None:
        b[32:96] = qs
    b[96:108] = scale_bytes if scale_bytes is not None else np.r_[np.zeros(8, np.uint8), np.full(4, 0xAA, np.uint8)]
    b[108:110] = np.array([d], np.float16).view(np.uint8)
    return b


@pytest.mark.parametrize("g,nib_byte,nib_hi,bits_byte,bits_shift", [
    (0, 0, False, 8, 0), (3, 3, False, 11, 0), (5, 5, False, 9, 2), (9, 1, True, 9, 4), (14, 6, True, 10, 6)])
def test_q3k_scale_of_group_g(g, nib_byte, nib_hi, bits_byte, bits_shift):
    """candle's auxs form: scales 0-3 = low nibbles of bytes 0-3 + bits 0-1
    of bytes 8-11; 4-7 = low nibbles of bytes 4-7 + bits 2-3; 8-11 = high
    nibbles of bytes 0-3 + bits 4-5; 12-15 = high nibbles of bytes 4-7 +
    bits 6-7; value scale - 32.  Group g gets 63 (value 31), every other 32."""
    sb = np.r_[np.zeros(8, np.uint8), np.full(4, 0xAA, np.uint8)]
    sb[nib_byte] |= 0xF0 if nib_hi else 0x0F
    sb[bits_byte] |= 3 << bits_shift
    qs = np.full(64, 0x55, np.uint8)  # every 2-bit field 1, hmask set: value 1
    got = O.dequantize(O.Q3_K, _q3k_block(qs=qs, scale_bytes=sb)[None], 256)[0]
    want = np.zeros(256)
    want[16 * g:16 * g + 16] = 31.0
    assert np.array_equal(got, want)


@pytest.mark.parametrize("hf,j,l", [(0, 0, 0), (0, 3, 20), (1, 0, 31), (1, 3, 9)])
def test_q3k_hmask_bit_lands_on_element(hf, j, l):
    """GGML dequantize_row_q3_K: bit 4hf + j of hmask[l] clear subtracts 4
    from element 128hf + 32j + l; bits 2j..2j+1 of qs[32hf + l] are its low
    two bits.  All scales 33 (value 1)."""
    sb = np.r_[np.full(8, 0x11, np.uint8), np.full(4, 0xAA, np.uint8)]  # 0b10_0001 = 33
    hm = np.full(32, 0xFF, np.uint8)
    hm[l] &= ~np.uint8(1 << (4 * hf + j))
    qs = np.zeros(64, np.uint8)
    qs[32 * hf + l] = 2 << (2 * j)
    got = O.dequantize(O.Q3_K, _q3k_block(hmask=hm, qs=qs, scale_bytes=sb)[None], 256)[0]
    want = np.zeros(256)
    want[128 * hf + 32 * j + l] = 2.0 - 4.0
    assert np.array_equal(got, want)


@pytest.mark.parametrize("e", [0, 5, 15, 16, 22, 31])
def test_q5_0_fifth_bit_and_nibble_land_on_element(e):
    """GGML dequantize_row_q5_0: bit e of the u32 qh is bit 4 of element e;
    qs[j] & 15 is element j, qs[j] >> 4 element j + 16; value d * (q - 16).
    The block is built byte by byte: every quant 16 (value 0) except e."""
    b = np.zeros(22, np.uint8)
    b[0:2] = np.array([0.5], np.float16).view(np.uint8)
    qh = np.uint32(0xFFFFFFFF) & ~np.uint32(1 << e)  # every fifth bit set (16) except e's
    b[2:6] = np.array([qh], "<u4").view(np.uint8)
    b[6:22] = 0
    j, hi = e % 16, e >= 16
    b[6 + j] = 0x70 if hi else 0x07  # e: q = 7 (fifth bit clear) -> value -9
    got = O.dequantize(O.Q5_0, b[None], 32)[0]
    want = np.zeros(32)
    want[e] = 0.5 * (7 - 16)
    assert np.array_equal(got, want)


def test_v3_build_is_bit_identical_to_the_baseline_build():
    """liboracle_v3.so (x86-64-v3, the upper-bound CPU line bench.py reports)
    compiles the same source with FMA contraction off: every output equals
    the baseline build's bit for bit."""
    import pytest

    if not O.cpu_has_v3():
        pytest.skip("this CPU cannot run x86-64-v3 code")
    rng = np.random.default_rng(3)
    for wtype, n, k in ((O.Q4_K, 96, 2048), (O.Q6_K, 64, 1024), (O.Q8_0, 40, 512), (O.Q5_K, 33, 768)):
        W = S.make_weight(wtype, n, k, seed=wtype)
        x = rng.standard_normal((5, k)).astype(np.float32)
        a = O.matmul(wtype, x, W.blocks, n, k, isa="baseline")
        b = O.matmul(wtype, x, W.blocks, n, k, isa="v3")
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), wtype
