"""GPU parity of the batch-1 Q4_K / Q6_K matvec with one weight row per lane
(csrc/k_rowlane.hip), the path a single activation row takes on a weight of
at least 11200 rows and k <= 8192 (Llama-3-8B ffn_up / ffn_gate, the
lm_heads, with persistent chunks beyond 256 of them), of its 16-row form
(lane = row + 16 * group phase), taken from 256 rows up to k = 16384
(Llama-3-8B ffn_down 4096 x 14336, the attention projections), and of its
8-row form (lane = row + 8 * group phase), taken from 1025 to 2048 rows up
to k = 8192 (TinyLlama's wo and w2; its wk, wv and wq|wk take the 16-row
form).  Q5_K, Q4_0, Q5_0, Q2_K and Q3_K weights take the same forms as
Q4_K; Q8_0
weights (up to k = 8192) the 16- and 8-row forms; for Q8_0, Q4_0 and Q5_0
the activation is quantised to Q8_0 blocks in the prologue (k a multiple of
256 for all).  The fused transforms (RMSNorm,
SiLU * up) and the two-weight launch are tested with the decode glue.

Against the oracle (candle-core 0.8.4 k_quants::matmul restated): every
integer block sum S and Smin bit-exact, outputs within max relative error
1e-5; the in-kernel Q8_K quantisation (16 lanes per block) must give the
same bytes as the quantizer kernel, which the edge rows check through the
integer sums (a quant that differs changes S or Smin).
"""
import numpy as np
import pytest

import arm_ai_amd as A
import oracle as O
from arm_ai_amd import synth as S
from tests.test_gpu_parity import _edge_rows, _xdeq_abs, check_matmul

pytestmark = pytest.mark.gpu

RL_MIN_N = 11200  # rows from which a one-row Q4_K matvec takes the row-per-lane kernel
RG_MIN_N = 256    # rows from which it takes the 16-row form (any k <= 16384)
RE_MIN_N, RE_MAX_N = 1025, 2048  # rows for which it takes the 8-row form instead (k <= 8192)


@pytest.mark.parametrize("n,k", [
    (14336, 4096),   # the headline shape: 256 workgroups of 56 rows, one group per wavefront
    (RL_MIN_N, 256),  # one group: a single quantising wavefront
    (11203, 2048),   # ragged: the last workgroup's rows and its last row block are partial
    (11264, 5632),   # 22 groups: three groups per wavefront, some wavefronts short
    (12000, 8192),   # 32 groups: four per wavefront, every wavefront quantises
])
def test_rowlane_matches_oracle(ctx, n, k):
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=n + k)
    x = S.make_activation(1, k, seed=k)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("n,k", [
    (4096, 14336),   # Llama-3-8B ffn_down: 256 workgroups, 56 groups over 14 wavefronts of four phases
    (4096, 4096),    # the attention projections: 16 groups, four wavefronts
    (RG_MIN_N, 8192),  # 32 groups, eight wavefronts (the fewest rows of this form)
    (RE_MAX_N + 8, 2048),  # the first rows past the 8-row form
    (3203, 16384),   # 64 groups (the most), ragged rows: the last workgroup's second row block is partial
    (5000, 8448),    # 33 groups: the ninth wavefront's lanes straddle the last group
    (RL_MIN_N, 9216),  # many rows but 36 groups: the 16-row form
])
def test_rowlane16_matches_oracle(ctx, n, k):
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=n + k + 1)
    x = S.make_activation(1, k, seed=k + 1)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("n,k", [
    (RE_MAX_N, 2048),  # TinyLlama wo: 256 workgroups of 8 rows, 8 groups over two wavefronts
    (2048, 5632),      # TinyLlama w2: 22 groups over six wavefronts (three walk, all quantise)
    (RE_MIN_N, 256),   # one group, ragged rows: the last workgroup has one
    (2043, 2304),      # ragged rows (the last workgroup has three), 9 groups: four wavefronts
    (1500, 4352),      # 17 groups: six wavefronts, ragged rows
    (1999, 6400),      # 25 groups: eight wavefronts, ragged rows
    (RE_MAX_N, 8192),  # 32 groups (the most for this form)
])
def test_rowlane8_matches_oracle(ctx, n, k):
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=n + k + 5)
    x = S.make_activation(1, k, seed=k + 5)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("n,k", [
    (32000, 2048),    # config 1's lm_head: 572 workgroups of 56 rows
    (RL_MIN_N, 256),  # one group
    (11203, 4096),    # ragged rows, 16 groups
    (12000, 8192),    # 32 groups: two per wavefront
    (4096, 14336),    # Llama-3-8B ffn_down in its Q6_K layers: the 16-row form, 56 groups
    (3203, 4096),     # 16-row form, ragged rows, four wavefronts
    (2048, 5632),     # TinyLlama w2 in its Q6_K layers: 8-row form, 22 groups over six wavefronts
    (1027, 4096),     # 8-row form, ragged rows (the last workgroup has three), 16 groups
    (256, 2048),      # TinyLlama wv: 16 workgroups of 16 rows, 8 groups
    (5000, 8448),     # 33 groups, a wavefront's lanes straddling the last group
])
def test_rowlane_q6k_matches_oracle(ctx, n, k):
    """Q6_K through the row-per-lane kernel (13 pieces per group, the scales
    and qh pieces held while the ql pieces stream, the d plane read per
    group), with llama.cpp's full int8 sub-scale range."""
    rng = np.random.default_rng(n + k + 3)
    W = S.make_weight(S.TYPE_Q6_K, n, k, seed=n + k + 2)
    W.sc[:] = rng.integers(-128, 128, size=W.sc.shape).astype(np.int8)
    W.blocks = S.pack_q6k(W.d, W.sc, W.q)
    x = S.make_activation(1, k, seed=k + 2)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("typ,n,k", [
    (S.TYPE_Q4_K, 32000, 4096),    # 572 chunks over 256 persistent workgroups: some walk three
    (S.TYPE_Q4_K, 60001, 1024),    # 1072 chunks, ragged rows, four groups (12 idle wavefronts)
    (S.TYPE_Q6_K, 128256, 4096),   # Llama-3-8B lm_head: 2291 chunks, about 4.5 per workgroup
    (S.TYPE_Q6_K, 70003, 768),     # three groups, ragged rows
])
def test_rowlane_persistent_chunks(ctx, typ, n, k):
    """More 56-row chunks than two per CU: workgroups quantise the activation
    once and walk several chunks, with the next chunk's pieces in flight."""
    rng = np.random.default_rng(n + k + 5)
    W = S.make_weight(typ, n, k, seed=n + k + 4)
    if typ == S.TYPE_Q6_K:
        W.sc[:] = rng.integers(-128, 128, size=W.sc.shape).astype(np.int8)
        W.blocks = S.pack_q6k(W.d, W.sc, W.q)
    x = S.make_activation(1, k, seed=k + 4)
    check_matmul(ctx, W, x)


def test_rowlane_q6k_extreme_values(ctx):
    """Every Q6_K quant at -32 and every sub-scale -128 against activation
    blocks of equal values: the largest sums, bit-exact."""
    n, k = RL_MIN_N, 4096
    rng = np.random.default_rng(8)
    W = S.make_weight(S.TYPE_Q6_K, n, k, seed=9)
    W.q[:] = -32
    W.sc[:] = -128
    W.blocks = S.pack_q6k(W.d, W.sc, W.q)
    x = np.repeat(np.abs(rng.standard_normal((1, k // 256))).astype(np.float32) + 0.5, 256, axis=1)
    check_matmul(ctx, W, x, cond=False)


@pytest.mark.parametrize("n,k", [
    (2048, 2048),     # config 1's Q8_0 matvec: 256 workgroups of 8 rows, 8 groups of eight blocks
    (256, 2048),      # 16 workgroups of 16 rows
    (1025, 256),      # one group, ragged rows: the last 8-row workgroup has one
    (2043, 2304),     # 9 groups over four wavefronts, ragged rows
    (3203, 4096),     # 16-row form, ragged rows: the last workgroup's second row block is partial
    (4096, 8192),     # 32 groups (the most for Q8_0), eight wavefronts
    (20000, 2048),    # many rows: Q8_0 keeps the 16-row form
])
def test_rowlane_q80_matches_oracle(ctx, n, k):
    """Q8_0 through the row-per-lane kernel: the activation quantised to Q8_0
    blocks in the prologue (two lanes per 32-element block), 17 pieces per
    group (the eight d first), every block's integer dot bit-exact."""
    W = S.make_weight(S.TYPE_Q8_0, n, k, seed=n + k + 9)
    x = S.make_activation(1, k, seed=k + 9)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("typ", [S.TYPE_Q4_0, S.TYPE_Q5_0, S.TYPE_Q5_K, S.TYPE_Q2_K, S.TYPE_Q3_K])
@pytest.mark.parametrize("n,k", [
    (14336, 4096),    # 56-row workgroups, one group per wavefront
    (11264, 5632),    # 56-row workgroups, two groups per wavefront (22 groups)
    (16001, 2048),    # more 56-row chunks than CUs: persistent workgroups, ragged rows
    (4096, 14336),    # the 16-row form with 16 wavefronts (56 groups)
    (3203, 4096),     # 16-row form, ragged rows
    (2043, 2304),     # 8-row form, ragged rows, 9 groups
])
def test_rowlane_legacy_and_q5k_match_oracle(ctx, typ, n, k):
    """Q4_0, Q5_0 (the activation in Q8_0 blocks; q - 8 and q - 16 taken as
    the block's quant sum times 8 or 16), Q5_K (the fifth bit from the qh
    pieces held in registers), Q2_K (d and dmin from the d plane) and Q3_K
    (the hmask pieces held; q - 4 and the scale - 32) through every
    row-per-lane form, integer sums bit-exact."""
    W = S.make_weight(typ, n, k, seed=n + k + typ)
    x = S.make_activation(1, k, seed=k + typ)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("typ,low", [(S.TYPE_Q4_0, False), (S.TYPE_Q5_0, False), (S.TYPE_Q5_K, False),
                                     (S.TYPE_Q2_K, False), (S.TYPE_Q3_K, False), (S.TYPE_Q3_K, True)])
def test_rowlane_legacy_and_q5k_extreme_values(ctx, typ, low):
    """Every quant at an end of its range (Q4_0 15, Q5_0 31 with every qh bit
    set, Q5_K 31 with scales and mins 63, Q2_K 3 with scales and mins 15,
    Q3_K 3 with scale 31 or -4 with scale -32) against activation blocks of
    equal values (every quant +-127 or -128), in the 56-row, 16-row and 8-row
    forms: the largest sums, bit-exact."""
    rng = np.random.default_rng(typ)
    for n, k in ((11200, 2048), (4096, 4096), (2048, 2048)):
        W = S.make_weight(typ, n, k, seed=typ + n)
        if typ == S.TYPE_Q4_0:
            W.q[:] = 15
            W.blocks = S.pack_q4_0(W.d, W.q)
        elif typ == S.TYPE_Q5_0:
            W.q[:] = 31
            W.blocks = S.pack_q5_0(W.d, W.q)
        elif typ == S.TYPE_Q5_K:
            W.q[:] = 31
            W.sc[:] = 63
            W.mn[:] = 63
            W.blocks = S.pack_q5k(W.d, W.dmin, W.sc, W.mn, W.q)
        elif typ == S.TYPE_Q2_K:
            W.q[:] = 3
            W.sc[:] = 15
            W.mn[:] = 15
            W.blocks = S.pack_q2k(W.d, W.dmin, W.sc, W.mn, W.q)
        else:
            W.q[:] = -4 if low else 3
            W.sc[:] = -32 if low else 31
            W.blocks = S.pack_q3k(W.d, W.sc, W.q)
        blk = 32 if typ in (S.TYPE_Q4_0, S.TYPE_Q5_0) else 256
        x = np.repeat(rng.standard_normal((1, k // blk)).astype(np.float32), blk, axis=1)
        check_matmul(ctx, W, x, cond=False)


@pytest.mark.parametrize("typ", [S.TYPE_Q8_0, S.TYPE_Q4_0, S.TYPE_Q5_0])
def test_rowlane_q80_edge_activations_and_entries(ctx, typ):
    """The edge rows of the Q8_0 quantizer (zeros, 1e-30, 1e30, equal values,
    ties) through the row-per-lane prologue (with the block quant sums Q4_0
    and Q5_0 take), block sums bit-exact; and the f32 device entry, the
    pre-quantised entry and the host entry giving the same bits."""
    from arm_ai_amd import hip

    n, k = 2048, 2048
    W = S.make_weight(typ, n, k, seed=91 + typ)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (n, k), W.blocks), ctx)
    for x in _edge_rows(k):
        x = x[None, :]
        xq = O.quantize(x, O.Q8_0)
        gS, gSm = mm.block_sums(x)
        oS, oSm = O.block_sums(W.type, k, W.blocks, xq)
        assert np.array_equal(gS, oS) and np.array_equal(gSm, oSm)
    x = S.make_activation(1, k, seed=92)
    y_host = mm.forward(x)
    dx = hip.to_device(x)
    dy = hip.DeviceBuffer(n * 4)
    mm.forward_device(dx.ptr, 1, dy.ptr)
    act = hip.DeviceBuffer(A.act_bytes(mm.act_type, 1, k))
    A.quantize_act_device(ctx, mm.act_type, dx.ptr, 1, k, act.ptr)
    dy2 = hip.DeviceBuffer(n * 4)
    mm.forward_preq_device(act.ptr, 1, dy2.ptr)
    ctx.synchronize()
    assert np.array_equal(dy.download(np.float32, (1, n)), y_host)
    assert np.array_equal(dy2.download(np.float32, (1, n)), y_host)
    mm.free()


def test_rowlane16_edge_activations(ctx):
    """The edge rows of the quantizer through the 16-row form's in-kernel
    quantisation, integer sums bit-exact."""
    k = 14336
    W = S.make_weight(S.TYPE_Q4_K, 4096, k, seed=78)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (W.n, W.k), W.blocks), ctx)
    for x in _edge_rows(k):
        x = x[None, :]
        xq = O.quantize(x, O.Q8_K)
        gS, gSm = mm.block_sums(x)
        oS, oSm = O.block_sums(W.type, k, W.blocks, xq)
        assert np.array_equal(gS, oS) and np.array_equal(gSm, oSm)
    mm.free()


def test_rowlane_edge_activations(ctx):
    """Zeros, 1e-30, 1e30, equal values (first max), exact ties (rounding away
    from zero), NaN and f32 subnormals through the in-kernel quantisation."""
    k = 4096
    W = S.make_weight(S.TYPE_Q4_K, RL_MIN_N, k, seed=77)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (W.n, W.k), W.blocks), ctx)
    for x in _edge_rows(k):
        x = x[None, :]
        xq = O.quantize(x, O.Q8_K)
        gS, gSm = mm.block_sums(x)
        oS, oSm = O.block_sums(W.type, k, W.blocks, xq)
        assert np.array_equal(gS, oS) and np.array_equal(gSm, oSm)
        y = mm.forward(x)
        r = O.matmul_preq(W.type, xq, W.blocks, W.n, k)
        ok = np.isfinite(r)
        assert np.array_equal(np.isfinite(y), ok)
        if ok.any():
            scale = max(float(np.abs(r[ok]).max()), 1e-30)
            assert float(np.abs(y[ok] - r[ok]).max()) / scale <= 1e-5
    mm.free()


def test_rowlane_extreme_values(ctx):
    """Every quant 15, every scale and min 63: the largest integer sums the
    kernel forms, bit-exact.  The f32 output is held to 1e-5 of the f64 value
    of those exact sums; against the oracle it is held to the conditioning-
    aware bar (rel_cond), because here candle's own summation order (the
    oracle's) is 3.4e-5 away from the exact value in rel_max terms."""
    from tests._metrics import rel_cond

    n, k = RL_MIN_N, 4096
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=5)
    W.q[:] = 15
    W.sc[:] = 63
    W.mn[:] = 63
    W.blocks = S.pack_q4k(W.d, W.dmin, W.sc, W.mn, W.q)
    # every block's first element (-1) is its max: quants -128 and, after the
    # clamp of +128, +127
    x = np.full((1, k), -1.0, np.float32)
    x[0, 1::2] = 1.0
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (n, k), W.blocks), ctx)
    xq = O.quantize(x, O.Q8_K)
    gS, gSm = mm.block_sums(x)
    oS, oSm = O.block_sums(W.type, k, W.blocks, xq)
    assert np.array_equal(gS, oS) and np.array_equal(gSm, oSm)
    y = mm.forward(x)[0].astype(np.float64)
    dx = O.q8k_fields(xq)[0].astype(np.float64)[0]
    exact = (W.d.astype(np.float64) * dx * oS[0] - W.dmin.astype(np.float64) * dx * oSm[0]).sum(axis=1)
    assert np.abs(y - exact).max() <= 1e-5 * np.abs(exact).max()
    r = O.matmul_preq(W.type, xq, W.blocks, n, k)
    _, xabs = _xdeq_abs(x, W.type)
    assert rel_cond(y[None, :], r, W, xabs) <= 1e-5
    mm.free()


def test_rowlane_device_and_prequantised_entries(ctx):
    """The f32 device entry, the pre-quantised entry and the host entry give
    the same bits at the headline shape."""
    from arm_ai_amd import hip

    n, k = 14336, 4096
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=21)
    x = S.make_activation(1, k, seed=22)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (n, k), W.blocks), ctx)
    y_host = mm.forward(x)
    dx = hip.to_device(x)
    dy = hip.DeviceBuffer(n * 4)
    mm.forward_device(dx.ptr, 1, dy.ptr)
    act = hip.DeviceBuffer(A.act_bytes(mm.act_type, 1, k))
    A.quantize_act_device(ctx, mm.act_type, dx.ptr, 1, k, act.ptr)
    dy2 = hip.DeviceBuffer(n * 4)
    mm.forward_preq_device(act.ptr, 1, dy2.ptr)
    ctx.synchronize()
    assert np.array_equal(dy.download(np.float32, (1, n)), y_host)
    assert np.array_equal(dy2.download(np.float32, (1, n)), y_host)
    mm.free()


def test_rowlane_and_general_matvec_agree(ctx):
    """The same rows through the row-per-lane kernel (n >= 11200) and through
    the general matvec (the first 11192 rows as a weight of their own): the
    integer sums are identical and the outputs agree to the tolerance."""
    k = 2048
    W = S.make_weight(S.TYPE_Q4_K, RL_MIN_N, k, seed=31)
    x = S.make_activation(1, k, seed=32)
    big = A.QMatMul.from_qtensor(A.QTensor(W.type, (W.n, k), W.blocks), ctx)
    n2 = RL_MIN_N - 8
    small = A.QMatMul.from_qtensor(A.QTensor(W.type, (n2, k), W.blocks[:n2]), ctx)
    sb, smb = big.block_sums(x)
    ss, sms = small.block_sums(x)
    assert np.array_equal(sb[:, :n2], ss) and np.array_equal(smb[:, :n2], sms)
    yb, ys = big.forward(x), small.forward(x)
    assert float(np.abs(yb[:, :n2] - ys).max()) <= 1e-5 * float(np.abs(ys).max())
    big.free()
    small.free()


@pytest.mark.parametrize("typ", [S.TYPE_Q5_K, S.TYPE_Q6_K, S.TYPE_Q8_0, S.TYPE_Q4_0, S.TYPE_Q5_0, S.TYPE_Q2_K,
                                 S.TYPE_Q3_K])
def test_rowlane_and_general_matvec_agree_every_type(ctx, typ):
    """At the row count where the row-per-lane kernel takes over (256 rows,
    16-row form) against the general matvec on the first 248 rows as a
    weight of their own: the integer sums are identical and the outputs agree
    to the tolerance, for every type the kernel takes."""
    k = 4096
    W = S.make_weight(typ, RG_MIN_N, k, seed=40 + typ)
    x = S.make_activation(1, k, seed=41 + typ)
    big = A.QMatMul.from_qtensor(A.QTensor(W.type, (W.n, k), W.blocks), ctx)
    n2 = RG_MIN_N - 8
    small = A.QMatMul.from_qtensor(A.QTensor(W.type, (n2, k), W.blocks[:n2]), ctx)
    sb, smb = big.block_sums(x)
    ss, sms = small.block_sums(x)
    assert np.array_equal(sb[:, :n2], ss) and np.array_equal(smb[:, :n2], sms)
    yb, ys = big.forward(x), small.forward(x)
    assert float(np.abs(yb[:, :n2] - ys).max()) <= 1e-5 * float(np.abs(ys).max())
    big.free()
    small.free()


def test_rowlane16_and_general_matvec_agree(ctx):
    """The 16-row form (n >= 256) against the general matvec on the first
    248 rows of the same weight: integer sums identical, outputs within the
    tolerance."""
    k = 14336
    W = S.make_weight(S.TYPE_Q4_K, RG_MIN_N, k, seed=33)
    x = S.make_activation(1, k, seed=34)
    big = A.QMatMul.from_qtensor(A.QTensor(W.type, (W.n, k), W.blocks), ctx)
    n2 = RG_MIN_N - 8
    small = A.QMatMul.from_qtensor(A.QTensor(W.type, (n2, k), W.blocks[:n2]), ctx)
    sb, smb = big.block_sums(x)
    ss, sms = small.block_sums(x)
    assert np.array_equal(sb[:, :n2], ss) and np.array_equal(smb[:, :n2], sms)
    yb, ys = big.forward(x), small.forward(x)
    assert float(np.abs(yb[:, :n2] - ys).max()) <= 1e-4 * float(np.abs(ys).max())
    big.free()
    small.free()


@pytest.mark.parametrize("typ", [S.TYPE_Q4_K, S.TYPE_Q6_K, S.TYPE_Q4_0, S.TYPE_Q5_0])
@pytest.mark.parametrize("n", [RL_MIN_N, 512])
def test_rowlane8w_edge_activations(ctx, typ, n):
    """The edge rows of the quantizer, plus ties of |x| across lanes (the
    first index wins) and within a Q8_0 block, through the forms whose
    prologue quantises one block per wavefront with four elements per lane
    (Q8_K: 64 lanes per block; Q8_0: eight per block) -- the 8-wavefront
    56-row form (RL_MIN_N rows: 200 workgroups) and the 16-row form with a
    grid of at most 128 workgroups (512 rows: 32) -- integer sums bit-exact,
    outputs within 1e-5."""
    k = 2048  # 8 groups: one per wavefront
    W = S.make_weight(typ, n, k, seed=80 + typ)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (W.n, W.k), W.blocks), ctx)
    extra = np.zeros((2, k), np.float32)
    extra[0, 256 + 7], extra[0, 256 + 8], extra[0, 256 + 200] = -3.0, 3.0, 3.0  # lanes 1, 2, 50 of block 1
    extra[1, 512 + 33], extra[1, 512 + 62] = 2.0, -2.0                        # one Q8_0 block, two lanes
    qtype = O.Q8_0 if typ in (S.TYPE_Q4_0, S.TYPE_Q5_0) else O.Q8_K
    for x in np.concatenate([_edge_rows(k), extra]):
        x = x[None, :]
        xq = O.quantize(x, qtype)
        gS, gSm = mm.block_sums(x)
        oS, oSm = O.block_sums(W.type, k, W.blocks, xq)
        assert np.array_equal(gS, oS) and np.array_equal(gSm, oSm)
        y = mm.forward(x)
        r = O.matmul_preq(W.type, xq, W.blocks, W.n, k)
        ok = np.isfinite(r)
        assert np.array_equal(np.isfinite(y), ok)
        if ok.any():
            scale = max(float(np.abs(r[ok]).max()), 1e-30)
            assert float(np.abs(y[ok] - r[ok]).max()) / scale <= 1e-5
    mm.free()
