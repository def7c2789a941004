"""GPU parity: the HIP kernels, called through the C ABI, against the oracle.

Bars (task statement): Q8_K / Q8_0 activation quantisation and every integer
block dot product bit-exact; f32 outputs within max relative error 1e-5
(1e-4 for K >= 14336), measured as rel_max and rel_cond (tests/_metrics.py).
"""
import numpy as np
import pytest

import arm_ai_amd as A
import oracle as O
from arm_ai_amd import synth as S
from tests._metrics import rel_cond, rel_max, tol_for_k

pytestmark = pytest.mark.gpu


def _xdeq_abs(x, wtype):
    xq = O.quantize(x, O.act_type(wtype))
    if wtype in (O.Q8_0, O.Q4_0, O.Q5_0):
        d, q = O.q8_0_fields(xq)
    else:
        d, q, _ = O.q8k_fields(xq)
    return xq, np.abs(d.astype(np.float32)[..., None] * q).reshape(x.shape[0], -1)


def check_matmul(ctx, W, x, *, sums=True, cond=True):
    wtype = W.type
    mm = A.QMatMul.from_qtensor(A.QTensor(wtype, (W.n, W.k), W.blocks), ctx)
    y = mm.forward(x)
    xq, xabs = _xdeq_abs(x, wtype)
    r = O.matmul_preq(wtype, xq, W.blocks, W.n, W.k)
    tol = tol_for_k(W.k)
    rm = rel_max(y, r)
    assert np.all(np.isfinite(y))
    assert rm <= tol, f"rel_max {rm:.3e} > {tol}"
    if cond:
        rc = rel_cond(y, r, W, xabs)
        assert rc <= tol, f"rel_cond {rc:.3e} > {tol}"
    if sums:
        gS, gSm = mm.block_sums(x)
        oS, oSm = O.block_sums(wtype, W.k, W.blocks, xq)
        assert np.array_equal(gS, oS), "integer block sums S differ"
        assert np.array_equal(gSm, oSm), "integer block sums Smin differ"
    mm.free()
    return y, r


# ------------------------------------------------------------ quantizers
def _edge_rows(k):
    rng = np.random.default_rng(17)
    rows = [
        np.zeros(k, np.float32),
        rng.standard_normal(k).astype(np.float32) * 1e-30,  # tiny values
        rng.standard_normal(k).astype(np.float32) * 1e30,
        np.full(k, -2.0, np.float32),  # all equal: first element is the max
    ]
    r = np.zeros(k, np.float32)
    r[0], r[1], r[2], r[3], r[4] = -128.0, 2.5, -2.5, 0.5, 1.5  # ties-away rounding
    r[300 % k], r[301 % k] = 3.0, -3.0
    rows.append(r)
    r = rng.standard_normal(k).astype(np.float32)
    r[5] = np.nan
    rows.append(r)
    r = np.zeros(k, np.float32)
    r[::37] = np.float32(1e-40)  # f32 subnormals
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("m,k", [(1, 2048), (8, 4096), (3, 14336), (512, 2048), (2, 256)])
def test_quantize_q8k_bitexact(ctx, m, k):
    x = S.make_activation(m, k, seed=m * 7 + k)
    x = np.concatenate([x, _edge_rows(k)])
    got = A.quantize_q8k(ctx, x)
    want = O.quantize(x, O.Q8_K)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("m,k", [(1, 2048), (5, 4096), (64, 1024), (1, 32)])
def test_quantize_q8_0_bitexact(ctx, m, k):
    x = S.make_activation(m, k, seed=m + k)
    x = np.concatenate([x, _edge_rows(k)])
    x[-3, :] *= np.float32(65504.0 * 127)  # f16 overflow of d -> inf
    got = A.quantize_q8_0(ctx, x)
    want = O.quantize(x, O.Q8_0)
    assert np.array_equal(got, want)


# --------------------------------------------------- benchmark configurations
def test_config0_q4k_tinyllama_ffn_up(ctx):
    W = S.make_weight(S.TYPE_Q4_K, 5632, 2048, seed=0)
    x = S.make_activation(1, 2048, seed=0)
    check_matmul(ctx, W, x)


def test_config1_q8_0(ctx):
    W = S.make_weight(S.TYPE_Q8_0, 2048, 2048, seed=1)
    x = S.make_activation(1, 2048, seed=1)
    check_matmul(ctx, W, x)


def test_config1_q6k_lm_head(ctx):
    W = S.make_weight(S.TYPE_Q6_K, 32000, 2048, seed=1)
    x = S.make_activation(1, 2048, seed=2)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("m", [1, 8])
def test_config4_llama3_ffn(ctx, n, k, m):
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=4)
    x = S.make_activation(m, k, seed=40 + m)
    check_matmul(ctx, W, x, cond=(m == 1))


def test_config4_llama3_lm_head_q6k(ctx):
    W = S.make_weight(S.TYPE_Q6_K, 128256, 4096, seed=5)
    x = S.make_activation(1, 4096, seed=50)
    check_matmul(ctx, W, x, sums=False, cond=False)


# ----------------------------------------------- prefill GEMM (int8 MFMA, m > 8)
@pytest.mark.parametrize("n,k", [(5632, 2048), (2048, 5632)])
def test_config3_prefill_gemm(ctx, n, k):
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=3)
    x = S.make_activation(512, k, seed=30 + k)
    check_matmul(ctx, W, x)


def test_config4_prefill_gemm_llama3_ffn_up(ctx):
    W = S.make_weight(S.TYPE_Q4_K, 14336, 4096, seed=4)
    x = S.make_activation(512, 4096, seed=44)
    check_matmul(ctx, W, x, sums=False, cond=False)


@pytest.mark.parametrize("m,n,k", [(9, 100, 256), (63, 129, 768), (65, 300, 512), (130, 257, 1024), (200, 64, 2048)])
def test_prefill_gemm_ragged_tiles(ctx, m, n, k):
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=m + n)
    x = S.make_activation(m, k, seed=m * n)
    check_matmul(ctx, W, x)


def test_prefill_gemm_extreme_values(ctx):
    """Largest integer sums the Q4_K . Q8_K product can form: all quants 15,
    all scales and mins 63, and activation blocks of equal values (every
    quant -128)."""
    n, k, m = 64, 1024, 16
    rng = np.random.default_rng(5)
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=5)
    W.q[:] = 15
    W.sc[:] = 63
    W.mn[:] = 63
    W.blocks = S.pack_q4k(W.d, W.dmin, W.sc, W.mn, W.q)
    x = np.repeat(rng.standard_normal((m, k // 256)).astype(np.float32), 256, axis=1)
    x[1::2] = -np.abs(x[1::2])
    check_matmul(ctx, W, x, cond=False)


@pytest.mark.parametrize("m,n,k", [
    (128, 128, 256),    # two m-tiles, one n-tile, one super-block
    (129, 300, 1280),   # a last m-tile of one row; 5 super-blocks split 3 + 2
    (384, 1000, 3840),  # 15 super-blocks: an odd count per split
    (511, 64, 2048),    # one partial n-tile, many splits
    (640, 4100, 512),   # ragged columns, two super-blocks
    (200, 301, 2304),   # n % 4 != 0: the reduction one column per thread (else four)
])
def test_prefill_gemm_odd_splits(ctx, m, n, k):
    """Longer prompts with ragged rows and columns and K splits of unequal
    super-block counts (the split-K reduction adds them in split order, four
    columns per thread where n % 4 == 0, else one)."""
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=m + n + 7)
    x = S.make_activation(m, k, seed=m * 3 + n)
    check_matmul(ctx, W, x)


def test_prefill_gemm_extreme_values_long_prompt(ctx):
    """The largest Q4_K . Q8_K sums over 256 rows (four m-tiles)."""
    n, k, m = 256, 1024, 256
    rng = np.random.default_rng(6)
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=6)
    W.q[:] = 15
    W.sc[:] = 63
    W.mn[:] = 63
    W.blocks = S.pack_q4k(W.d, W.dmin, W.sc, W.mn, W.q)
    x = np.repeat(rng.standard_normal((m, k // 256)).astype(np.float32), 256, axis=1)
    x[1::2] = -np.abs(x[1::2])
    check_matmul(ctx, W, x, cond=False)


# ----------------------------------------- Q6_K prefill GEMM (f16 MFMA, m > 8)
@pytest.mark.parametrize("n,k,m", [(256, 2048, 512), (2048, 5632, 512), (32000, 2048, 16)])
def test_prefill_gemm_q6k(ctx, n, k, m):
    """TinyLlama attn_v and ffn_down at a 512-token prefill, and the lm_head
    shape at 16 rows: integer block sums bit-exact, outputs within tolerance."""
    W = S.make_weight(S.TYPE_Q6_K, n, k, seed=n + k)
    x = S.make_activation(m, k, seed=m + k)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("m,n,k", [(9, 100, 256), (63, 129, 768), (65, 300, 512), (130, 257, 1024), (200, 64, 2048)])
def test_prefill_gemm_q6k_ragged_tiles(ctx, m, n, k):
    W = S.make_weight(S.TYPE_Q6_K, n, k, seed=m + n + 1)
    x = S.make_activation(m, k, seed=m * n + 1)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("m,n,k", [(1, 300, 2048), (3, 300, 2048), (8, 96, 1024), (16, 256, 2048),
                                   (512, 256, 2048), (77, 129, 768)])
def test_q6k_full_range_sub_scales(ctx, m, n, k):
    """Q6_K sub-scales over the whole int8 range, as llama.cpp's quantizer
    writes them (the largest sub-block scale of each super-block maps to
    -128): sc * (q6 - 32) reaches 4096, beyond the integers f16 holds
    exactly, so the prefill GEMM splits each scale into two digits.  Every
    path -- matvec (m = 1), matrix-core matvec (m = 3, 8), GEMM (m >= 16) --
    keeps the integer block sums bit-exact."""
    rng = np.random.default_rng(m * 7 + n)
    W = S.make_weight(S.TYPE_Q6_K, n, k, seed=m + n)
    W.sc[:] = rng.integers(-128, 128, size=W.sc.shape).astype(np.int8)
    W.sc[..., 0] = -128  # the quantizer's own extreme in every super-block
    W.blocks = S.pack_q6k(W.d, W.sc, W.q)
    x = S.make_activation(m, k, seed=m + k)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("sc", [-128, 127, -32])
def test_prefill_gemm_q6k_extreme_values(ctx, sc):
    """Largest Q6_K . Q8_K sums: every quant -32, every sub-scale at an end of
    the int8 range that llama.cpp's quantizer uses (-128: S = 2^27 per
    super-block, its high-digit chain exactly 2^23; 127: the low digit 15,
    its chain 480 * 256 * 128 < 2^24) or -32, against activation blocks of
    equal values (every quant +-128)."""
    n, k, m = 64, 1024, 16
    rng = np.random.default_rng(6)
    W = S.make_weight(S.TYPE_Q6_K, n, k, seed=6)
    W.q[:] = -32
    W.sc[:] = sc
    W.blocks = S.pack_q6k(W.d, W.sc, W.q)
    x = np.repeat(np.abs(rng.standard_normal((m, k // 256))).astype(np.float32) + 0.5, 256, axis=1)
    x[1::2] = -x[1::2]
    check_matmul(ctx, W, x, cond=False)


# ------------------------------------------------------ batch and K coverage
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 7, 8, 11])
@pytest.mark.parametrize("wtype", [S.TYPE_Q4_K, S.TYPE_Q5_K, S.TYPE_Q6_K, S.TYPE_Q8_0, S.TYPE_Q4_0, S.TYPE_Q2_K,
                                   S.TYPE_Q3_K, S.TYPE_Q5_0])
def test_batches(ctx, wtype, m):
    W = S.make_weight(wtype, 300, 2048, seed=m + wtype)
    x = S.make_activation(m, 2048, seed=100 + m)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("k", [256, 512, 5632, 16384, 20480])
@pytest.mark.parametrize("wtype", [S.TYPE_Q4_K, S.TYPE_Q5_K, S.TYPE_Q6_K, S.TYPE_Q8_0, S.TYPE_Q4_0, S.TYPE_Q2_K,
                                   S.TYPE_Q3_K, S.TYPE_Q5_0])
@pytest.mark.parametrize("m", [1, 8])
def test_k_coverage(ctx, wtype, k, m):
    W = S.make_weight(wtype, 70, k, seed=k + m)
    x = S.make_activation(m, k, seed=k)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize("wtype,n,k", [
    (S.TYPE_Q4_K, 4096, 14336),   # Llama-3-8B ffn_down at batch 8: four chunk wavefronts per tile
    (S.TYPE_Q4_K, 32768, 8192),   # one chunk per tile, eight steps per wavefront (more than stay in flight)
    (S.TYPE_Q6_K, 4096, 14336),
])
def test_batch8_long_rows(ctx, wtype, n, k):
    """The matrix-core matvec at batch 8 on long rows: every step of a
    wavefront's chunk, with later steps' weights in flight."""
    W = S.make_weight(wtype, n, k, seed=n + k + 8)
    x = S.make_activation(8, k, seed=k + 8)
    check_matmul(ctx, W, x, cond=False)


@pytest.mark.parametrize("n,k,m", [
    (200, 8960, 5),    # 35 super-blocks: 9 quads, the last one of three, parts of 3 quads
    (64, 9216, 8),     # 9 quads in 3 parts
    (4096, 16384, 2),  # 16 quads in 4 parts, many tile groups per workgroup
    (24, 14336, 8),    # fewer tiles than a workgroup takes
])
def test_batch_q4k_k_parts(ctx, n, k, m):
    """Q4_K rows of more than 8 quads at batch 2-8: K split over
    workgroups, the parts added by a second launch; block sums bit-exact."""
    W = S.make_weight(S.TYPE_Q4_K, n, k, seed=n + k + m)
    x = S.make_activation(m, k, seed=k + m + 1)
    check_matmul(ctx, W, x, cond=(k < 14336))


@pytest.mark.parametrize("k", [55296, 65536])
@pytest.mark.parametrize("wtype", [S.TYPE_Q4_K, S.TYPE_Q8_0])
@pytest.mark.parametrize("m", [1, 3])
def test_long_rows_large_lds(ctx, wtype, k, m):
    # activation records above 64 KB of LDS per workgroup, batch split into passes
    W = S.make_weight(wtype, 24, k, seed=k + m + wtype)
    x = S.make_activation(m, k, seed=k + 1)
    check_matmul(ctx, W, x)


def test_single_row_weight(ctx):
    W = S.make_weight(S.TYPE_Q4_K, 1, 256, seed=3)
    x = S.make_activation(2, 256, seed=3)
    check_matmul(ctx, W, x)


# ------------------------------------ Q5_K (matvec m <= 8, f16 MFMA GEMM m > 8)
@pytest.mark.parametrize("n,k,m", [(5632, 2048, 1), (2048, 5632, 1), (14336, 4096, 1), (4096, 14336, 8),
                                   (2048, 2048, 40)])
def test_q5k_matvec(ctx, n, k, m):
    """TinyLlama / Llama-3 FFN shapes of a Q5_K_M file, batch 1 and 8, and a
    40-row prefill (the GEMM): block sums bit-exact."""
    W = S.make_weight(S.TYPE_Q5_K, n, k, seed=n + k + 5)
    x = S.make_activation(m, k, seed=m + k + 5)
    check_matmul(ctx, W, x, cond=(m <= 8 and k < 14336))


def test_q5k_extreme_values(ctx):
    """Largest Q5_K . Q8_K sums: every quant 31 (all five bits set), scales
    and mins 63, activation blocks of equal values (quants -128)."""
    n, k, m = 40, 1024, 3
    rng = np.random.default_rng(25)
    W = S.make_weight(S.TYPE_Q5_K, n, k, seed=25)
    W.q[:] = 31
    W.sc[:] = 63
    W.mn[:] = 63
    W.blocks = S.pack_q5k(W.d, W.dmin, W.sc, W.mn, W.q)
    x = np.repeat(rng.standard_normal((m, k // 256)).astype(np.float32), 256, axis=1)
    check_matmul(ctx, W, x, cond=False)


@pytest.mark.parametrize("n,k,m", [(2048, 2048, 512), (5632, 2048, 64), (2048, 5632, 33), (32000, 2048, 16)])
def test_prefill_gemm_q5k(ctx, n, k, m):
    """TinyLlama attn_q / ffn_up / ffn_down shapes of a Q5_K_M file at
    prefill (k-splits of two super-blocks at 512 rows) and the lm_head shape
    at 16 rows: integer block sums S and Smin bit-exact."""
    W = S.make_weight(S.TYPE_Q5_K, n, k, seed=n + k + 13)
    x = S.make_activation(m, k, seed=m + k + 13)
    check_matmul(ctx, W, x, cond=(k < 14336))


@pytest.mark.parametrize("m,n,k", [(9, 100, 256), (63, 129, 768), (65, 300, 512), (130, 257, 1024), (200, 64, 2048)])
def test_prefill_gemm_q5k_ragged_tiles(ctx, m, n, k):
    W = S.make_weight(S.TYPE_Q5_K, n, k, seed=m + n + 13)
    x = S.make_activation(m, k, seed=m * n + 13)
    check_matmul(ctx, W, x)


def test_prefill_gemm_q5k_extreme_values(ctx):
    """Largest Q5_K . Q8_K sums on the GEMM: every quant 31, scales and mins
    63, activation blocks of equal values (quants +-128 / 127): each
    64-element f32 MFMA chain reaches 64 * 1953 * 128 < 2^24 and S four times
    that; Smin 16 * 2048 * 63."""
    n, k, m = 64, 1024, 16
    rng = np.random.default_rng(26)
    W = S.make_weight(S.TYPE_Q5_K, n, k, seed=26)
    W.q[:] = 31
    W.sc[:] = 63
    W.mn[:] = 63
    W.blocks = S.pack_q5k(W.d, W.dmin, W.sc, W.mn, W.q)
    x = np.repeat(np.abs(rng.standard_normal((m, k // 256))).astype(np.float32) + 0.5, 256, axis=1)
    x[1::2] = -x[1::2]
    check_matmul(ctx, W, x, cond=False)


# ------------------------------------------------------------ Q4_0 (matvec at any m)
@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (14336, 4096, 1), (4096, 14336, 8), (300, 96, 3),
                                   (129, 1056, 5), (2048, 2048, 20)])
def test_q4_0_matvec(ctx, n, k, m):
    """Llama-3 FFN shapes of a Q4_0 file, rows whose block count is not a
    multiple of 8 (96 and 1056 columns: padding blocks in the tile layout),
    and a 20-row batch (passes of 8): block sums bit-exact."""
    W = S.make_weight(S.TYPE_Q4_0, n, k, seed=n + k + 7)
    x = S.make_activation(m, k, seed=m + k + 7)
    check_matmul(ctx, W, x, cond=(k < 14336))


@pytest.mark.parametrize("n,k,m", [(1024, 2048, 64), (300, 1056, 40), (2048, 96, 17)])
def test_q4_0_prefill_gemm(ctx, n, k, m):
    """m > 8: the Q8_0 GEMM on the upload's expanded copy (values q - 8 as
    int8), including rows with padding blocks: block sums bit-exact."""
    W = S.make_weight(S.TYPE_Q4_0, n, k, seed=n + k + 9)
    x = S.make_activation(m, k, seed=m + k + 9)
    check_matmul(ctx, W, x, cond=False)


def test_q4_0_extreme_values(ctx):
    """Every quant 0 (value -8) against activation blocks of equal values
    (quants +-127): |S| = 32 * 8 * 127 per block, and every quant 15."""
    n, k, m = 64, 512, 2
    rng = np.random.default_rng(27)
    for qv in (0, 15):
        W = S.make_weight(S.TYPE_Q4_0, n, k, seed=27)
        W.q[:] = qv
        W.blocks = S.pack_q4_0(W.d, W.q)
        x = np.repeat(rng.standard_normal((m, k // 32)).astype(np.float32), 32, axis=1)
        check_matmul(ctx, W, x, cond=False)


# ----------------------------- Q5_0 (matvec m <= 8, Q8_0 GEMM on a copy m > 8)
@pytest.mark.parametrize("n,k,m", [(14336, 4096, 1), (4096, 14336, 8), (300, 96, 3), (1024, 2048, 64),
                                   (300, 1056, 40)])
def test_q5_0_matvec_and_gemm(ctx, n, k, m):
    """Llama-3 FFN shapes of a Q5_0 file, rows whose block count is not a
    multiple of 8 (padding blocks), and m > 8 through the Q8_0 GEMM on the
    upload's expanded copy (values q - 16): block sums bit-exact."""
    W = S.make_weight(S.TYPE_Q5_0, n, k, seed=n + k + 6)
    x = S.make_activation(m, k, seed=m + k + 6)
    check_matmul(ctx, W, x, cond=(k < 14336 and m <= 8))


@pytest.mark.parametrize("qv,m", [(0, 2), (31, 2), (0, 20), (31, 20)])
def test_q5_0_extreme_values(ctx, qv, m):
    """Every quant 0 (value -16) or 31 (value 15) against activation blocks of
    equal values, on the matvec (2 rows) and the GEMM (20 rows)."""
    n, k = 64, 512
    rng = np.random.default_rng(33)
    W = S.make_weight(S.TYPE_Q5_0, n, k, seed=33)
    W.q[:] = qv
    W.blocks = S.pack_q5_0(W.d, W.q)
    x = np.repeat(rng.standard_normal((m, k // 32)).astype(np.float32), 32, axis=1)
    check_matmul(ctx, W, x, cond=False)


# ------------------------------------------- Q2_K, Q3_K (matvec at any m)
@pytest.mark.parametrize("wtype", [S.TYPE_Q2_K, S.TYPE_Q3_K])
@pytest.mark.parametrize("n,k,m", [(14336, 4096, 1), (4096, 14336, 8), (5632, 2048, 1), (300, 2048, 20)])
def test_q2k_q3k_matvec(ctx, wtype, n, k, m):
    """Llama-3 and TinyLlama FFN shapes of Q2_K / Q3_K files, batch 1 and 8,
    and 20 rows (passes of 8): block sums bit-exact."""
    W = S.make_weight(wtype, n, k, seed=n + k + wtype)
    x = S.make_activation(m, k, seed=m + k + wtype)
    check_matmul(ctx, W, x, cond=(k < 14336))


def test_q2k_extreme_values(ctx):
    """Every quant 3, scales and mins 15, activation blocks of equal values
    (quants +-128 / 127): the largest |S| and |Smin| a Q2_K block reaches."""
    n, k, m = 40, 1024, 3
    rng = np.random.default_rng(31)
    W = S.make_weight(S.TYPE_Q2_K, n, k, seed=31)
    W.q[:] = 3
    W.sc[:] = 15
    W.mn[:] = 15
    W.blocks = S.pack_q2k(W.d, W.dmin, W.sc, W.mn, W.q)
    x = np.repeat(rng.standard_normal((m, k // 256)).astype(np.float32), 256, axis=1)
    check_matmul(ctx, W, x, cond=False)


@pytest.mark.parametrize("qv,scv", [(-4, -32), (3, 31), (-4, 31)])
def test_q3k_extreme_values(ctx, qv, scv):
    """Every quant -4 (hmask bits clear) or 3, every scale -32 or 31,
    activation blocks of equal values."""
    n, k, m = 40, 1024, 3
    rng = np.random.default_rng(32)
    W = S.make_weight(S.TYPE_Q3_K, n, k, seed=32)
    W.q[:] = qv
    W.sc[:] = scv
    W.blocks = S.pack_q3k(W.d, W.sc, W.q)
    x = np.repeat(rng.standard_normal((m, k // 256)).astype(np.float32), 256, axis=1)
    check_matmul(ctx, W, x, cond=False)


# ------------------------------------------ Q8_0 prefill GEMM (int8 MFMA, m > 8)
@pytest.mark.parametrize("n,k,m", [(768, 2048, 256), (4096, 4096, 16)])
def test_prefill_gemm_q8_0(ctx, n, k, m):
    """A 256-token prefill and a 16-row batch (four k-splits per tile):
    integer block sums bit-exact, outputs within tolerance."""
    W = S.make_weight(S.TYPE_Q8_0, n, k, seed=n + k + 2)
    x = S.make_activation(m, k, seed=m + k + 2)
    check_matmul(ctx, W, x)


@pytest.mark.parametrize(
    "m,n,k",
    [(9, 100, 256), (63, 129, 768), (65, 300, 512), (130, 257, 1024), (200, 64, 2048),
     (33, 50, 32), (40, 70, 96), (17, 130, 1056)],
)
def test_prefill_gemm_q8_0_ragged_tiles(ctx, m, n, k):
    """Partial tiles in m and n, and k an odd number of blocks (32, 96, 1056:
    the last step's second block is padding)."""
    W = S.make_weight(S.TYPE_Q8_0, n, k, seed=m + n + 2)
    x = S.make_activation(m, k, seed=m * n + 2)
    check_matmul(ctx, W, x)


def test_prefill_gemm_q8_0_extreme_values(ctx):
    """Largest Q8_0 . Q8_0 block sums: every weight quant -128 and activation
    blocks of equal values (every quant +-127), |S| = 32 * 128 * 127, the
    widest sum the GEMM's offset accumulator (1.5 * 2^23 + S read as f32)
    must hold exactly."""
    n, k, m = 64, 1024, 16
    rng = np.random.default_rng(7)
    W = S.make_weight(S.TYPE_Q8_0, n, k, seed=7)
    W.q[:] = -128
    W.blocks = S.pack_q8_0(W.d, W.q)
    x = np.repeat(rng.standard_normal((m, k // 32)).astype(np.float32), 32, axis=1)
    x[1::2] = -np.abs(x[1::2])
    x[::2] = np.abs(x[::2])
    check_matmul(ctx, W, x, cond=False)


def test_prefill_gemm_q8_0_subnormal_and_zero_scales(ctx):
    W = S.make_weight(S.TYPE_Q8_0, 128, 1024, seed=18)
    rng = np.random.default_rng(18)
    d = (rng.integers(1, 1024, size=W.d.shape).astype(np.uint16)).view(np.float16)
    d[::5] = 0
    W.blocks = S.pack_q8_0(d, W.q)
    W.d = d
    x = S.make_activation(40, 1024, seed=19)
    check_matmul(ctx, W, x, cond=False)


@pytest.mark.parametrize("m", [3, 20])
@pytest.mark.parametrize("wtype", [S.TYPE_Q4_K, S.TYPE_Q5_K, S.TYPE_Q6_K, S.TYPE_Q8_0, S.TYPE_Q4_0, S.TYPE_Q2_K,
                                   S.TYPE_Q3_K, S.TYPE_Q5_0])
def test_subnormal_and_zero_scales(ctx, wtype, m):
    """f16 subnormal and zero d / dmin through the matvec (3 rows) and the
    GEMMs (20 rows)."""
    W = S.make_weight(wtype, 128, 1024, seed=8)
    rng = np.random.default_rng(8)
    d = (rng.integers(1, 1024, size=W.d.shape).astype(np.uint16)).view(np.float16)  # f16 subnormals
    d[::5] = 0
    if wtype in (S.TYPE_Q4_K, S.TYPE_Q5_K):
        pack = S.pack_q4k if wtype == S.TYPE_Q4_K else S.pack_q5k
        W.blocks = pack(d, d[:, ::-1].copy(), W.sc, W.mn, W.q)
        W.dmin = d[:, ::-1].copy()
    elif wtype == S.TYPE_Q6_K:
        W.blocks = S.pack_q6k(d, W.sc, W.q)
    elif wtype == S.TYPE_Q4_0:
        W.blocks = S.pack_q4_0(d, W.q)
    elif wtype == S.TYPE_Q5_0:
        W.blocks = S.pack_q5_0(d, W.q)
    elif wtype == S.TYPE_Q2_K:
        W.blocks = S.pack_q2k(d, d[:, ::-1].copy(), W.sc, W.mn, W.q)
        W.dmin = d[:, ::-1].copy()
    elif wtype == S.TYPE_Q3_K:
        W.blocks = S.pack_q3k(d, W.sc, W.q)
    else:
        W.blocks = S.pack_q8_0(d, W.q)
    W.d = d
    x = S.make_activation(m, 1024, seed=9)
    check_matmul(ctx, W, x, cond=False)


# ----------------------------------------------------------- API behaviour
def test_m_zero_and_shape_errors(ctx):
    W = S.make_weight(S.TYPE_Q4_K, 16, 512, seed=1)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (16, 512), W.blocks), ctx)
    y = mm.forward(np.zeros((0, 512), np.float32))
    assert y.shape == (0, 16)
    with pytest.raises(A.QMatMulError):
        mm.forward(np.zeros((1, 256), np.float32))
    L = A._lib.load()
    x = np.zeros((1, 256), np.float32)
    dst = np.zeros((1, 16), np.float32)
    rc = L.aq_qmatmul_f32(ctx.handle, mm.handle, x.ctypes.data, 1, 256, dst.ctypes.data)
    assert rc == A._lib.AQ_ERR_SHAPE
    with pytest.raises(A.AqError):
        A.QMatMul.from_device_blocks(ctx, 99, (16, 512), 1, 16 * 2 * 144)
    mm.free()


def test_higher_rank_input_and_determinism(ctx):
    W = S.make_weight(S.TYPE_Q6_K, 96, 1024, seed=2)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (96, 1024), W.blocks), ctx)
    x = S.make_activation(6, 1024, seed=2).reshape(2, 3, 1024)
    y1 = mm.forward(x)
    y2 = mm.forward(x)
    assert y1.shape == (2, 3, 96)
    assert np.array_equal(y1, y2)
    r = O.matmul(W.type, x.reshape(6, 1024), W.blocks, 96, 1024).reshape(2, 3, 96)
    assert rel_max(y1, r) <= 1e-5
    mm.free()


@pytest.mark.parametrize("wtype,m", [(S.TYPE_Q4_K, 4), (S.TYPE_Q6_K, 1), (S.TYPE_Q8_0, 8), (S.TYPE_Q4_K, 40),
                                     (S.TYPE_Q5_K, 3), (S.TYPE_Q5_K, 24), (S.TYPE_Q4_0, 2), (S.TYPE_Q2_K, 3),
                                     (S.TYPE_Q3_K, 12), (S.TYPE_Q5_0, 5), (S.TYPE_Q5_0, 40)])
def test_device_pointer_entry_points(ctx, wtype, m):
    from arm_ai_amd import hip

    W = S.make_weight(wtype, 512, 2048, seed=12)
    x = S.make_activation(m, 2048, seed=12)
    mm = A.QMatMul.from_qtensor(A.QTensor(W.type, (512, 2048), W.blocks), ctx)
    y_host = mm.forward(x)
    dx = hip.to_device(x)
    dy = hip.DeviceBuffer(m * 512 * 4)
    mm.forward_device(dx.ptr, m, dy.ptr)
    ctx.synchronize()
    assert np.array_equal(dy.download(np.float32, (m, 512)), y_host)
    # quantise once, reuse: same bytes as the fused call
    act = hip.DeviceBuffer(A.act_bytes(mm.act_type, m, 2048))
    A.quantize_act_device(ctx, mm.act_type, dx.ptr, m, 2048, act.ptr)
    dy2 = hip.DeviceBuffer(m * 512 * 4)
    mm.forward_preq_device(act.ptr, m, dy2.ptr)
    ctx.synchronize()
    assert np.array_equal(dy2.download(np.float32, (m, 512)), y_host)
    # weights uploaded from device memory give the same result
    dblocks = hip.to_device(W.blocks)
    mm2 = A.QMatMul.from_device_blocks(ctx, W.type, (512, 2048), dblocks.ptr, W.blocks.size)
    assert np.array_equal(mm2.forward(x), y_host)
    mm.free()
    mm2.free()


# ------------------------------------------------------- chunked weight upload
@pytest.mark.parametrize("wtype", [S.TYPE_Q2_K, S.TYPE_Q6_K, S.TYPE_Q5_0, S.TYPE_Q4_0, S.TYPE_Q8_0, S.TYPE_Q4_K])
def test_upload_in_many_chunks(ctx, wtype, monkeypatch):
    """A weight staged through the upload buffer in many chunks (8 rows each,
    n % 8 != 0) gives the same device bytes' results as a one-chunk upload:
    the tile rows, the Q2_K / Q6_K d planes and the Q4_0 / Q5_0 expanded GEMM
    copies are offset per chunk.  Checked through the matvec (3 rows) and
    the prefill GEMM (20 rows) against the oracle and the one-chunk upload."""
    n, k = 203, 2048
    W = S.make_weight(wtype, n, k, seed=wtype + 90)
    one = A.QMatMul.from_qtensor(A.QTensor(wtype, (n, k), W.blocks), ctx)
    row_bytes = W.blocks.nbytes // n
    monkeypatch.setenv("ARM_AI_AMD_UPLOAD_STAGE_BYTES", str(8 * row_bytes))
    many = A.QMatMul.from_qtensor(A.QTensor(wtype, (n, k), W.blocks), ctx)
    monkeypatch.delenv("ARM_AI_AMD_UPLOAD_STAGE_BYTES")
    for m in (3, 20):
        x = S.make_activation(m, k, seed=m)
        y_many, y_one = many.forward(x), one.forward(x)
        assert np.array_equal(y_many, y_one)
        sm, smm = many.block_sums(x)
        so, smo = one.block_sums(x)
        assert np.array_equal(sm, so) and np.array_equal(smm, smo)
        r = O.matmul(wtype, x, W.blocks, n, k)
        assert rel_max(y_many, r) <= 1e-5
    many.free()
    one.free()
