"""Known-answer vectors (tests/golden/golden.npz, written by
tests/golden/make_golden.py from an independent numpy restatement of the GGUF
formats and quantizers, cross-checked there against the C oracle).

CPU: the oracle reproduces every vector (bytes and integers exactly; its f32
matmul output exactly, since it is deterministic).  GPU: the library, called
through the C ABI, reproduces the quantised bytes and the integer block sums
exactly and the f32 outputs within the path's tolerance (max relative error
1e-5 at these K).
"""
import os

import numpy as np
import pytest

import oracle as O

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
K = 512
WTYPES = (("q4k", O.Q4_K), ("q6k", O.Q6_K), ("q8_0", O.Q8_0))


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ---------------------------------------------------------------- oracle
def test_oracle_activation_quantizers():
    assert np.array_equal(O.quantize(G["act_x"], O.Q8_K).reshape(-1), G["act_q8k"])
    assert np.array_equal(O.quantize(G["act_x"], O.Q8_0).reshape(-1), G["act_q8_0"])


@pytest.mark.parametrize("name,wtype", WTYPES)
def test_oracle_block_sums_and_outputs(name, wtype):
    w, x = G[f"{name}_w"], G[f"{name}_x"]
    xq = O.quantize(x, O.act_type(wtype))
    S, Smin = O.block_sums(wtype, K, w, xq)
    assert np.array_equal(S, G[f"{name}_S"]) and np.array_equal(Smin, G[f"{name}_Smin"])
    assert np.array_equal(O.matmul(wtype, x, w, G[f"{name}_S"].shape[1], K), G[f"{name}_y"])


def test_oracle_crate_quantizers():
    q, s = O.quantize_int8_per_token(G["crate_i8_x"], *G["crate_i8_x"].shape)
    assert np.array_equal(q, G["crate_i8_q"]) and np.array_equal(s, G["crate_i8_s"])
    q, s = O.quantize_q8_groups(G["crate_q8g_x"], G["crate_q8g_x"].size)
    assert np.array_equal(q, G["crate_q8g_q"]) and np.array_equal(s, G["crate_q8g_s"])
    p, s = O.quantize_int4_q4_0(G["crate_q4_x"], *G["crate_q4_x"].shape)
    assert np.array_equal(p, G["crate_q4_p"]) and np.array_equal(s, G["crate_q4_s"])


def test_planted_mistakes_fail():
    # a sign flip of one activation row and one flipped quant bit must not pass
    x = G["act_x"].copy()
    x[0] = -x[0]
    assert not np.array_equal(O.quantize(x, O.Q8_K).reshape(-1), G["act_q8k"])
    w = G["q4k_w"].copy()
    w[16] ^= 0x01  # lowest bit of the first qs byte of row 0, block 0
    xq = O.quantize(G["q4k_x"], O.Q8_K)
    S, _ = O.block_sums(O.Q4_K, K, w, xq)
    assert not np.array_equal(S, G["q4k_S"])
    assert np.any(G["q4k_Smin"] != 0) and np.any(G["q6k_S"] < 0)


# ------------------------------------------------------------------- GPU
@pytest.mark.gpu
def test_gpu_activation_quantizers(ctx):
    import arm_ai_amd as A

    assert np.array_equal(A.quantize_q8k(ctx, G["act_x"]).reshape(-1), G["act_q8k"])
    assert np.array_equal(A.quantize_q8_0(ctx, G["act_x"]).reshape(-1), G["act_q8_0"])


@pytest.mark.gpu
@pytest.mark.parametrize("name,wtype", WTYPES)
def test_gpu_block_sums_and_outputs(ctx, name, wtype):
    import arm_ai_amd as A

    w, x = G[f"{name}_w"], G[f"{name}_x"]
    n = G[f"{name}_S"].shape[1]
    mm = A.QMatMul.from_qtensor(A.QTensor(wtype, (n, K), w), ctx)
    for rows in (x[:1], x):  # one row (matvec) and three rows (the batched path)
        S, Smin = mm.block_sums(rows)
        assert np.array_equal(S, G[f"{name}_S"][: len(rows)])
        assert np.array_equal(Smin, G[f"{name}_Smin"][: len(rows)])
        assert _rel(mm.forward(rows), G[f"{name}_y"][: len(rows)]) <= 1e-5
    mm.free()


@pytest.mark.gpu
def test_gpu_crate_quantizers(ctx):
    from arm_ai_amd import crate_ops as C

    q, s = C.quantize_int8_per_token(ctx, G["crate_i8_x"], *G["crate_i8_x"].shape)
    assert np.array_equal(q, G["crate_i8_q"]) and np.array_equal(s, G["crate_i8_s"])
    p, s = C.quantize_int4_q4_0(ctx, G["crate_q4_x"], *G["crate_q4_x"].shape)
    assert np.array_equal(p, G["crate_q4_p"]) and np.array_equal(s, G["crate_q4_s"])
