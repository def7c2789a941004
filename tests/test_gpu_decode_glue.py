"""GPU tests of the decode-step glue kernels (k_decode.hip) through the C ABI,
each against a numpy restatement of the candle-transformers quantized_llama
operation it stands for (rms_norm, silu, rope_i + grouped-query attention
over a KV cache, first-maximum argmax).  f32 sums are reordered on the GPU, so
values are compared at 1e-5 relative; argmax and the cache writes are exact.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch

    import arm_ai_amd as A

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need torch to see the GPU (import torch before the library)")
    ctx = A.Context(0)
    yield torch, A._lib, ctx
    ctx.close()


def _dev(torch, a):
    """A device copy, complete before the library's stream uses it."""
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    torch.cuda.synchronize()
    return t


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def test_rmsnorm_with_and_without_residual(env):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(0)
    m, n, eps = 3, 2048, 1e-5
    x = rng.standard_normal((m, n)).astype(np.float32)
    d = rng.standard_normal((m, n)).astype(np.float32)
    w = (1 + 0.05 * rng.standard_normal(n)).astype(np.float32)
    dx, dd, dw = _dev(torch, x), _dev(torch, d), _dev(torch, w)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_rmsnorm(ctx.handle, dx.data_ptr(), None, dw.data_ptr(), m, n, ctypes.c_float(eps),
                                 out.data_ptr()))
    ctx.synchronize()
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    assert _rel(out.cpu().numpy(), x / np.sqrt(ms + eps) * w) <= 1e-5
    assert np.array_equal(dx.cpu().numpy(), x)  # no delta: x untouched
    lib.check(L.aq_llama_rmsnorm(ctx.handle, dx.data_ptr(), dd.data_ptr(), dw.data_ptr(), m, n, ctypes.c_float(eps),
                                 out.data_ptr()))
    ctx.synchronize()
    h = x + d
    assert np.array_equal(dx.cpu().numpy(), h)  # the residual add is written back exactly
    ms = np.mean(h.astype(np.float64) ** 2, axis=-1, keepdims=True)
    assert _rel(out.cpu().numpy(), h / np.sqrt(ms + eps) * w) <= 1e-5


def test_silu_mul(env):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(1)
    n = 5632
    gu = (4 * rng.standard_normal(2 * n)).astype(np.float32)
    gu[0], gu[1] = -100.0, 100.0  # exp overflow / underflow ends
    dgu = _dev(torch, gu)
    out = torch.empty(n, dtype=torch.float32, device="cuda:0")
    lib.check(L.aq_llama_silu_mul(ctx.handle, dgu.data_ptr(), n, out.data_ptr()))
    ctx.synchronize()
    g, u = gu[:n].astype(np.float64), gu[n:].astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert _rel(got, want) <= 1e-5


def _rope(x, c, s):
    out = np.empty_like(x)
    a, b = x[..., 0::2], x[..., 1::2]
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


@pytest.mark.parametrize(
    "n_head,n_kv,hd,pos,max_seq",
    [(32, 4, 64, 0, 1024), (32, 4, 64, 517, 1024), (8, 8, 128, 300, 1024), (4, 2, 32, 1023, 1024),
     # contexts past the rows each thread loads ahead (one key row, up to
     # eight value rows per thread), the narrowest and widest heads
     (32, 4, 64, 4095, 4096), (8, 2, 256, 2500, 4096), (16, 4, 8, 3000, 4096), (8, 1, 128, 1800, 2048),
     # three query heads per kv head (SmolLM-135M: 9 / 3)
     (9, 3, 64, 0, 640), (9, 3, 64, 600, 640), (6, 2, 128, 2047, 2048)],
)
def test_attn_decode_against_numpy(env, n_head, n_kv, hd, pos, max_seq):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(pos + hd)
    qk = rng.standard_normal((n_head + n_kv) * hd).astype(np.float32)
    v = rng.standard_normal(n_kv * hd).astype(np.float32)
    kc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    theta = 1.0 / (10000.0 ** (np.arange(0, hd, 2, dtype=np.float32) / hd))
    ang = np.arange(max_seq, dtype=np.float32)[:, None] * theta[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    dqk, dv, dkc, dvc = _dev(torch, qk), _dev(torch, v), _dev(torch, kc), _dev(torch, vc)
    dcos, dsin = _dev(torch, cos), _dev(torch, sin)
    dpos = torch.tensor([pos], dtype=torch.int64, device="cuda:0")
    out = torch.empty(n_head * hd, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_attn_decode(ctx.handle, dqk.data_ptr(), dv.data_ptr(), dcos.data_ptr(), dsin.data_ptr(),
                                     dpos.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), n_head, n_kv, hd, max_seq,
                                     out.data_ptr()))
    ctx.synchronize()
    q = _rope(qk[:n_head * hd].reshape(n_head, hd), cos[pos], sin[pos])
    k = _rope(qk[n_head * hd:].reshape(n_kv, hd), cos[pos], sin[pos])
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, pos], vc2[:, pos] = k, v.reshape(n_kv, hd)
    rep = n_head // n_kv
    want = np.empty((n_head, hd))
    for h in range(n_head):
        kk = kc2[h // rep, :pos + 1].astype(np.float64)
        s = kk @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        want[h] = p @ vc2[h // rep, :pos + 1].astype(np.float64)
    assert _rel(out.cpu().numpy().reshape(n_head, hd), want) <= 1e-5
    # k, v stored at pos; every other cache entry untouched
    assert np.array_equal(dkc.cpu().numpy()[:, pos], k)
    assert np.array_equal(dvc.cpu().numpy(), vc2)
    got_k = dkc.cpu().numpy()
    got_k[:, pos] = kc[:, pos]
    assert np.array_equal(got_k, kc)


def test_argmax_first_max_history_and_position(env):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(2)
    x = rng.standard_normal(32000).astype(np.float32)
    x[777] = x[31000] = 50.0  # tie: the first index wins
    x[5] = np.nan  # a NaN never wins
    dx = _dev(torch, x)
    tok = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    pos = torch.tensor([10], dtype=torch.int64, device="cuda:0")
    hist = torch.full((16,), -1, dtype=torch.int64, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_argmax(ctx.handle, dx.data_ptr(), x.size, tok.data_ptr(), pos.data_ptr(), hist.data_ptr(), 16))
    ctx.synchronize()
    assert int(tok.item()) == 777
    assert int(pos.item()) == 11
    h = hist.cpu().numpy()
    assert h[10] == 777 and np.all(np.delete(h, 10) == -1)


@pytest.mark.parametrize("n,where", [(128256, 120001), (128256, 3)])
def test_argmax_llama3_vocab_tie_across_rounds(env, n, where):
    """A Llama-3 vocabulary (several rounds of eight float4 per thread): the
    maximum in a later round, then tied with one in the first round (the
    earlier index wins)."""
    torch, lib, ctx = env
    L = lib.load()
    x = np.random.default_rng(n + where).standard_normal(n).astype(np.float32)
    x[where] = 30.0
    tok = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    pos = torch.tensor([3], dtype=torch.int64, device="cuda:0")
    dx = _dev(torch, x)
    torch.cuda.synchronize()
    lib.check(L.aq_llama_argmax(ctx.handle, dx.data_ptr(), n, tok.data_ptr(), pos.data_ptr(), None, 0))
    ctx.synchronize()
    assert int(tok.item()) == where and int(pos.item()) == 4
    x[n - 1 - where] = 30.0
    dx = _dev(torch, x)
    torch.cuda.synchronize()
    lib.check(L.aq_llama_argmax(ctx.handle, dx.data_ptr(), n, tok.data_ptr(), pos.data_ptr(), None, 0))
    ctx.synchronize()
    assert int(tok.item()) == min(where, n - 1 - where) and int(pos.item()) == 5


@pytest.mark.parametrize("n,where", [(32001, 32000), (32003, 32001), (32003, 5), (7, 6), (1, 0)])
def test_argmax_vocab_not_a_multiple_of_four(env, n, where):
    """Vocabularies such as 32001 or 32003 (some Llama-2 fine-tunes): the
    elements past the last float4 are read one by one, and a maximum among
    them, or tied with one before them, is picked as candle picks it."""
    torch, lib, ctx = env
    L = lib.load()
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    x[where] = 40.0
    tok = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    pos = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    dx = _dev(torch, x)
    torch.cuda.synchronize()
    lib.check(L.aq_llama_argmax(ctx.handle, dx.data_ptr(), n, tok.data_ptr(), pos.data_ptr(), None, 0))
    ctx.synchronize()
    assert int(tok.item()) == where
    if n > 4 and where >= n - (n % 4):  # a tie with an earlier element: the earlier one wins
        x[1] = 40.0
        dx = _dev(torch, x)
        torch.cuda.synchronize()
        lib.check(L.aq_llama_argmax(ctx.handle, dx.data_ptr(), n, tok.data_ptr(), pos.data_ptr(), None, 0))
        ctx.synchronize()
        assert int(tok.item()) == 1


def test_embed_lookup_and_out_of_range(env):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(3)
    table = rng.standard_normal((100, 64)).astype(np.float32)
    dt = _dev(torch, table)
    out = torch.empty(64, dtype=torch.float32, device="cuda:0")
    for t, want in ((42, table[42]), (100, np.zeros(64, np.float32)), (-1, np.zeros(64, np.float32))):
        tok = torch.tensor([t], dtype=torch.int64, device="cuda:0")
        torch.cuda.synchronize()
        lib.check(L.aq_llama_embed(ctx.handle, dt.data_ptr(), 100, tok.data_ptr(), 64, out.data_ptr()))
        ctx.synchronize()
        assert np.array_equal(out.cpu().numpy(), want)


def test_glue_argument_errors(env):
    torch, lib, ctx = env
    L = lib.load()
    buf = torch.zeros(1024, dtype=torch.float32, device="cuda:0")
    pos = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    p = buf.data_ptr()
    # head_dim that does not divide the workgroup, n_head not a multiple of n_kv, max_seq too large
    for n_head, n_kv, hd, ms in ((4, 2, 48, 16), (6, 4, 64, 16), (4, 2, 64, 9000)):
        rc = L.aq_llama_attn_decode(ctx.handle, p, p, p, p, pos.data_ptr(), p, p, n_head, n_kv, hd, ms, p)
        assert rc != 0
    assert L.aq_llama_silu_mul(ctx.handle, None, 4, p) != 0
    assert L.aq_llama_argmax(ctx.handle, p, 0, pos.data_ptr(), pos.data_ptr(), None, 0) != 0


# ------------------------------------------------ matvec with a fused input transform
def _weight(A, S, wtype, n, k, ctx, seed):
    W = S.make_weight(wtype, n, k, seed=seed)
    return W, A.QMatMul.from_qtensor(A.QTensor(wtype, (n, k), W.blocks), ctx)


@pytest.mark.parametrize("wtype,n,k,with_delta", [
    (12, 2304, 2048, True), (14, 256, 2048, False), (12, 1000, 4096, True), (8, 300, 1024, True),
    (13, 2304, 2048, True),
    # the row-per-lane kernel's fused norm: 56-row workgroups, persistent
    # chunks, the 16-row form with four and eight wavefronts, ragged rows
    (12, 11264, 2048, True), (14, 32000, 2048, False), (12, 28672, 4096, True),
    (12, 4096, 4096, True), (14, 5000, 8192, True), (12, 3203, 2048, False),
])
def test_matvec_fused_rmsnorm(env, wtype, n, k, with_delta):
    """y = W . rms_norm(x + delta) * w_norm in one launch, against the oracle's
    matmul of the same input formed in numpy; h_out = x + delta exactly."""
    import oracle as O

    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(n + k)
    W, mm = _weight(A, S, wtype, n, k, ctx, seed=n)
    x = rng.standard_normal(k).astype(np.float32)
    d = rng.standard_normal(k).astype(np.float32) if with_delta else np.zeros(k, np.float32)
    wn = (1 + 0.05 * rng.standard_normal(k)).astype(np.float32)
    dx, dd, dwn = _dev(torch, x), _dev(torch, d), _dev(torch, wn)
    hout = torch.full((k,), np.nan, dtype=torch.float32, device="cuda:0")
    y = torch.empty(n, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, mm.handle, dx.data_ptr(),
                                              dd.data_ptr() if with_delta else None, dwn.data_ptr(),
                                              ctypes.c_float(1e-5), k, hout.data_ptr(), y.data_ptr()))
    ctx.synchronize()
    h = x + d
    assert np.array_equal(hout.cpu().numpy(), h)
    ms = np.float32(np.mean(h.astype(np.float64) ** 2))
    xin = ((h / np.sqrt(ms + np.float32(1e-5))) * wn).astype(np.float32)[None, :]
    r = O.matmul(wtype, xin, W.blocks, n, k)[0]
    # the row's sum of squares is reduced in another order, which can move a
    # Q8_K quant by one step: compare at 1e-3 of the output's scale
    assert _rel(y.cpu().numpy(), r) <= 1e-3
    mm.free()


@pytest.mark.parametrize("wtype,n,k", [(12, 2048, 5632), (14, 2048, 5632), (12, 300, 256), (13, 2048, 5632),
                                        (12, 200, 1024),     # below 256 rows: the general matvec
                                        (12, 14336, 4096),   # 56-row workgroups
                                        (14, 4096, 14336),   # the 16-row form with 16 wavefronts
                                        (12, 30000, 2048),   # persistent chunks
                                        (8, 2048, 2048)])    # Q8_0: the activation quantised to Q8_0 blocks
def test_matvec_fused_silu_mul(env, wtype, n, k):
    import oracle as O

    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(k)
    W, mm = _weight(A, S, wtype, n, k, ctx, seed=k)
    gu = (2 * rng.standard_normal(2 * k)).astype(np.float32)
    dgu = _dev(torch, gu)
    y = torch.empty(n, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_qmatmul_silu_mul_f32_device(ctx.handle, mm.handle, dgu.data_ptr(), k, y.data_ptr()))
    ctx.synchronize()
    g, u = gu[:k], gu[k:]
    xin = ((g / (np.float32(1) + np.exp(-g))) * u).astype(np.float32)[None, :]
    r = O.matmul(wtype, xin, W.blocks, n, k)[0]
    assert _rel(y.cpu().numpy(), r) <= 1e-3
    mm.free()


def _unpair(y, ffn):
    p = np.asarray(y).reshape(-1, ffn // 4, 2, 4)
    return p[:, :, 0, :].reshape(-1, ffn), p[:, :, 1, :].reshape(-1, ffn)


def test_swiglu_pairs(env):
    """silu(g) * u of rows of a paired gate|up output (column 8b + j: gate 4b + j
    for j < 4, up four on), rows at a stride wider than the row: the same
    values as aq_llama_silu_mul_rows on the split halves, bit for bit, and
    candle's formula within f32 rounding."""
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(3)
    m, ffn, ld = 3, 5632, 2 * 5632 + 8
    y = (4 * rng.standard_normal((m, ld))).astype(np.float32)
    y[0, 0], y[1, 9] = -100.0, 100.0  # exp overflow / underflow ends (gate entries)
    dy = _dev(torch, y)
    out = torch.empty((m, ffn), dtype=torch.float32, device="cuda:0")
    lib.check(L.aq_llama_swiglu_pairs(ctx.handle, dy.data_ptr(), ld, m, ffn, out.data_ptr()))
    g, u = _unpair(y[:, :2 * ffn], ffn)
    dg, du = _dev(torch, g), _dev(torch, u)
    o2 = torch.empty((m, ffn), dtype=torch.float32, device="cuda:0")
    lib.check(L.aq_llama_silu_mul_rows(ctx.handle, dg.data_ptr(), du.data_ptr(), ffn, m, ffn, o2.data_ptr()))
    ctx.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got, o2.cpu().numpy())
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    assert np.all(np.isfinite(got))
    assert _rel(got, g64 / (1 + np.exp(-g64)) * u64) <= 1e-5
    assert L.aq_llama_swiglu_pairs(ctx.handle, dy.data_ptr(), ld, m, 5630, out.data_ptr()) == lib.AQ_ERR_SHAPE


@pytest.mark.parametrize("wtype,n,k", [
    (12, 11264, 2048),   # TinyLlama w1|w3: 56-row workgroups
    (12, 28672, 4096),   # Llama-3-8B w1|w3: 56-row workgroups, 16 wavefronts
    (14, 11264, 2048),   # Q6_K, 56 rows
    (12, 1024, 4096),    # the 16-row form
    (14, 1600, 2048),    # the 8-row form
    (8, 2048, 2048),     # Q8_0 (8-row form, Q8_0-block activation)
    (12, 200, 1024),     # below 256 rows: the general fused-norm matmul, then the pairs
])
def test_matvec_fused_rmsnorm_swiglu(env, wtype, n, k):
    """The fused-norm matvec of a paired gate|up weight writing silu(g) * u:
    bit for bit the fused-norm matvec of the same weight followed by
    aq_llama_swiglu_pairs, the residual written as there, and within the
    oracle's tolerance of silu(g) * u of the oracle's matmul."""
    import oracle as O

    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(n + k)
    W, mm = _weight(A, S, wtype, n, k, ctx, seed=n)
    x = rng.standard_normal(k).astype(np.float32)
    d = rng.standard_normal(k).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    dx, dd, dw = _dev(torch, x), _dev(torch, d), _dev(torch, wn)
    eps = ctypes.c_float(1e-5)
    ffn = n // 2
    h1 = torch.empty(ffn, dtype=torch.float32, device="cuda:0")
    xo1 = torch.empty(k, dtype=torch.float32, device="cuda:0")
    y = torch.empty(n, dtype=torch.float32, device="cuda:0")
    h2 = torch.empty(ffn, dtype=torch.float32, device="cuda:0")
    xo2 = torch.empty(k, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    for _ in range(2):  # twice: the second call finds its scratch grown
        lib.check(L.aq_qmatmul_rmsnorm_swiglu_f32_device(ctx.handle, mm.handle, dx.data_ptr(), dd.data_ptr(),
                                                         dw.data_ptr(), eps, k, xo1.data_ptr(), h1.data_ptr()))
    lib.check(L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, mm.handle, dx.data_ptr(), dd.data_ptr(), dw.data_ptr(), eps,
                                              k, xo2.data_ptr(), y.data_ptr()))
    lib.check(L.aq_llama_swiglu_pairs(ctx.handle, y.data_ptr(), n, 1, ffn, h2.data_ptr()))
    ctx.synchronize()
    got = h1.cpu().numpy()
    assert np.array_equal(got, h2.cpu().numpy())
    assert np.array_equal(xo1.cpu().numpy(), xo2.cpu().numpy())
    assert np.array_equal(xo1.cpu().numpy(), x + d)
    h = x + d
    ms = np.float32(np.mean(h.astype(np.float64) ** 2))
    xin = ((h / np.sqrt(ms + np.float32(1e-5))) * wn).astype(np.float32)[None, :]
    g, u = _unpair(O.matmul(wtype, xin, W.blocks, n, k), ffn)
    want = (g / (np.float32(1) + np.exp(-g))) * u
    # the norm's sum of squares is reduced in another order, which can move a
    # Q8_K quant by one step: compare at 1e-3 of the output's scale
    assert _rel(got, want[0]) <= 1e-3
    mm.free()


@pytest.mark.parametrize("wtype,vocab,k,tie,alias", [
    (14, 32000, 2048, False, True),   # TinyLlama's head: persistent 56-row chunks; the next x over the input
    (14, 32000, 2048, True, False),   # the largest logit in two rows of different workgroups
    (12, 4000, 2048, True, False),    # the 16-row form
    (8, 2048, 2048, False, False),    # Q8_0, the 8-row form
    (12, 200, 1024, False, True),     # below 256 rows: the general matvec, then argmax and embedding launches
    (8, 49152, 576, True, False),     # SmolLM-135M's tied head (Q8_0, rows of 576): first maxima of 96 ranges
    (6, 3000, 576, False, True),      # a Q5_0 head on the general matvec
])
def test_head_argmax_embed(env, wtype, vocab, k, tie, alias):
    """aq_llama_head_argmax_embed against its three steps run apart (the
    fused-norm head, aq_llama_argmax over the logits, aq_llama_embed of the
    token): the same logits bit for bit, the same token (the first row of the
    largest logit, also when two workgroups hold it), history, position and
    embedding row."""
    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(vocab + k)
    W = S.make_weight(wtype, vocab, k, seed=vocab)
    x = rng.standard_normal(k).astype(np.float32)
    d = rng.standard_normal(k).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    table = rng.standard_normal((vocab, k)).astype(np.float32)
    dx, dd, dw, dt = _dev(torch, x), _dev(torch, d), _dev(torch, wn), _dev(torch, table)
    eps = ctypes.c_float(1e-5)
    pos0, hist_len = 37, 64

    def separate(mm):
        logits = torch.empty(vocab, dtype=torch.float32, device="cuda:0")
        tok = torch.zeros(1, dtype=torch.int64, device="cuda:0")
        pos = torch.full((1,), pos0, dtype=torch.int64, device="cuda:0")
        hist = torch.zeros(hist_len, dtype=torch.int64, device="cuda:0")
        xn = torch.empty(k, dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        lib.check(L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, mm.handle, dx.data_ptr(), dd.data_ptr(), dw.data_ptr(),
                                                  eps, k, None, logits.data_ptr()))
        lib.check(L.aq_llama_argmax(ctx.handle, logits.data_ptr(), vocab, tok.data_ptr(), pos.data_ptr(),
                                    hist.data_ptr(), hist_len))
        lib.check(L.aq_llama_embed(ctx.handle, dt.data_ptr(), vocab, tok.data_ptr(), k, xn.data_ptr()))
        ctx.synchronize()
        return [t.cpu().numpy() for t in (logits, tok, pos, hist, xn)]

    mm = A.QMatMul.from_qtensor(A.QTensor(wtype, (vocab, k), W.blocks), ctx)
    want = separate(mm)
    expect = int(np.argmax(want[0]))
    if tie:  # copy the winning row to an earlier row of another workgroup: it must win
        m = expect
        r2 = m - 150 if m >= 150 else m + 150
        rows = np.asarray(W.blocks).reshape(vocab, -1).copy()
        rows[r2] = rows[m]
        mm.free()
        mm = A.QMatMul.from_qtensor(A.QTensor(wtype, (vocab, k), rows.reshape(-1)), ctx)
        want = separate(mm)
        expect = min(m, r2)
        assert want[0][r2] == want[0][m]
    assert int(want[1][0]) == expect
    logits = torch.empty(vocab, dtype=torch.float32, device="cuda:0")
    tok = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    pos = torch.full((1,), pos0, dtype=torch.int64, device="cuda:0")
    hist = torch.zeros(hist_len, dtype=torch.int64, device="cuda:0")
    dx2 = _dev(torch, x)
    xn = dx2 if alias else torch.empty(k, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_head_argmax_embed(ctx.handle, mm.handle, dx2.data_ptr(), dd.data_ptr(), dw.data_ptr(), eps, k,
                                           logits.data_ptr(), tok.data_ptr(), pos.data_ptr(), hist.data_ptr(),
                                           hist_len, dt.data_ptr(), k, xn.data_ptr()))
    ctx.synchronize()
    got = [t.cpu().numpy() for t in (logits, tok, pos, hist, xn)]
    assert np.array_equal(got[0], want[0])
    assert int(got[1][0]) == expect and int(got[2][0]) == pos0 + 1 and int(got[3][pos0]) == expect
    assert np.array_equal(got[3], want[3])
    assert np.array_equal(got[4], table[expect])
    mm.free()


def test_matvec_fused_errors(env):
    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    W, mm = _weight(A, S, 12, 64, 16384, ctx, seed=1)
    buf = torch.zeros(2 * 16384, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    p = buf.data_ptr()
    # too long a row for the fused norm: a clean AQ_ERR_SHAPE, nothing launched
    assert L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, mm.handle, p, None, p, ctypes.c_float(1e-5), 16384, None,
                                           p) == lib.AQ_ERR_SHAPE
    # wrong k, aliased residual output
    assert L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, mm.handle, p, None, p, ctypes.c_float(1e-5), 8192, None,
                                           p) == lib.AQ_ERR_SHAPE
    assert L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, mm.handle, p, None, p, ctypes.c_float(1e-5), 16384, p,
                                           p) == lib.AQ_ERR_INVALID_ARG
    mm.free()


@pytest.mark.parametrize("t1,n1,t2,n2,k", [
    (12, 2304, 14, 256, 2048),   # TinyLlama wq|wk + wv: both row-per-lane, one launch
    (12, 1000, 12, 300, 4096),
    (14, 5120, 14, 1024, 8192),  # eight wavefronts per workgroup
    (14, 512, 14, 96, 1024),     # the second below 256 rows: one launch each
    (12, 12000, 14, 256, 2048),  # the first in 56-row workgroups: one launch each
    (12, 2048, 14, 1536, 2048),  # both in 8-row workgroups: one launch
    (12, 2048, 12, 512, 4096),   # 8-row and 16-row forms: one launch each
    (12, 200, 14, 96, 1024),     # neither row-per-lane: the general two-weight kernel
    (6, 768, 8, 192, 576),       # SmolLM-135M wq|wk (Q5_0) + wv (Q8_0), rows of 576: the general kernel, one launch
    (6, 300, 6, 100, 576),       # two Q5_0 weights
    (8, 200, 8, 64, 1024),       # two Q8_0 weights below 256 rows
    (12, 2048, 8, 256, 2048),    # Q4_K with Q8_0: one launch each
])
def test_matvec2_fused_rmsnorm_equals_two_calls(env, t1, n1, t2, n2, k):
    """The two-weight call gives the bytes the two single calls give."""
    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(n1 + n2)
    _, m1 = _weight(A, S, t1, n1, k, ctx, seed=n1)
    _, m2 = _weight(A, S, t2, n2, k, ctx, seed=n2 + 1)
    x, d = _dev(torch, rng.standard_normal(k).astype(np.float32)), _dev(torch, rng.standard_normal(k).astype(np.float32))
    wn = _dev(torch, (1 + 0.05 * rng.standard_normal(k)).astype(np.float32))
    outs = [torch.full((n,), np.nan, dtype=torch.float32, device="cuda:0") for n in (n1, n2, n1, n2)]
    h1 = torch.full((k,), np.nan, dtype=torch.float32, device="cuda:0")
    h2 = torch.full((k,), np.nan, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    eps = ctypes.c_float(1e-5)
    lib.check(L.aq_qmatmul2_rmsnorm_f32_device(ctx.handle, m1.handle, m2.handle, x.data_ptr(), d.data_ptr(),
                                               wn.data_ptr(), eps, k, h1.data_ptr(), outs[0].data_ptr(),
                                               outs[1].data_ptr()))
    lib.check(L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, m1.handle, x.data_ptr(), d.data_ptr(), wn.data_ptr(), eps,
                                              k, h2.data_ptr(), outs[2].data_ptr()))
    lib.check(L.aq_qmatmul_rmsnorm_f32_device(ctx.handle, m2.handle, x.data_ptr(), d.data_ptr(), wn.data_ptr(), eps,
                                              k, None, outs[3].data_ptr()))
    ctx.synchronize()
    o = [t.cpu().numpy() for t in outs]
    assert np.array_equal(o[0], o[2]) and np.array_equal(o[1], o[3])
    assert np.array_equal(h1.cpu().numpy(), h2.cpu().numpy())
    # a k the weights do not have
    assert L.aq_qmatmul2_rmsnorm_f32_device(ctx.handle, m1.handle, m2.handle, x.data_ptr(), None, wn.data_ptr(), eps,
                                            k + 32, None, outs[0].data_ptr(), outs[1].data_ptr()) == lib.AQ_ERR_SHAPE
    for mm in (m1, m2):
        mm.free()


# ---------------------------------------------------------------- prompt glue quantised in the same launch
def _act(torch, lib, m, k):
    L = lib.load()
    return torch.zeros(int(L.aq_act_bytes(15, m, k)), dtype=torch.uint8, device="cuda:0")  # AQ_TYPE_Q8_K


def _planes(buf):
    """The activation buffer's bytes (all of its planes)."""
    return buf.cpu().numpy()


@pytest.mark.parametrize("m,n,with_delta", [(1, 256, False), (3, 2048, True), (512, 2048, True), (5, 4096, False),
                                            (2, 8192, True)])
def test_rmsnorm_act_equals_rmsnorm_then_quantize(env, m, n, with_delta):
    """aq_llama_rmsnorm_act: the residual add, the normed values and every
    quantised plane (qs, d, bsums, their f16 forms, the f16 quants) bit for bit
    as aq_llama_rmsnorm followed by aq_quantize_act_device."""
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(m + n)
    x = (2 * rng.standard_normal((m, n))).astype(np.float32)
    d = rng.standard_normal((m, n)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    x[0, 5] = 0.0
    dx1, dx2, dd, dw = _dev(torch, x), _dev(torch, x), _dev(torch, d), _dev(torch, w)
    h1 = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    h2 = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    a1, a2 = _act(torch, lib, m, n), _act(torch, lib, m, n)
    torch.cuda.synchronize()
    delta = dd.data_ptr() if with_delta else None
    eps = ctypes.c_float(1e-5)
    lib.check(L.aq_llama_rmsnorm(ctx.handle, dx1.data_ptr(), delta, dw.data_ptr(), m, n, eps, h1.data_ptr()))
    lib.check(L.aq_quantize_act_device(ctx.handle, 15, h1.data_ptr(), m, n, a1.data_ptr()))
    lib.check(L.aq_llama_rmsnorm_act(ctx.handle, dx2.data_ptr(), delta, dw.data_ptr(), m, n, eps, h2.data_ptr(),
                                     a2.data_ptr()))
    ctx.synchronize()
    assert np.array_equal(dx1.cpu().numpy(), dx2.cpu().numpy())
    assert np.array_equal(h1.cpu().numpy(), h2.cpu().numpy())
    assert np.array_equal(_planes(a1), _planes(a2))
    # without the f32 copy: the same planes
    a3 = _act(torch, lib, m, n)
    dx3 = _dev(torch, x)
    torch.cuda.synchronize()
    lib.check(L.aq_llama_rmsnorm_act(ctx.handle, dx3.data_ptr(), delta, dw.data_ptr(), m, n, eps, None,
                                     a3.data_ptr()))
    ctx.synchronize()
    assert np.array_equal(_planes(a1), _planes(a3))


@pytest.mark.parametrize("m,ffn,pad", [(1, 256, 0), (7, 5632, 0), (64, 5632, 8), (3, 14336, 0)])
def test_swiglu_pairs_act_equals_swiglu_pairs_then_quantize(env, m, ffn, pad):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(ffn + m)
    ld = 2 * ffn + pad
    y = (3 * rng.standard_normal((m, ld))).astype(np.float32)
    y[0, 0], y[0, 1] = -100.0, 100.0  # exp overflow / underflow ends of silu
    dy = _dev(torch, y)
    o1 = torch.empty((m, ffn), dtype=torch.float32, device="cuda:0")
    o2 = torch.empty((m, ffn), dtype=torch.float32, device="cuda:0")
    a1, a2 = _act(torch, lib, m, ffn), _act(torch, lib, m, ffn)
    torch.cuda.synchronize()
    lib.check(L.aq_llama_swiglu_pairs(ctx.handle, dy.data_ptr(), ld, m, ffn, o1.data_ptr()))
    lib.check(L.aq_quantize_act_device(ctx.handle, 15, o1.data_ptr(), m, ffn, a1.data_ptr()))
    lib.check(L.aq_llama_swiglu_pairs_act(ctx.handle, dy.data_ptr(), ld, m, ffn, o2.data_ptr(), a2.data_ptr()))
    ctx.synchronize()
    assert np.array_equal(o1.cpu().numpy(), o2.cpu().numpy())
    assert np.array_equal(_planes(a1), _planes(a2))


@pytest.mark.parametrize("wtype,n,k,m", [(14, 256, 2048, 512), (14, 2048, 5632, 64), (13, 512, 2048, 33),
                                         (12, 2304, 2048, 96)])
def test_prequantised_gemm_reads_the_planes_f16_quants(env, wtype, n, k, m):
    """aq_qmatmul_preq_device on planes from the fused prompt glue: the f16
    MFMA GEMMs (Q6_K, Q5_K) read the activation's own f16 quants; the result
    equals the f32-input call, which quantises first."""
    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    W = S.make_weight(wtype, n, k, seed=n + k)
    mm = A.QMatMul.from_qtensor(A.QTensor(wtype, (n, k), W.blocks), ctx)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wn = np.ones(k, np.float32)
    dx, dwn = _dev(torch, x), _dev(torch, wn)
    h = torch.empty((m, k), dtype=torch.float32, device="cuda:0")
    act = _act(torch, lib, m, k)
    y1 = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    y2 = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_rmsnorm_act(ctx.handle, dx.data_ptr(), None, dwn.data_ptr(), m, k, ctypes.c_float(1e-5),
                                     h.data_ptr(), act.data_ptr()))
    lib.check(L.aq_qmatmul_preq_device(ctx.handle, mm.handle, act.data_ptr(), m, k, y1.data_ptr()))
    lib.check(L.aq_qmatmul_f32_device(ctx.handle, mm.handle, h.data_ptr(), m, k, y2.data_ptr()))
    ctx.synchronize()
    assert np.array_equal(y1.cpu().numpy(), y2.cpu().numpy())
    mm.free()


@pytest.mark.parametrize("t1,t2,n1,n2,k,m", [
    (12, 14, 2304, 256, 2048, 512),   # TinyLlama wq|wk and wv, a 512-token prompt: one launch
    (12, 14, 2304, 256, 2048, 100),   # ragged m-tiles
    (12, 13, 2304, 256, 2048, 33),    # a Q5_K wv
    (12, 14, 5120, 1024, 4096, 64),   # Llama-3-8B heads
    (12, 14, 2304, 256, 2048, 5),     # batch rows: two matrix-core matvec calls
    (12, 12, 2304, 256, 2048, 40),    # two Q4_K weights: two GEMM calls
])
def test_qmatmul2_preq_equals_two_calls(env, t1, t2, n1, n2, k, m):
    """aq_qmatmul2_preq_device against two aq_qmatmul_preq_device calls on
    the same planes: the paired launch runs the Q4_K GEMM unsplit, so only the
    f32 order of its split-K partials may differ (within 1e-6 of the largest
    output); the cases that make the two calls are bit-identical."""
    import arm_ai_amd as A
    from arm_ai_amd import synth as S

    torch, lib, ctx = env
    L = lib.load()
    W1 = S.make_weight(t1, n1, k, seed=n1 + k)
    W2 = S.make_weight(t2, n2, k, seed=n2 + k + 1)
    mm1 = A.QMatMul.from_qtensor(A.QTensor(t1, (n1, k), W1.blocks), ctx)
    mm2 = A.QMatMul.from_qtensor(A.QTensor(t2, (n2, k), W2.blocks), ctx)
    x = np.random.default_rng(m + k).standard_normal((m, k)).astype(np.float32)
    dx, dwn = _dev(torch, x), _dev(torch, np.ones(k, np.float32))
    act = _act(torch, lib, m, k)
    f32 = dict(dtype=torch.float32, device="cuda:0")
    y1, y2 = torch.empty((m, n1), **f32), torch.empty((m, n2), **f32)
    r1, r2 = torch.empty((m, n1), **f32), torch.empty((m, n2), **f32)
    torch.cuda.synchronize()
    lib.check(L.aq_llama_rmsnorm_act(ctx.handle, dx.data_ptr(), None, dwn.data_ptr(), m, k, ctypes.c_float(1e-5),
                                     None, act.data_ptr()))
    lib.check(L.aq_qmatmul2_preq_device(ctx.handle, mm1.handle, mm2.handle, act.data_ptr(), m, k, y1.data_ptr(),
                                        y2.data_ptr()))
    lib.check(L.aq_qmatmul_preq_device(ctx.handle, mm1.handle, act.data_ptr(), m, k, r1.data_ptr()))
    lib.check(L.aq_qmatmul_preq_device(ctx.handle, mm2.handle, act.data_ptr(), m, k, r2.data_ptr()))
    ctx.synchronize()
    paired = m > 8 and t1 == 12 and t2 in (13, 14)
    for got, want in ((y1, r1), (y2, r2)):
        got, want = got.cpu().numpy(), want.cpu().numpy()
        assert np.all(np.isfinite(got))
        if paired:
            assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))
        else:
            assert np.array_equal(got, want)
    assert L.aq_qmatmul2_preq_device(ctx.handle, mm1.handle, mm2.handle, act.data_ptr(), m, k + 256, y1.data_ptr(),
                                     y2.data_ptr()) == lib.AQ_ERR_SHAPE
    mm1.free()
    mm2.free()


def test_prompt_glue_act_errors(env):
    torch, lib, ctx = env
    L = lib.load()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda:0")
    f = torch.zeros(4096, dtype=torch.float32, device="cuda:0")
    p, a = f.data_ptr(), buf.data_ptr()
    eps = ctypes.c_float(1e-5)
    assert L.aq_llama_rmsnorm_act(ctx.handle, p, None, p, 2, 576, eps, None, a) == lib.AQ_ERR_SHAPE  # not whole blocks
    assert L.aq_llama_rmsnorm_act(ctx.handle, p, None, p, 2, 256, eps, None, a + 16) == lib.AQ_ERR_INVALID_ARG
    assert L.aq_llama_rmsnorm_act(ctx.handle, p, None, p, 2, 256, eps, None, None) == lib.AQ_ERR_INVALID_ARG
    assert L.aq_llama_rmsnorm_act(ctx.handle, p, None, p, 1, 16384, eps, None, a) == lib.AQ_ERR_SHAPE  # over 8192
    assert L.aq_llama_swiglu_pairs_act(ctx.handle, p, 1280, 2, 640, None, a) == lib.AQ_ERR_SHAPE  # not whole blocks
    assert L.aq_llama_swiglu_pairs_act(ctx.handle, p, 256, 2, 256, None, a) == lib.AQ_ERR_SHAPE  # ld < 2 * ffn
    assert L.aq_llama_swiglu_pairs_act(ctx.handle, p, 514, 2, 256, None, a) == lib.AQ_ERR_INVALID_ARG  # ld % 4
    assert L.aq_llama_swiglu_pairs_act(ctx.handle, p + 4, 512, 2, 256, None, a) == lib.AQ_ERR_INVALID_ARG  # y align
    assert L.aq_llama_rmsnorm_act(ctx.handle, p, None, p, 0, 256, eps, None, a) == lib.AQ_OK
    ctx.synchronize()
