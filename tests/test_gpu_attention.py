"""GPU tests of the attention kernels (k_attn.hip) and the prompt's row-wise
glue through the C ABI, against numpy restatements of candle-transformers
quantized_llama's attention (rope_i, KV cache append, grouped-query heads,
softmax(q.k/sqrt(hd)) with the causal mask, . v) in float64.  f32 sums are
reordered on the GPU: values at 1e-5 relative to the largest output; cache
writes are exact (the rotation is written without FMA contraction, as numpy
computes it in f32).

Decode: the split-context kernels (head_dim 64 / 128, 1..8 query heads per kv
head; a partial record per slice, then a combining launch) at positions on
and around the slice boundaries, up to the longest context, called back to
back on one context (the partial records are reused by every call).
Prefill: prompts at offset 0 and later, lengths that are not a multiple of
the 32-row query tile, q / k / v read with row strides from one merged
buffer."""
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
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    torch.cuda.synchronize()
    return t


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _rope(x, c, s):
    """rope_i in f32, as numpy evaluates a*c - b*s (no FMA)."""
    out = np.empty_like(x)
    a, b = x[..., 0::2], x[..., 1::2]
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


def _tables(hd, max_seq):
    theta = 1.0 / (10000.0 ** (np.arange(0, hd, 2, dtype=np.float32) / hd))
    ang = np.arange(max_seq, dtype=np.float32)[:, None] * theta[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _attend(q, kc, vc, upto, rep):
    """q [n_head, hd] f32; caches [n_kv, max_seq, hd]; positions 0..upto."""
    n_head, hd = q.shape
    out = np.empty((n_head, hd))
    for h in range(n_head):
        kk = kc[h // rep, :upto + 1].astype(np.float64)
        s = kk @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ vc[h // rep, :upto + 1].astype(np.float64)
    return out


def _decode_call(torch, lib, ctx, n_head, n_kv, hd, max_seq, kc, vc, qk, v, pos, dcos, dsin):
    L = lib.load()
    dqk, dv = _dev(torch, qk), _dev(torch, v)
    dpos = torch.tensor([pos], dtype=torch.int64, device="cuda:0")
    out = torch.empty(n_head * hd, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_attn_decode(ctx.handle, dqk.data_ptr(), dv.data_ptr(), dcos.data_ptr(), dsin.data_ptr(),
                                     dpos.data_ptr(), kc.data_ptr(), vc.data_ptr(), n_head, n_kv, hd, max_seq,
                                     out.data_ptr()))
    ctx.synchronize()
    return out.cpu().numpy().reshape(n_head, hd)


@pytest.mark.parametrize(
    "n_head,n_kv,hd,max_seq,positions",
    [
        # TinyLlama heads: slices of at least 16 positions, 64 slices of 4 kv heads
        (32, 4, 64, 1024, [0, 1, 31, 32, 33, 63, 64, 600, 1023]),
        # max_seq not a multiple of 16: 38 slices can hold positions, the last from 592
        (32, 4, 64, 600, [0, 15, 16, 591, 592, 599]),
        (32, 4, 64, 8192, [8191, 2048, 2049, 4097]),  # slices longer than 16 (8192 / 64 = 128 per slice)
        (32, 8, 128, 2048, [0, 63, 64, 511, 512, 2047]),  # Llama-3-8B heads: 4 per kv head, 32 slices
        (8, 4, 64, 512, [0, 100, 511]),  # 2 per kv head
        (8, 8, 128, 512, [0, 5, 300]),   # one query head per kv head
        (64, 8, 128, 256, [0, 255]),     # 8 per kv head at head_dim 128
        (9, 3, 64, 640, [0, 15, 16, 511, 512, 639]),  # SmolLM-135M heads: 3 per kv head, 85 slices
        (15, 5, 64, 300, [0, 17, 299]),  # 3 per kv head, five kv heads
    ],
)
def test_split_decode_against_numpy_back_to_back(env, n_head, n_kv, hd, max_seq, positions):
    """Several calls on one context in a row, each checked: a record left
    over from a longer context must not enter a shorter one's combine."""
    torch, lib, ctx = env
    rng = np.random.default_rng(n_head * hd + max_seq)
    kc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    cos, sin = _tables(hd, max_seq)
    dkc, dvc, dcos, dsin = _dev(torch, kc), _dev(torch, vc), _dev(torch, cos), _dev(torch, sin)
    rep = n_head // n_kv
    for pos in positions:
        qk = (2 * rng.standard_normal((n_head + n_kv) * hd)).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        got = _decode_call(torch, lib, ctx, n_head, n_kv, hd, max_seq, dkc, dvc, qk, v, pos, dcos, dsin)
        q = _rope(qk[:n_head * hd].reshape(n_head, hd), cos[pos], sin[pos])
        k = _rope(qk[n_head * hd:].reshape(n_kv, hd), cos[pos], sin[pos])
        kc[:, pos], vc[:, pos] = k, v.reshape(n_kv, hd)
        assert _rel(got, _attend(q, kc, vc, pos, rep)) <= 1e-5, f"pos {pos}"
        assert np.array_equal(dkc.cpu().numpy(), kc), f"pos {pos}: k cache"
        assert np.array_equal(dvc.cpu().numpy(), vc), f"pos {pos}: v cache"


def test_split_decode_sharp_softmax(env):
    """Scores 60 apart between slices: the combine's rescaling by e^(m_s - M)
    must take the slice maxima into account (a plain sum of the slices' e^(s -
    m_s) would weight every slice alike)."""
    torch, lib, ctx = env
    n_head, n_kv, hd, max_seq, pos = 32, 4, 64, 1024, 700
    rng = np.random.default_rng(9)
    kc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    kc[:, 333] *= 20.0  # one key far above the others
    cos, sin = _tables(hd, max_seq)
    dkc, dvc, dcos, dsin = _dev(torch, kc), _dev(torch, vc), _dev(torch, cos), _dev(torch, sin)
    qk = rng.standard_normal((n_head + n_kv) * hd).astype(np.float32)
    qk[:n_head * hd] *= 3.0
    v = rng.standard_normal(n_kv * hd).astype(np.float32)
    got = _decode_call(torch, lib, ctx, n_head, n_kv, hd, max_seq, dkc, dvc, qk, v, pos, dcos, dsin)
    q = _rope(qk[:n_head * hd].reshape(n_head, hd), cos[pos], sin[pos])
    kc[:, pos] = _rope(qk[n_head * hd:].reshape(n_kv, hd), cos[pos], sin[pos])
    vc[:, pos] = v.reshape(n_kv, hd)
    assert _rel(got, _attend(q, kc, vc, pos, n_head // n_kv)) <= 1e-5


def _prefill_ref(q, k, v, kc, vc, cos, sin, index_pos, n_head, n_kv, hd):
    """Returns (out [m, n_head*hd], kc, vc after the append)."""
    m = q.shape[0]
    rep = n_head // n_kv
    kc, vc = kc.copy(), vc.copy()
    P = np.arange(index_pos, index_pos + m)
    qr = _rope(q.reshape(m, n_head, hd), cos[P][:, None, :], sin[P][:, None, :])
    kr = _rope(k.reshape(m, n_kv, hd), cos[P][:, None, :], sin[P][:, None, :])
    kc[:, P] = kr.transpose(1, 0, 2)
    vc[:, P] = v.reshape(m, n_kv, hd).transpose(1, 0, 2)
    out = np.empty((m, n_head, hd))
    for r in range(m):
        out[r] = _attend(qr[r], kc, vc, index_pos + r, rep)
    return out.reshape(m, n_head * hd), kc, vc


@pytest.mark.parametrize(
    "n_head,n_kv,hd,index_pos,m,max_seq",
    [(4, 2, 64, 0, 7, 64), (32, 4, 64, 0, 512, 640), (32, 4, 64, 0, 100, 128), (8, 8, 128, 5, 70, 128),
     (32, 8, 128, 0, 65, 128), (32, 4, 64, 200, 1, 256), (16, 2, 64, 37, 130, 256),
     (9, 3, 64, 0, 512, 640), (9, 3, 64, 512, 3, 640)],  # SmolLM-135M heads: 3 per kv head
)
def test_prefill_against_numpy(env, n_head, n_kv, hd, index_pos, m, max_seq):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(m + index_pos + hd)
    width = (n_head + n_kv) * hd
    qk = rng.standard_normal((m, width)).astype(np.float32)  # the merged wq|wk output: strided q and k
    v = rng.standard_normal((m, n_kv * hd)).astype(np.float32)
    kc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((n_kv, max_seq, hd)).astype(np.float32)
    cos, sin = _tables(hd, max_seq)
    dqk, dv, dkc, dvc = _dev(torch, qk), _dev(torch, v), _dev(torch, kc), _dev(torch, vc)
    dcos, dsin = _dev(torch, cos), _dev(torch, sin)
    out = torch.empty((m, n_head * hd), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_attn_prefill(ctx.handle, dqk.data_ptr(), width, dqk.data_ptr() + 4 * n_head * hd, width,
                                      dv.data_ptr(), n_kv * hd, dcos.data_ptr(), dsin.data_ptr(), index_pos, m,
                                      dkc.data_ptr(), dvc.data_ptr(), n_head, n_kv, hd, max_seq, out.data_ptr()))
    ctx.synchronize()
    want, kc2, vc2 = _prefill_ref(qk[:, :n_head * hd], qk[:, n_head * hd:], v, kc, vc, cos, sin, index_pos, n_head,
                                  n_kv, hd)
    assert _rel(out.cpu().numpy(), want) <= 1e-5
    assert np.array_equal(dkc.cpu().numpy(), kc2)
    assert np.array_equal(dvc.cpu().numpy(), vc2)


def test_prefill_sharp_softmax(env):
    """One key row twenty times the others and queries three times larger:
    scores far apart across the key blocks of the four wavefronts, so the
    running maxima (base-2 units) and the combine's rescaling decide the
    result."""
    torch, lib, ctx = env
    L = lib.load()
    n_head, n_kv, hd, m, max_seq = 32, 4, 64, 300, 320
    rng = np.random.default_rng(21)
    width = (n_head + n_kv) * hd
    qk = rng.standard_normal((m, width)).astype(np.float32)
    qk[:, :n_head * hd] *= 3.0
    qk[57, n_head * hd:] *= 20.0  # key 57 far above the others for every later query
    v = rng.standard_normal((m, n_kv * hd)).astype(np.float32)
    kc = np.zeros((n_kv, max_seq, hd), np.float32)
    vc = np.zeros((n_kv, max_seq, hd), np.float32)
    cos, sin = _tables(hd, max_seq)
    dqk, dv, dkc, dvc = _dev(torch, qk), _dev(torch, v), _dev(torch, kc), _dev(torch, vc)
    dcos, dsin = _dev(torch, cos), _dev(torch, sin)
    out = torch.empty((m, n_head * hd), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_attn_prefill(ctx.handle, dqk.data_ptr(), width, dqk.data_ptr() + 4 * n_head * hd, width,
                                      dv.data_ptr(), n_kv * hd, dcos.data_ptr(), dsin.data_ptr(), 0, m,
                                      dkc.data_ptr(), dvc.data_ptr(), n_head, n_kv, hd, max_seq, out.data_ptr()))
    ctx.synchronize()
    want, _, _ = _prefill_ref(qk[:, :n_head * hd], qk[:, n_head * hd:], v, kc, vc, cos, sin, 0, n_head, n_kv, hd)
    assert _rel(out.cpu().numpy(), want) <= 1e-5


def test_prefill_then_decode_continue_the_same_cache(env):
    """A prompt through the prefill kernel, then decode steps at the next
    positions read the cache it wrote (the layout both kernels share)."""
    torch, lib, ctx = env
    L = lib.load()
    n_head, n_kv, hd, max_seq, m = 32, 4, 64, 256, 40
    rng = np.random.default_rng(77)
    q = rng.standard_normal((m, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((m, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((m, n_kv * hd)).astype(np.float32)
    kc = np.zeros((n_kv, max_seq, hd), np.float32)
    vc = np.zeros((n_kv, max_seq, hd), np.float32)
    cos, sin = _tables(hd, max_seq)
    dq, dk, dv = _dev(torch, q), _dev(torch, k), _dev(torch, v)
    dkc, dvc, dcos, dsin = _dev(torch, kc), _dev(torch, vc), _dev(torch, cos), _dev(torch, sin)
    out = torch.empty((m, n_head * hd), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_attn_prefill(ctx.handle, dq.data_ptr(), n_head * hd, dk.data_ptr(), n_kv * hd, dv.data_ptr(),
                                      n_kv * hd, dcos.data_ptr(), dsin.data_ptr(), 0, m, dkc.data_ptr(),
                                      dvc.data_ptr(), n_head, n_kv, hd, max_seq, out.data_ptr()))
    ctx.synchronize()
    _, kc, vc = _prefill_ref(q, k, v, kc, vc, cos, sin, 0, n_head, n_kv, hd)
    for pos in range(m, m + 3):
        qk = rng.standard_normal((n_head + n_kv) * hd).astype(np.float32)
        vv = rng.standard_normal(n_kv * hd).astype(np.float32)
        got = _decode_call(torch, lib, ctx, n_head, n_kv, hd, max_seq, dkc, dvc, qk, vv, pos, dcos, dsin)
        qr = _rope(qk[:n_head * hd].reshape(n_head, hd), cos[pos], sin[pos])
        kc[:, pos] = _rope(qk[n_head * hd:].reshape(n_kv, hd), cos[pos], sin[pos])
        vc[:, pos] = vv.reshape(n_kv, hd)
        assert _rel(got, _attend(qr, kc, vc, pos, n_head // n_kv)) <= 1e-5


def test_prefill_argument_errors(env):
    torch, lib, ctx = env
    L = lib.load()
    buf = torch.zeros(1 << 16, dtype=torch.float32, device="cuda:0")
    p = buf.data_ptr()
    ok = dict(ldq=256, ldk=128, ldv=128, index_pos=0, m=4, n_head=4, n_kv=2, hd=64, max_seq=64)

    def call(**kw):
        a = {**ok, **kw}
        return L.aq_llama_attn_prefill(ctx.handle, p, a["ldq"], p, a["ldk"], p, a["ldv"], p, p, a["index_pos"], a["m"],
                                       p, p, a["n_head"], a["n_kv"], a["hd"], a["max_seq"], p)

    assert call(hd=32) != 0            # head_dim other than 64 / 128
    assert call(index_pos=62) != 0     # past the end of the cache
    assert call(n_kv=3) != 0           # n_head not a multiple of n_kv
    assert call(ldq=128) != 0          # q rows shorter than n_head * head_dim
    assert call(index_pos=-1) != 0
    assert call(m=0) == 0              # nothing to do


def test_embed_rows_and_silu_mul_rows(env):
    torch, lib, ctx = env
    L = lib.load()
    rng = np.random.default_rng(5)
    table = rng.standard_normal((100, 64)).astype(np.float32)
    toks = np.array([3, 99, 100, -5, 42, 3], np.int64)
    dt, dtok = _dev(torch, table), _dev(torch, toks)
    out = torch.empty((len(toks), 64), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_embed_rows(ctx.handle, dt.data_ptr(), 100, dtok.data_ptr(), len(toks), 64, out.data_ptr()))
    ctx.synchronize()
    want = np.stack([table[t] if 0 <= t < 100 else np.zeros(64, np.float32) for t in toks])
    assert np.array_equal(out.cpu().numpy(), want)

    m, n = 5, 700
    gu = (4 * rng.standard_normal((m, 2 * n))).astype(np.float32)
    gu[0, 0], gu[1, 1] = -100.0, 100.0
    dgu = _dev(torch, gu)
    o = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_silu_mul_rows(ctx.handle, dgu.data_ptr(), dgu.data_ptr() + 4 * n, 2 * n, m, n, o.data_ptr()))
    ctx.synchronize()
    g, u = gu[:, :n].astype(np.float64), gu[:, n:].astype(np.float64)
    got = o.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert _rel(got, g / (1 + np.exp(-g)) * u) <= 1e-5
    # separate g and u buffers (unmerged w1 / w3): ld = n
    dg, du = _dev(torch, gu[:, :n]), _dev(torch, gu[:, n:])
    o2 = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    lib.check(L.aq_llama_silu_mul_rows(ctx.handle, dg.data_ptr(), du.data_ptr(), n, m, n, o2.data_ptr()))
    ctx.synchronize()
    assert np.array_equal(o2.cpu().numpy(), got)
