"""The quantized matmuls' call sites (a Llama decoder driven like ArmAI.LlamaCandle).

GPU tests: the driver (arm_ai_amd.llama, quantized projections on the GPU
through the C ABI) against oracle/llama_ref.py (numpy glue + the oracle's
k_quants::matmul) on a small model, teacher-forced: prefill logits, decode
logits, the graph-captured decode step against the eager one, and greedy
generation.  Weights come from synth.make_weight_unit (values centred and
scaled by 1/sqrt(k), so activations stay of order one and nothing saturates
or overflows; RuntimeWarnings are errors).  Tolerance: the activation
quantisation is bit-exact, but the f32 glue (torch on the GPU vs numpy)
rounds differently and a Q8_K block whose input moved by one ulp can round a
quant the other way, so logits are compared at 1e-3 of their largest
magnitude.

CPU test: the reference restatement's rope_i pairing against its closed form.
"""
import numpy as np
import pytest

from oracle.llama_ref import RefLlama

LOGIT_TOL = 1e-3

pytestmark = pytest.mark.filterwarnings("error::RuntimeWarning")


def _tiny_cfg():
    from arm_ai_amd.llama import LlamaConfig

    return LlamaConfig(n_layer=2, hidden=256, ffn=512, n_head=4, n_kv_head=2, vocab=512, max_seq=64)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ---------------------------------------------------------------- CPU
def test_ref_rope_closed_form():
    from arm_ai_amd.llama import synthetic_weights

    cfg = _tiny_cfg()
    hw = synthetic_weights(cfg, seed=1, unit=True)
    ref = RefLlama(hw)
    hd = cfg.hidden // cfg.n_head
    # position 0 is the identity; a pair (1, 0) at position p becomes (cos, sin)(p * theta_i)
    x = np.zeros((3, 1, hd), np.float32)
    x[:, 0, 0::2] = 1.0
    out = ref.rope(x, 5)
    for L in range(3):
        for i in range(hd // 2):
            ang = (5 + L) * (cfg.rope_theta ** (-2.0 * i / hd))
            assert abs(out[L, 0, 2 * i] - np.cos(ang)) < 2e-5
            assert abs(out[L, 0, 2 * i + 1] - np.sin(ang)) < 2e-5
    assert np.array_equal(ref.rope(x, 0)[0], x[0])


# ---------------------------------------------------------------- GPU
@pytest.fixture(scope="module")
def tiny():
    import torch

    import arm_ai_amd as A

    if not torch.cuda.is_available():
        if A.device_count() > 0:
            pytest.fail("the library sees a GPU but torch does not (torch must be imported first)")
        pytest.skip("no GPU")
    from arm_ai_amd.llama import Llama, synthetic_weights

    cfg = _tiny_cfg()
    hw = synthetic_weights(cfg, seed=3, unit=True)
    ctx = A.Context(0)
    model = Llama(ctx, hw)
    yield hw, model
    model.free()
    ctx.close()


@pytest.mark.gpu
def test_prefill_and_decode_logits_match_reference(tiny):
    hw, model = tiny
    ref = RefLlama(hw)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, hw.cfg.vocab, size=7).tolist()
    g = model.forward(prompt, 0).cpu().numpy()
    r = ref.forward(prompt, 0)
    assert np.all(np.isfinite(g))
    assert _rel(g, r) <= LOGIT_TOL, f"prefill logits rel {_rel(g, r):.3e}"
    pos = len(prompt)
    for step in range(3):  # teacher-forced: both sides see the same tokens
        tok = int(rng.integers(0, hw.cfg.vocab))
        g = model.forward([tok], pos).cpu().numpy()
        r = ref.forward([tok], pos)
        assert _rel(g, r) <= LOGIT_TOL, f"decode step {step} logits rel {_rel(g, r):.3e}"
        pos += 1


@pytest.fixture(scope="module")
def tiny_q5km():
    """The same architecture with the Q5_K_M type mix (Q5_K projections; wv,
    half the w2 and the output head Q6_K): the decode step's one-weight
    fused-norm path, since the two-weight launch takes Q4_K / Q6_K only."""
    import torch

    import arm_ai_amd as A

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from arm_ai_amd.llama import Llama, synthetic_weights, tinyllama_q5km_types

    hw = synthetic_weights(_tiny_cfg(), seed=13, types=tinyllama_q5km_types, unit=True)
    ctx = A.Context(0)
    model = Llama(ctx, hw)
    yield hw, model
    model.free()
    ctx.close()


@pytest.mark.gpu
def test_q5km_logits_and_graph_step_match_reference(tiny_q5km):
    hw, model = tiny_q5km
    ref = RefLlama(hw)
    rng = np.random.default_rng(15)
    prompt = rng.integers(0, hw.cfg.vocab, size=9).tolist()
    g = model.forward(prompt, 0).cpu().numpy()
    r = ref.forward(prompt, 0)
    assert _rel(g, r) <= LOGIT_TOL, f"prefill logits rel {_rel(g, r):.3e}"
    pos = len(prompt)
    for step in range(2):  # teacher-forced decode
        tok = int(rng.integers(0, hw.cfg.vocab))
        g = model.forward([tok], pos).cpu().numpy()
        r = ref.forward([tok], pos)
        assert _rel(g, r) <= LOGIT_TOL, f"decode step {step} logits rel {_rel(g, r):.3e}"
        pos += 1
    toks_e = model.generate(prompt, 6, graph=False).tokens
    toks_g = model.generate(prompt, 6, graph=True).tokens
    assert toks_e == toks_g


def _low_bit_types(cfg, layer):
    """A Q3_K_M / Q2_K-style mix over the types with no fused two-weight
    launch: Q3_K attention and FFN projections, Q5_0 wv, Q2_K wo, and w2
    alternating Q2_K / Q5_0."""
    from arm_ai_amd import synth

    return {"wq": synth.TYPE_Q3_K, "wk": synth.TYPE_Q3_K, "wv": synth.TYPE_Q5_0, "wo": synth.TYPE_Q2_K,
            "w1": synth.TYPE_Q3_K, "w3": synth.TYPE_Q3_K, "w2": synth.TYPE_Q2_K if layer % 2 else synth.TYPE_Q5_0}


@pytest.mark.gpu
def test_low_bit_types_logits_and_graph_step_match_reference():
    """Prefill (GEMMs for Q5_0, matvec passes for Q2_K / Q3_K), eager decode
    and the graph-captured decode step on Q2_K, Q3_K and Q5_0 weights."""
    import torch

    import arm_ai_amd as A
    from arm_ai_amd.llama import Llama, synthetic_weights

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    hw = synthetic_weights(_tiny_cfg(), seed=17, types=_low_bit_types, unit=True)
    ctx = A.Context(0)
    model = Llama(ctx, hw)
    try:
        ref = RefLlama(hw)
        rng = np.random.default_rng(17)
        prompt = rng.integers(0, hw.cfg.vocab, size=12).tolist()
        g = model.forward(prompt, 0).cpu().numpy()
        r = ref.forward(prompt, 0)
        assert _rel(g, r) <= LOGIT_TOL, f"prefill logits rel {_rel(g, r):.3e}"
        pos = len(prompt)
        for step in range(2):
            tok = int(rng.integers(0, hw.cfg.vocab))
            g = model.forward([tok], pos).cpu().numpy()
            r = ref.forward([tok], pos)
            assert _rel(g, r) <= LOGIT_TOL, f"decode step {step} logits rel {_rel(g, r):.3e}"
            pos += 1
        assert model.generate(prompt, 6, graph=False).tokens == model.generate(prompt, 6, graph=True).tokens
    finally:
        model.free()
        ctx.close()


@pytest.mark.gpu
def test_graph_decode_step_matches_eager(tiny):
    hw, model = tiny
    prompt = [1, 2, 3, 4, 5]
    model.forward(prompt, 0)
    eager = model.forward([9], 5).cpu().numpy()
    model.forward(prompt, 0)  # same cache contents again
    first = None
    for rep in range(3):  # replays with eager work in between, each checked
        graph = model.decode_step_graph(9, 5).cpu().numpy()
        # the static step attends over max_seq positions (masked), so its f32
        # sums may round differently from the eager step's, not from each other
        assert _rel(graph, eager) <= LOGIT_TOL, f"replay {rep}: rel {_rel(graph, eager):.3e}"
        if first is None:
            first = graph
        assert np.array_equal(graph, first), f"replay {rep} differs from the first replay"
        model.forward(prompt, 0)


@pytest.mark.gpu
def test_generate_greedy_eager_and_graph_agree(tiny):
    hw, model = tiny
    ref = RefLlama(hw)
    prompt = [7, 100, 33, 250, 3, 9]
    a = model.generate(prompt, 6)
    b = model.generate(prompt, 6, graph=True)
    assert len(a.tokens) == 6
    assert a.tokens == b.tokens
    # the reference's greedy choice at each step, fed the GPU's tokens
    toks = list(prompt)
    logits = ref.forward(toks, 0)
    margin_ok = []
    for t in a.tokens:
        top2 = np.sort(logits)[-2:]
        if top2[1] - top2[0] > 1e-2 * np.max(np.abs(logits)):
            assert t == int(np.argmax(logits))
            margin_ok.append(True)
        logits = ref.forward([t], len(toks))
        toks.append(t)
    assert margin_ok, "no step had a clear argmax"
    st = a.stats(len(prompt))
    assert st["n_new"] == 6 and st["n_prompt"] == len(prompt) and st["decode_ms_per_tok"] is not None


@pytest.mark.gpu
def test_generate_stops_after_stop_token_and_edge_cases(tiny):
    hw, model = tiny
    prompt = [11, 12, 13]
    first = model.generate(prompt, 1).tokens
    assert len(first) == 1
    r = model.generate(prompt, 5, stop_tokens=(first[0],))
    assert r.tokens == first  # the stop token is emitted, then generation ends
    assert model.generate([], 5).tokens == []
    assert model.generate(prompt, 0).tokens == []


@pytest.mark.gpu
def test_odd_vocab_graph_generate():
    """A vocabulary that is not a multiple of four (514): the graph-captured
    step (device argmax) and the eager path pick the same tokens."""
    import torch

    import arm_ai_amd as A
    from arm_ai_amd.llama import Llama, LlamaConfig, synthetic_weights

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    cfg = LlamaConfig(n_layer=2, hidden=256, ffn=512, n_head=4, n_kv_head=2, vocab=514, max_seq=64)
    hw = synthetic_weights(cfg, seed=21, unit=True)
    ctx = A.Context(0)
    model = Llama(ctx, hw)
    try:
        prompt = [3, 513, 100, 7]
        assert model.generate(prompt, 6, graph=False).tokens == model.generate(prompt, 6, graph=True).tokens
    finally:
        model.free()
        ctx.close()


@pytest.mark.gpu
def test_generate_streams_each_token_before_the_next_step(tiny):
    """generate(..., on_token=cb), the streaming form of llama_candle_stream_op
    (native/arm_ai_nif/src/lib.rs:1682-1699, gpu_llama.rs generate_greedy_with):
    the callback fires once per token, in order, with the tokens of the eager
    generate; with the graph, token j (j >= 1) is delivered after exactly j
    replays (the device position reads prompt + j when the callback runs), so
    no step runs ahead of the delivery; a stop token is delivered and ends the
    stream."""
    hw, model = tiny
    prompt = [7, 100, 33, 250, 3, 9]
    eager = model.generate(prompt, 8).tokens
    assert len(eager) == 8
    for graph in (False, True):
        seen, pos_at = [], []

        def cb(t, graph=graph):
            seen.append(t)
            if graph and len(seen) > 1:
                pos_at.append(int(model._pos.item()))

        res = model.generate(prompt, 8, graph=graph, on_token=cb)
        assert seen == res.tokens == eager, f"graph={graph}"
        if graph:
            assert pos_at == [len(prompt) + j for j in range(1, 8)]
    stop = eager[3]
    first = eager.index(stop)
    seen = []
    res = model.generate(prompt, 8, stop_tokens=(stop,), graph=True, on_token=seen.append)
    assert res.tokens == eager[:first + 1] == seen
    seen = []
    assert model.generate(prompt, 8, stop_tokens=(eager[0],), graph=True, on_token=seen.append).tokens == eager[:1]
    assert seen == eager[:1]


@pytest.mark.gpu
def test_reserve_leaves_no_trace(tiny):
    """Llama reserves a prompt's buffers at construction (one forward of
    min(max_seq, 512) tokens at offset 0, then the KV cache cleared): a model
    built without it gives the same logits and tokens, bit for bit, and the
    reserving model's cache starts at zero."""
    import arm_ai_amd as A
    from arm_ai_amd.llama import Llama

    hw, model = tiny
    rng = np.random.default_rng(41)
    prompt = rng.integers(0, hw.cfg.vocab, size=20).tolist()
    ctx = A.Context(0)
    fresh = Llama(ctx, hw, reserve=0)
    try:
        reserved = Llama(ctx, hw)
        try:
            assert float(reserved.k_cache.abs().sum()) == 0.0 and float(reserved.v_cache.abs().sum()) == 0.0
            a = reserved.forward(prompt, 0).cpu().numpy()
            b = fresh.forward(prompt, 0).cpu().numpy()
            assert np.array_equal(a, b)
            assert reserved.generate(prompt, 5).tokens == fresh.generate(prompt, 5).tokens
        finally:
            reserved.free()
    finally:
        fresh.free()
        ctx.close()


# ------------------------------------------------------------ SmolLM-135M shape
def test_swiglu_pair_rows_interleaves_gate_and_up_rows_in_fours():
    """Row 8b + j of the paired weight is gate row 4b + j (j < 4) or up row
    4b + j - 4, every row's quantized blocks unchanged; mismatched pairs are
    refused."""
    from arm_ai_amd import synth
    from arm_ai_amd.llama import swiglu_pair_rows
    from arm_ai_amd.qmatmul import QTensor

    ffn, k = 24, 256
    rb = 144  # one Q4_K block per row
    w1 = QTensor(synth.TYPE_Q4_K, (ffn, k), np.repeat(np.arange(ffn, dtype=np.uint8), rb))
    w3 = QTensor(synth.TYPE_Q4_K, (ffn, k), np.repeat(np.arange(100, 100 + ffn, dtype=np.uint8), rb))
    p = swiglu_pair_rows(w1, w3)
    assert p.dtype == synth.TYPE_Q4_K and tuple(p.shape) == (2 * ffn, k)
    rows = np.asarray(p.data).reshape(2 * ffn, rb)
    assert np.all(rows == rows[:, :1])
    want = [4 * (r // 8) + r % 4 + (0 if r % 8 < 4 else 100) for r in range(2 * ffn)]
    assert rows[:, 0].tolist() == want
    with pytest.raises(ValueError):
        swiglu_pair_rows(w1, QTensor(synth.TYPE_Q6_K, (ffn, k), np.zeros(ffn * 210, np.uint8)))
    with pytest.raises(ValueError):
        swiglu_pair_rows(QTensor(synth.TYPE_Q4_K, (6, k), np.zeros(6 * rb, np.uint8)),
                         QTensor(synth.TYPE_Q4_K, (6, k), np.zeros(6 * rb, np.uint8)))


def test_gguf_fallback_types_for_rows_not_a_multiple_of_256():
    """llama.cpp's Q4_K_M writes the fallback type where a row (k) is not a
    multiple of 256: SmolLM-135M's hidden 576 turns Q4_K into Q5_0 and Q6_K
    into Q8_0; w2 (k = 1536) keeps its K-quant."""
    from arm_ai_amd import synth
    from arm_ai_amd.llama import fallback_q4km_types, gguf_fallback_type, smollm_135m_config

    cfg = smollm_135m_config()
    assert cfg.head_dim == 64 and cfg.n_head // cfg.n_kv_head == 3
    t0, t1 = fallback_q4km_types(cfg, 0), fallback_q4km_types(cfg, 1)
    assert t0 == {"wq": synth.TYPE_Q5_0, "wk": synth.TYPE_Q5_0, "wv": synth.TYPE_Q8_0, "wo": synth.TYPE_Q5_0,
                  "w1": synth.TYPE_Q5_0, "w3": synth.TYPE_Q5_0, "w2": synth.TYPE_Q4_K}
    assert t1["w2"] == synth.TYPE_Q6_K
    assert gguf_fallback_type(synth.TYPE_Q6_K, 576) == synth.TYPE_Q8_0
    assert gguf_fallback_type(synth.TYPE_Q4_K, 512) == synth.TYPE_Q4_K


@pytest.fixture(scope="module")
def smollm():
    """SmolLM-135M's widths and heads (hidden 576, FFN 1536, 9 query / 3 kv
    heads, vocabulary 49152) with three of its 30 layers, the Q4_K_M mix with
    the fallback types (Q5_0, Q8_0) of rows that are not a multiple of 256,
    and the Q8_0 output head of the tied embedding."""
    import torch

    import arm_ai_amd as A
    from arm_ai_amd import synth
    from arm_ai_amd.llama import Llama, fallback_q4km_types, smollm_135m_config, synthetic_weights

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    cfg = smollm_135m_config(max_seq=96)
    cfg.n_layer = 3
    hw = synthetic_weights(cfg, seed=31, types=fallback_q4km_types, output_type=synth.TYPE_Q8_0, unit=True)
    ctx = A.Context(0)
    model = Llama(ctx, hw)
    yield hw, model
    model.free()
    ctx.close()


@pytest.mark.gpu
def test_smollm_shape_matmuls_glue_graph_step_and_generate(smollm):
    """Prefill (Q5_0 / Q8_0 GEMMs on k = 576, the Q4_K / Q6_K ones on k =
    1536, prompt attention at three query heads per kv head) and two decode
    steps, checked as the full-size test checks config 2: every projection
    on the GPU's own input against the oracle (block sums bit-exact on one
    row), layer 0's glue step by step, the logits against an independent CPU
    run at the bar the Q8 rounding-boundary compounding allows (a norm output
    one ulp apart moves quants of 32-element Q8_0 blocks across a boundary:
    measured 3e-3 on the hidden state after one layer, 1.3e-2 on the logits
    after three); then the graph-captured step against the eager one and
    greedy generation, graph against eager teacher-forced."""
    from tests.test_llama_fullsize import _check_records, _Glue, _graph_vs_eager, _host_blocks, _layer_records

    hw, model = smollm
    cfg = hw.cfg
    ref = RefLlama(hw)
    host_of = _host_blocks(model, hw)
    assert "w13" in model.layers[0]  # rows of 576: [g | u], silu(g) * u in the w2 launch
    glue = _Glue(ref, 0, "w13p" in model.layers[0])
    rng = np.random.default_rng(33)
    prompt = rng.integers(0, cfg.vocab, size=40).tolist()
    pos = 0
    for i, toks in enumerate([prompt, [int(rng.integers(0, cfg.vocab))], [int(rng.integers(0, cfg.vocab))]]):
        what = "prefill" if i == 0 else f"decode step {i - 1}"
        with model.capture_hidden({0, 1}) as hx, model.trace_matmuls((0, 1, len(toks) - 1), full_layers=(0,)) as recs:
            g = model.forward(toks, pos).cpu().numpy()
        assert np.all(np.isfinite(g))
        assert len(recs) == 5 * cfg.n_layer + 1
        _check_records(recs, host_of, what)
        for name, e in glue.check(hx[0], _layer_records(recs, 0), hx[1], pos).items():
            assert e <= 1e-5, f"{what}, layer 0: {name} rel {e:.3e}"
        r = ref.forward(toks, pos)
        assert _rel(g, r) <= 5e-2, f"{what}: logits against the independent CPU run rel {_rel(g, r):.3e}"
        pos += len(toks)
    gerr = _graph_vs_eager(model, rng.integers(0, cfg.vocab, size=4).tolist(), pos)
    assert max(gerr) <= 5e-2, f"graph step vs eager rel {max(gerr):.3e}"
    # greedy generation: the graph's tokens against the eager argmax fed the
    # same tokens, wherever the eager margin is clear of the step difference
    toks = model.generate(prompt, 8, graph=True).tokens
    lg = model.forward(prompt, 0).cpu().numpy()
    margin = 2.0 * max(max(gerr), 1e-3)
    for i, t in enumerate(toks):
        top2 = np.sort(lg)[-2:]
        if top2[1] - top2[0] > margin * np.max(np.abs(lg)):
            assert t == int(np.argmax(lg)), f"token {i}"
        if i + 1 < len(toks):
            lg = model.forward([t], len(prompt) + i).cpu().numpy()
