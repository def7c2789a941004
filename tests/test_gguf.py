"""GGUF reader / writer (arm_ai_amd.gguf): the load path of ArmAI.LlamaCandle
(llama_candle.rs:35-48, candle's gguf_file::Content::read and
ModelWeights::from_gguf).

CPU tests: a synthetic model written and read back byte for byte;
dequantisation of Q4_K / Q6_K / Q8_0 blocks against the generator's element
arrays (the GGML formulas, computed independently of the reader's unpacking);
the tied-output rule; and the error paths the reference's own tests pin for
load/2 (test/llama_candle_test.exs: missing file and empty path return an
error), plus malformed files.  GPU test: a model loaded from its GGUF file
gives the same logits as the in-memory one.
"""
import struct

import numpy as np
import pytest

from arm_ai_amd import gguf, synth
from arm_ai_amd.llama import LlamaConfig, synthetic_weights
from arm_ai_amd.qmatmul import QTensor


def _cfg():
    return LlamaConfig(n_layer=2, hidden=256, ffn=512, n_head=4, n_kv_head=2, vocab=512, max_seq=64)


def test_round_trip_bytes_and_config(tmp_path):
    hw = synthetic_weights(_cfg(), seed=4)
    p = str(tmp_path / "m.gguf")
    gguf.save_llama(p, hw)
    cfg2, hw2 = gguf.load_llama(p, max_seq=64)
    c = hw.cfg
    assert (cfg2.n_layer, cfg2.hidden, cfg2.ffn, cfg2.n_head, cfg2.n_kv_head, cfg2.vocab) == (
        c.n_layer, c.hidden, c.ffn, c.n_head, c.n_kv_head, c.vocab)
    assert cfg2.rope_theta == c.rope_theta and np.float32(cfg2.rms_eps) == np.float32(c.rms_eps)
    for a, b in zip(hw.layers, hw2.layers):
        for k in a:
            assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape
            assert np.array_equal(a[k].data, b[k].data), k
    for a, b in zip(hw.attn_norm + hw.ffn_norm, hw2.attn_norm + hw2.ffn_norm):
        assert np.array_equal(a, b)
    assert np.array_equal(hw.tok_embeddings, hw2.tok_embeddings)
    assert np.array_equal(hw.norm, hw2.norm)
    assert np.array_equal(hw.output.data, hw2.output.data) and hw2.output.shape == hw.output.shape


@pytest.mark.parametrize("wtype", [synth.TYPE_Q4_K, synth.TYPE_Q5_K, synth.TYPE_Q6_K, synth.TYPE_Q8_0, synth.TYPE_Q4_0,
                                   synth.TYPE_Q2_K, synth.TYPE_Q3_K, synth.TYPE_Q5_0])
def test_dequantize_matches_element_formulas(wtype):
    W = synth.make_weight(wtype, 7, 512, seed=wtype)
    got = gguf.dequantize(wtype, W.blocks, 7 * 512).reshape(7, 512)
    want = W.dequantize()  # f64 from the generator's element arrays
    assert np.allclose(got, want, rtol=2e-6, atol=1e-9)


def test_quantized_embedding_and_tied_output(tmp_path):
    hw = synthetic_weights(_cfg(), seed=5)
    W = synth.make_weight(synth.TYPE_Q6_K, hw.cfg.vocab, hw.cfg.hidden, seed=9)
    emb = QTensor(synth.TYPE_Q6_K, (hw.cfg.vocab, hw.cfg.hidden), W.blocks)
    p = str(tmp_path / "tied.gguf")
    gguf.save_llama(p, hw, embedding=emb, tie_output=True)
    _, hw2 = gguf.load_llama(p)
    assert np.array_equal(hw2.output.data, W.blocks.reshape(-1))  # output head = the embedding's blocks
    assert np.allclose(hw2.tok_embeddings, W.dequantize(), rtol=2e-6, atol=1e-9)


def test_metadata_types_arrays_and_alignment(tmp_path):
    p = str(tmp_path / "md.gguf")
    t = np.arange(8, dtype="<f4")
    gguf.write_gguf(p, {"a.u": 7, "a.f": 0.5, "a.s": "x", "a.b": True, "a.tokens": ["<s>", "</s>", "hi"],
                        "a.ints": [1, -2, 3]}, [("t", (8,), gguf.GGML_F32, t)], alignment=64)
    g = gguf.GGUFFile(p)
    assert g.version == 3
    assert g.get("a.u") == 7 and g.get("a.f") == 0.5 and g.get("a.s") == "x" and g.get("a.b") is True
    assert g.get("a.tokens") == ["<s>", "</s>", "hi"]
    assert list(g.get("a.ints")) == [1, -2, 3]
    assert g.data_start % 64 == 0
    assert np.array_equal(g.f32("t"), t)


def test_load_errors(tmp_path):
    # the reference's own load/2 error tests: missing file, empty path
    with pytest.raises(gguf.GGUFError):
        gguf.load_llama(str(tmp_path / "__nope.gguf"))
    with pytest.raises(gguf.GGUFError):
        gguf.load_llama("")
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + b"\0" * 64)
    with pytest.raises(gguf.GGUFError, match="magic"):
        gguf.GGUFFile(str(bad))
    v1 = tmp_path / "v1.gguf"
    v1.write_bytes(b"GGUF" + struct.pack("<III", 1, 0, 0))
    with pytest.raises(gguf.GGUFError, match="version"):
        gguf.GGUFFile(str(v1))
    hw = synthetic_weights(_cfg(), seed=6)
    p = tmp_path / "trunc.gguf"
    gguf.save_llama(str(p), hw)
    data = p.read_bytes()
    p.write_bytes(data[:len(data) // 2])
    with pytest.raises(gguf.GGUFError):
        gguf.load_llama(str(p))
    p.write_bytes(data[:40])
    with pytest.raises(gguf.GGUFError):
        gguf.GGUFFile(str(p))
    # a projection of a type the matmuls do not take
    q = tmp_path / "f32proj.gguf"
    gguf.write_gguf(str(q), {"general.architecture": "llama"},
                    [("blk.0.attn_q.weight", (256, 4), gguf.GGML_F32, np.zeros((4, 256), "<f4"))])
    with pytest.raises(gguf.GGUFError):
        gguf.GGUFFile(str(q)).qtensor("blk.0.attn_q.weight")
    with pytest.raises(gguf.GGUFError, match="architecture"):
        gguf.write_gguf(str(q), {"general.architecture": "gpt2"}, [])
        gguf.load_llama(str(q))


@pytest.mark.gpu
def test_loaded_model_gives_the_same_logits(tmp_path):
    import torch

    import arm_ai_amd as A
    from arm_ai_amd.llama import Llama

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need torch to see the GPU")
    hw = synthetic_weights(_cfg(), seed=7)
    p = str(tmp_path / "m.gguf")
    gguf.save_llama(p, hw)
    _, hw2 = gguf.load_llama(p, max_seq=64)
    ctx = A.Context(0)
    a, b = Llama(ctx, hw), Llama(ctx, hw2)
    prompt = [3, 1, 4, 1, 5, 9]
    la = a.forward(prompt, 0).cpu().numpy()
    lb = b.forward(prompt, 0).cpu().numpy()
    assert np.array_equal(la, lb)
    ga = a.generate(prompt, 5, graph=True).tokens
    gb = b.generate(prompt, 5, graph=True).tokens
    assert ga == gb
    a.free()
    b.free()
    ctx.close()
