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


# ---------------------------------------------------------------- a byte stream built from the spec
# The file below is assembled field by field with struct.pack from the public
# GGUF specification (ggml docs/gguf.md), without write_gguf, so a reader and
# writer that shared a misreading (count widths, dims order, alignment padding,
# array encoding) cannot pass together.
def _spec_str(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def _spec_kv(key: bytes, vtype: int, payload: bytes) -> bytes:
    return _spec_str(key) + struct.pack("<I", vtype) + payload


def _spec_file(version: int, alignment: int | None, pad_byte: int = 0):
    """A two-tensor GGUF byte string and what a correct reader must find in it."""
    W = synth.make_weight(synth.TYPE_Q4_K, 3, 512, seed=31)  # n = 3 rows, k = 512 columns
    norm = np.array([1.5, -2.0, 0.25, 8.0, 0.0, -0.125], "<f4")
    kvs = [
        _spec_kv(b"general.architecture", gguf.T_STR, _spec_str(b"llama")),
        _spec_kv(b"t.u8", gguf.T_U8, struct.pack("<B", 200)),
        _spec_kv(b"t.i8", gguf.T_I8, struct.pack("<b", -100)),
        _spec_kv(b"t.u16", gguf.T_U16, struct.pack("<H", 65000)),
        _spec_kv(b"t.i16", gguf.T_I16, struct.pack("<h", -32000)),
        _spec_kv(b"t.i32", gguf.T_I32, struct.pack("<i", -7)),
        _spec_kv(b"t.f64", gguf.T_F64, struct.pack("<d", 0.1)),
        _spec_kv(b"t.u64", gguf.T_U64, struct.pack("<Q", 2 ** 40 + 3)),
        _spec_kv(b"t.i64", gguf.T_I64, struct.pack("<q", -(2 ** 40))),
        _spec_kv(b"t.bool", gguf.T_BOOL, struct.pack("<B", 1)),
        # typed arrays: (element type u32, count u64, elements)
        _spec_kv(b"t.arr_i16", gguf.T_ARR, struct.pack("<IQ", gguf.T_I16, 3) + struct.pack("<3h", -1, 2, -3)),
        _spec_kv(b"t.arr_f32", gguf.T_ARR, struct.pack("<IQ", gguf.T_F32, 2) + struct.pack("<2f", 0.5, -4.0)),
        _spec_kv(b"t.arr_str", gguf.T_ARR, struct.pack("<IQ", gguf.T_STR, 2) + _spec_str(b"<s>") + _spec_str(b"\xc3\xa9")),
    ]
    if alignment is not None:
        kvs.append(_spec_kv(b"general.alignment", gguf.T_U32, struct.pack("<I", alignment)))
    align = alignment or 32
    # tensor 0: the 1-D norm at offset 0; tensor 1: the weight at the next aligned offset
    off1 = (norm.nbytes + align - 1) // align * align
    infos = (_spec_str(b"blk.0.attn_norm.weight") + struct.pack("<I", 1) + struct.pack("<Q", 6)
             + struct.pack("<IQ", gguf.GGML_F32, 0)
             + _spec_str(b"blk.0.attn_q.weight") + struct.pack("<I", 2) + struct.pack("<2Q", 512, 3)
             + struct.pack("<IQ", synth.TYPE_Q4_K, off1))
    head = b"GGUF" + struct.pack("<IQQ", version, 2, len(kvs)) + b"".join(kvs) + infos
    data_start = (len(head) + align - 1) // align * align
    body = bytearray(head + bytes([pad_byte]) * (data_start - len(head)))
    body += norm.tobytes() + bytes([pad_byte]) * (off1 - norm.nbytes) + W.blocks.tobytes()
    return bytes(body), data_start, off1, W, norm


@pytest.mark.parametrize("version,alignment", [(3, 64), (2, 64), (3, None), (3, 256)])
def test_reader_against_a_spec_built_file(tmp_path, version, alignment):
    raw, data_start, off1, W, norm = _spec_file(version, alignment, pad_byte=0xAA)
    p = tmp_path / "spec.gguf"
    p.write_bytes(raw)
    g = gguf.GGUFFile(str(p))
    assert g.version == version
    assert g.data_start == data_start and data_start % (alignment or 32) == 0
    md = g.metadata
    assert md["general.architecture"] == "llama"
    assert (md["t.u8"], md["t.i8"], md["t.u16"], md["t.i16"], md["t.i32"]) == (200, -100, 65000, -32000, -7)
    assert md["t.f64"] == 0.1 and md["t.u64"] == 2 ** 40 + 3 and md["t.i64"] == -(2 ** 40) and md["t.bool"] is True
    assert md["t.arr_i16"].dtype == np.dtype("<i2") and list(md["t.arr_i16"]) == [-1, 2, -3]
    assert md["t.arr_f32"].dtype == np.dtype("<f4") and list(md["t.arr_f32"]) == [0.5, -4.0]
    assert md["t.arr_str"] == ["<s>", "é"]
    if alignment is not None:
        assert md["general.alignment"] == alignment
    tn, tq = g.tensor("blk.0.attn_norm.weight"), g.tensor("blk.0.attn_q.weight")
    assert (tn.dims, tn.type, tn.offset) == ((6,), gguf.GGML_F32, 0)
    assert (tq.dims, tq.type, tq.offset) == ((512, 3), synth.TYPE_Q4_K, off1)
    assert tq.shape == (3, 512) and tq.nbytes == 3 * 2 * 144
    # the bytes at data_start + offset, not at the end of the infos
    assert np.array_equal(g.f32("blk.0.attn_norm.weight"), norm)
    q = g.qtensor("blk.0.attn_q.weight")
    assert q.shape == (3, 512) and np.array_equal(np.asarray(q.data).reshape(-1), W.blocks.reshape(-1))
    assert np.array_equal(np.asarray(g.raw("blk.0.attn_q.weight")), np.frombuffer(raw, np.uint8)[data_start + off1:])


def test_spec_built_file_rejects_bad_alignment_and_short_data(tmp_path):
    raw, data_start, off1, _, _ = _spec_file(3, 48)  # not a power of two
    p = tmp_path / "a48.gguf"
    p.write_bytes(raw)
    with pytest.raises(gguf.GGUFError, match="alignment"):
        gguf.GGUFFile(str(p))
    raw, *_ = _spec_file(3, 64)
    p.write_bytes(raw[:-1])  # the weight's last byte is missing
    with pytest.raises(gguf.GGUFError, match="past the end"):
        gguf.GGUFFile(str(p))
