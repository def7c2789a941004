"""The Rust NIF shim (native/arm_ai_nif) checked without a Rust toolchain
(cargo is not in this image): its FFI declarations against include/aq.h, its
calls against its declarations, its hipcc flags against the library's own
build, and the API it gives lib.rs against the names the reference's NIFs
call (native/arm_ai_nif/src/lib.rs:1659-1699 calls
llama_candle::load_model, generate_greedy, generate_greedy_with and reads
GenerateResult's tokens / prefill_us / decode_us)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NIF = os.path.join(ROOT, "native", "arm_ai_nif")

C_TO_RUST = {"int": "c_int", "int64_t": "i64", "size_t": "usize", "float": "f32", "void": "c_void", "char": "c_char",
             "aq_ctx": "AqCtx", "aq_qweight": "AqQWeight", "int8_t": "i8", "uint8_t": "u8", "uint16_t": "u16",
             "int32_t": "i32", "uint32_t": "u32"}


def _read(*p):
    with open(os.path.join(*p)) as f:
        return f.read()


def _c_type_to_rust(t):
    t = t.strip()
    const = t.startswith("const ")
    base = t.replace("const ", "").replace("*", "").strip()
    stars = t.count("*")
    r = C_TO_RUST[base]
    if stars == 0:
        return r
    if stars == 1:
        return ("*const " if const else "*mut ") + r
    return "*mut *mut " + r


def _header_protos():
    src = re.sub(r"/\*.*?\*/", "", _read(ROOT, "include", "aq.h"), flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"\b((?:const\s+)?[a-z_0-9]+\s*\*?)\s*(aq_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src):
        types = []
        for p in params.split(","):
            p = p.strip()
            if not p or p == "void":
                continue
            types.append(_c_type_to_rust(re.match(r"(.*?)[A-Za-z_][A-Za-z_0-9]*$", p).group(1)))
        out[name] = (types, _c_type_to_rust(ret))
    return out


def _rust_decls(path):
    src = _read(path)
    block = src[src.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    out = {}
    for name, params, ret in re.findall(r"pub fn ([a-zA-Z_0-9]+)\((.*?)\)\s*->\s*([^;]+);", block, flags=re.S):
        types = [a.split(":", 1)[1].strip() for a in _split_top(params) if a.strip()]
        out[name] = (types, ret.strip())
    return out


def _split_top(s):
    """Split at commas outside (), [], <>, {}."""
    parts, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([<{":
            depth += 1
        elif ch in ")]>}":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur)
    return parts


def _calls(src, prefix):
    """(name, argument count) of every call `prefix...(` in Rust source."""
    src = re.sub(r"//[^\n]*", "", src)
    out = []
    for m in re.finditer(r"\b(" + prefix + r"[A-Za-z0-9_]*)\(", src):
        if src[max(0, m.start() - 7):m.start()].strip().endswith("fn"):
            continue  # a declaration
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(src[i], 0)
            i += 1
        args = src[m.end():i - 1]
        out.append((m.group(1), len([a for a in _split_top(args) if a.strip()])))
    return out


def test_ffi_declares_every_header_function_with_its_c_types():
    hdr = _header_protos()
    rs = _rust_decls(os.path.join(NIF, "src", "aq_sys.rs"))
    assert len(hdr) >= 50
    assert sorted(rs) == sorted(hdr)
    for name, (types, ret) in hdr.items():
        assert rs[name] == (types, ret), f"{name}: header {types} -> {ret}, Rust {rs[name]}"


def test_shim_calls_match_their_declarations():
    aq = _rust_decls(os.path.join(NIF, "src", "aq_sys.rs"))
    hip = _rust_decls(os.path.join(NIF, "src", "hip_sys.rs"))
    seen = set()
    for f in ("gpu_llama.rs", "gpu_qmatmul.rs", "hip_sys.rs"):
        src = _read(NIF, "src", f)
        for name, n in _calls(src, "aq_"):
            if name in ("aq_type",):  # the shim's own helper
                continue
            assert name in aq, f"{f}: {name} is not in include/aq.h"
            assert n == len(aq[name][0]), f"{f}: {name} called with {n} arguments, declared with {len(aq[name][0])}"
            seen.add(name)
        for name, n in _calls(src, "hip"):
            if name in ("hip_check",):
                continue
            assert name in hip, f"{f}: {name} is not declared in hip_sys.rs"
            assert n == len(hip[name][0]), f"{f}: {name} called with {n} arguments"
    # the decode step and the prompt path use the library's glue entries
    for need in ("aq_llama_attn_prefill", "aq_llama_attn_decode", "aq_qmatmul2_rmsnorm_f32_device",
                 "aq_llama_argmax", "aq_qmatmul_f32_device", "aq_qweight_upload"):
        assert need in seen, need


def test_build_rs_compiles_with_the_library_flags():
    rs = _read(NIF, "build.rs")
    flags = re.findall(r'"([^"]+)"', rs[rs.index("const HIPCC_FLAGS"):rs.index("];")])
    from arm_ai_amd import build

    assert flags == [f for f in build.HIPCC_FLAGS if not f.startswith("--offload-arch")]
    assert '"-packed-fp32-ops"' in rs and "--offload-arch={arch}" in rs
    assert "CARGO_FEATURE_GPU_MI355X" in rs  # a no-op without the feature


def test_module_gives_lib_rs_the_llama_candle_api():
    src = _read(NIF, "src", "gpu_llama.rs")
    assert re.search(r"pub fn load_model\(path: &str\) -> Result<LlamaResource, String>", src)
    assert re.search(r"pub fn generate_greedy\(res: &LlamaResource, prompt: &\[u32\], max_new: usize, "
                     r"stop_tokens: &\[u32\]\)\s*-> Result<GenerateResult, String>", src)
    assert re.search(r"pub fn generate_greedy_with\(res: &LlamaResource, prompt: &\[u32\], max_new: usize, "
                     r"stop_tokens: &\[u32\],\s*on_token: &mut dyn FnMut\(u32\)\) -> Result<GenerateResult, String>",
                     src)
    res = src[src.index("pub struct GenerateResult"):]
    res = res[:res.index("}")]
    for field in ("pub tokens: Vec<u32>", "pub prefill_us: u64", "pub decode_us: u64"):
        assert field in res
    assert "pub model: Mutex<GpuLlama>" in src
    # per-token delivery for the stream NIF: one token read back per replay
    body = src[src.index("pub fn generate_greedy_with"):]
    assert "generate_chunked(res, prompt, max_new, stop_tokens, on_token, 1)" in body[:400]
