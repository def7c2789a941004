"""Benchmark of the quantized-matmul hot path on one MI355X.

Metric: "Q4_K matvec HBM GB/s (% of peak) + prefill int8 TOPS; decode
tok/s" (the reference's headline).  The headline workload is the Llama-3-8B FFN up/gate
projection (config 4): Q4_K weight 14336 x 4096, batch 1.  A step is one pass
of the hot path over one activation row: Q8_K quantisation of x (f32 [1, 4096])
and the Q4_K matvec, i.e. candle's QMatMul::forward for that call.  At batch
<= 8 both run in one kernel (the matvec quantises x into LDS itself).

* Inputs are resident in HBM before timing.  Enough copies of the weight
  to hold 1.25 times the 256 MB Infinity Cache (11 of the headline's 33 MB)
  are used round-robin, so every step streams its weight from HBM.
* The K timed steps are captured once into a HIP graph and replayed, so the
  number is the GPU's, not the Python launch loop's.
* value = algorithmic bytes per step / time per step, bytes =
  weight (N*K/256*144) + f32 input (M*K*4) + f32 output (M*N*4).
* roofline: that one kernel (the step), K launches replayed from a graph
  between two HIP events on the library's stream; algorithmic bytes per
  launch = weight + f32 x + f32 y.  The pre-quantised variant of the matvec
  (activation already Q8_K in HBM) is reported under "extra".
* cpu_baseline: the oracle (a C restatement of candle's k_quants::matmul,
  generic vec_dot_unopt order, x86-64 baseline ISA, OpenMP over columns)
  on the same weight and input, all host cores.

* roofline.traffic: HBM bytes per launch of that kernel from two rocprofv3
  --pmc runs (FETCH_SIZE, WRITE_SIZE), each scaled by what the counter reads
  for a device-to-device copy of known size (`--copy-calibration`); read from
  profiles/traffic_matvec_q4k_14336x4096_b1.json, null if absent.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
       python bench.py --case NAME          (one of the extra configurations alone, e.g. for a profile)
       python bench.py --copy-calibration   (ten 64 MiB device-to-device copies, for PMC scaling)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA
MALL_BYTES = 256 << 20
METRIC = "Q4_K matvec HBM GB/s (% of peak) + prefill int8 TOPS; decode tok/s"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def copies_for(nbytes: int) -> int:
    return max(2, int(np.ceil(1.25 * MALL_BYTES / nbytes)))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


class Workload:
    """A weight (rotated over `copies` HBM copies) and an activation, ready on the device."""

    def __init__(self, ctx, wtype: int, n: int, k: int, m: int, seed: int):
        import arm_ai_amd as A
        from arm_ai_amd import hip
        from arm_ai_amd import synth as S

        self.wtype, self.n, self.k, self.m = wtype, n, k, m
        t0 = time.time()
        self.W = S.make_weight(wtype, n, k, seed=seed)
        self.x = S.make_activation(m, k, seed=seed + 1000)
        self.copies = copies_for(self.W.nbytes)
        qt = A.QTensor(wtype, (n, k), self.W.blocks)
        self.mms = [A.QMatMul.from_qtensor(qt, ctx) for _ in range(self.copies)]
        self.dx = hip.to_device(self.x)
        self.dy = hip.DeviceBuffer(m * n * 4)
        at = self.mms[0].act_type
        self.dact = hip.DeviceBuffer(A.act_bytes(at, m, k))
        A.quantize_act_device(ctx, at, self.dx.ptr, m, k, self.dact.ptr)
        ctx.synchronize()
        self.ctx = ctx
        act_q = m * (k // 32) * 34 if wtype in (8, 2, 6) else m * (k // 256) * 292
        self.weight_bytes = self.W.nbytes
        self.step_bytes = self.W.nbytes + m * k * 4 + m * n * 4  # quantizer fused into the step
        self.kernel_bytes = self.W.nbytes + act_q + m * n * 4  # matvec kernel alone
        log(f"workload type={wtype} n={n} k={k} m={m}: {self.copies} copies of {self.W.nbytes/1e6:.1f} MB ready in {time.time()-t0:.1f}s")

    def step(self, i: int) -> None:
        self.mms[i % self.copies].forward_device(self.dx.ptr, self.m, self.dy.ptr)

    def kernel(self, i: int) -> None:
        self.mms[i % self.copies].forward_preq_device(self.dact.ptr, self.m, self.dy.ptr)

    def free(self) -> None:
        for mm in self.mms:
            mm.free()
        self.mms = []


def time_graph(ctx, fn, count: int, warmup: int) -> tuple[float, float]:
    """Run fn(i) `warmup` times eagerly, capture `count` calls in a graph, replay once
    untimed, then time one replay.  Returns (ms per call from HIP events, wall ms per call)."""
    from arm_ai_amd import hip

    for i in range(warmup):
        fn(i)
    ctx.synchronize()
    g = hip.Graph(ctx.stream, lambda: [fn(i) for i in range(count)])
    g.launch()
    ctx.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    t0 = time.perf_counter()
    e0.record(ctx.stream)
    g.launch()
    e1.record(ctx.stream)
    e1.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    ms = e0.elapsed_ms(e1)
    return ms / count, wall / count


ISA_NOTES = {
    "baseline": "x86-64 baseline (-O3, no FMA contraction), OpenMP dynamic chunks of 256 columns",
    "v3": "x86-64-v3 (AVX2, FMA, BMI2; -O3, no FMA contraction, bit-identical results): the vectorised upper bound",
}


def cpu_baseline(wl: Workload, runs: int = 21, budget_s: float = 20.0, isa: str = "baseline") -> dict:
    import oracle as O

    threads = os.cpu_count() or 1
    x, W = wl.x, wl.W
    for _ in range(3):
        O.matmul(wl.wtype, x, W.blocks, wl.n, wl.k, nthreads=threads, isa=isa)
    times = []
    t_start = time.perf_counter()
    while len(times) < runs and time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        O.matmul(wl.wtype, x, W.blocks, wl.n, wl.k, nthreads=threads, isa=isa)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {
        "value": round(wl.step_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full {wl.n}x{wl.k} matmul at M={wl.m} (Q8_K quantisation + vec_dot_unopt), median of {len(times)} runs, {med*1e3:.2f} ms each",
        "cpu": cpu_model(),
        "isa": ISA_NOTES[isa],
    }


def cpu_prefill_baseline(wl: Workload, runs: int = 3) -> dict:
    """The oracle's k_quants::matmul at the prefill shape (every row quantised,
    then every column's vec_dot_unopt), all host cores: median of a few runs."""
    import oracle as O

    threads = os.cpu_count() or 1
    O.matmul(wl.wtype, wl.x, wl.W.blocks, wl.n, wl.k, nthreads=threads)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        O.matmul(wl.wtype, wl.x, wl.W.blocks, wl.n, wl.k, nthreads=threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"ms": round(med * 1e3, 2), "TOPS": round(2.0 * wl.m * wl.n * wl.k / med / 1e12, 4), "cores": threads,
            "kind": "port", "cpu": cpu_model(), "isa": ISA_NOTES["baseline"],
            "sample": f"the full {wl.m}x{wl.n}x{wl.k} matmul, median of {runs} runs"}


def traffic_from_profile():
    """HBM bytes per launch of the headline kernel from the committed PMC summary (or None)."""
    path = os.path.join(ROOT, "profiles", "traffic_matvec_q4k_14336x4096_b1.json")
    try:
        with open(path) as f:
            return int(json.load(f)["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def measure(ctx, wtype, n, k, m, steps, warmup, seed):
    wl = Workload(ctx, wtype, n, k, m, seed)
    step_ms, step_wall = time_graph(ctx, wl.step, steps, warmup)
    kern_ms, _ = time_graph(ctx, wl.kernel, steps, warmup)
    out = {
        "n": n, "k": k, "m": m, "weight_type": {12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 8: "Q8_0", 2: "Q4_0", 6: "Q5_0", 10: "Q2_K", 11: "Q3_K"}[wtype],
        "step_us": round(step_ms * 1e3, 3),
        "step_GBps": round(wl.step_bytes / (step_ms / 1e3) / 1e9, 1),
        "matvec_us": round(kern_ms * 1e3, 3),
        "matvec_GBps": round(wl.kernel_bytes / (kern_ms / 1e3) / 1e9, 1),
        "matvec_frac_hbm": round(wl.kernel_bytes / (kern_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
    }
    out["step_frac_hbm"] = round(wl.step_bytes / (step_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4)
    return wl, step_ms, step_wall, kern_ms, out


def measure_prefill(ctx, wtype, n, k, m, steps, warmup, seed, cpu=False):
    """Prefill GEMM at m rows: quantiser kernel + GEMM (step) and the GEMM alone
    (Q4_K, Q8_0, Q4_0: int8 MFMA; Q5_K, Q6_K: f16 MFMA after the f16 copy of
    the quants, which the GEMM time includes)."""
    wl = Workload(ctx, wtype, n, k, m, seed)
    step_ms, _ = time_graph(ctx, wl.step, steps, warmup)
    kern_ms, _ = time_graph(ctx, wl.kernel, steps, warmup)
    ops = 2.0 * m * n * k
    out = {
        "n": n, "k": k, "m": m, "weight_type": {12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 8: "Q8_0", 2: "Q4_0", 6: "Q5_0", 10: "Q2_K", 11: "Q3_K"}[wtype],
        "step_us": round(step_ms * 1e3, 3),
        "step_TOPS": round(ops / (step_ms / 1e3) / 1e12, 1),
        "gemm_us": round(kern_ms * 1e3, 3),
        "gemm_TOPS": round(ops / (kern_ms / 1e3) / 1e12, 1),
        "gemm_frac_int8_peak": round(ops / (kern_ms / 1e3) / 1e12 / INT8_PEAK_TOPS, 4),
    }
    if wtype in (13, 14):  # the kernel runs on the f16 matrix cores
        out["gemm_frac_f16_peak"] = round(ops / (kern_ms / 1e3) / 1e12 / F16_PEAK_TFLOPS, 4)
    if cpu:
        out["cpu_baseline"] = cpu_prefill_baseline(wl)
    wl.free()
    return out


MATVEC_CASES = {  # name: (weight type, n, k, m, seed)
    "c0_q4k_5632x2048_b1": (12, 5632, 2048, 1, 0),
    "c1_q8_0_2048x2048_b1": (8, 2048, 2048, 1, 1),
    "c1_q6k_32000x2048_b1": (14, 32000, 2048, 1, 2),
    "c4_q4k_4096x14336_b1": (12, 4096, 14336, 1, 5),
    "c4_q4k_14336x4096_b8": (12, 14336, 4096, 8, 6),
    "c4_q4k_4096x14336_b8": (12, 4096, 14336, 8, 8),
    "c4_q6k_4096x14336_b1": (14, 4096, 14336, 1, 20),  # ffn_down in a Q4_K_M file's Q6_K layers
    "c4_q6k_128256x4096_b1": (14, 128256, 4096, 1, 7),
    "c4_q6k_128256x4096_b8": (14, 128256, 4096, 8, 9),
    "q5k_14336x4096_b1": (13, 14336, 4096, 1, 13),  # a Q5_K_M file's ffn_up, batch 1
    "q4_0_14336x4096_b1": (2, 14336, 4096, 1, 14),  # a Q4_0 file's ffn_up, batch 1
    "q3k_14336x4096_b1": (11, 14336, 4096, 1, 17),  # a Q3_K_M file's ffn_up, batch 1
    "q2k_14336x4096_b1": (10, 14336, 4096, 1, 18),  # a Q2_K file's ffn_up, batch 1
    "q5_0_14336x4096_b1": (6, 14336, 4096, 1, 19),  # a Q5_0 file's ffn_up, batch 1
}
# Reference points, not this library: the vendor's plain int8 x int8 -> int32
# GEMM (hipBLASLt through torch._int_mm) at the prefill GEMMs' shapes, with no
# dequantisation work at all -- what the int8 matrix cores reach at M = 512 on
# this GPU without Q4_K decoding.
VENDOR_CASES = {  # name: (m, n, k)
    "ref_vendor_int8_gemm_512x14336x4096": (512, 14336, 4096),
    "ref_vendor_int8_gemm_512x5632x2048": (512, 5632, 2048),
    "ref_vendor_int8_gemm_512x2048x5632": (512, 2048, 5632),
}
DECODE_CASES = {  # name: (model, prompt tokens, new tokens, seed)
    "c2_tinyllama_decode": ("tinyllama", 512, 128, 2),
    # SmolLM-135M's shape (docs/perf_llm.md:98-99 quotes its Q4_K_M decode on
    # a phone): hidden 576, so its Q4_K_M file holds the fallback types
    "smollm135m_decode": ("smollm135m", 512, 128, 3),
}
CRATE_CASES = {  # the NIF crate's own kernels: name: (kind, m, n, k)
    "crate_q4_x_q8_gemv_4096x4096": ("q4_x_q8", 1, 4096, 4096),
    "crate_int4_gemv_f32_4096x4096": ("q4_0", 1, 4096, 4096),
    "crate_int8_weight_gemv_4096x4096": ("i8w", 1, 4096, 4096),
    "crate_int8_per_token_m512_4096x4096": ("i8i8", 512, 4096, 4096),
}
PREFILL_CASES = {  # name: (weight type, n, k, m, seed)
    "c3_prefill_q4k_5632x2048_m512": (12, 5632, 2048, 512, 3),
    "c3_prefill_q4k_2048x5632_m512": (12, 2048, 5632, 512, 3),
    "c4_prefill_q4k_14336x4096_m512": (12, 14336, 4096, 512, 4),
    "c2_prefill_q6k_2048x5632_m512": (14, 2048, 5632, 512, 10),  # TinyLlama ffn_down (Q6_K layers)
    "c2_prefill_q6k_256x2048_m512": (14, 256, 2048, 512, 11),    # TinyLlama attn_v
    "prefill_q8_0_4096x4096_m512": (8, 4096, 4096, 512, 12),     # a Q8_0 GGUF's projection
    "prefill_q4_0_4096x4096_m512": (2, 4096, 4096, 512, 15),     # Q4_0: the Q8_0 GEMM on the expanded copy
    "prefill_q5k_5632x2048_m512": (13, 5632, 2048, 512, 16),     # a Q5_K_M file's TinyLlama ffn_up
    "prefill_q5_0_4096x4096_m512": (6, 4096, 4096, 512, 20),     # Q5_0: the Q8_0 GEMM on the expanded copy
}


def cpu_decode_baseline(hw, prompt, n_steps=4, seed=0) -> dict:
    """Decode on the host with the CPU restatement of candle's quantized_llama
    (oracle/llama_ref.py: numpy f32 glue, the oracle's k_quants::matmul on all
    host cores) at the GPU run's context: the KV cache of every layer filled
    to the prompt's length (random values: a step's cost does not depend on
    them, and a CPU prefill of 512 rows would take tens of seconds), then
    n_steps greedy steps from there, timed -- positions len(prompt) ..
    len(prompt) + n_steps - 1, the GPU run's first n_steps."""
    from oracle.llama_ref import RefLlama

    cfg = hw.cfg
    ref = RefLlama(hw)
    rng = np.random.default_rng(seed)
    n = len(prompt)
    ref.k = [rng.standard_normal((cfg.n_kv_head, n, cfg.head_dim)).astype(np.float32) for _ in range(cfg.n_layer)]
    ref.v = [rng.standard_normal((cfg.n_kv_head, n, cfg.head_dim)).astype(np.float32) for _ in range(cfg.n_layer)]
    tok = int(prompt[-1])
    t0 = time.perf_counter()
    for i in range(n_steps):
        tok = int(np.argmax(ref.forward([tok], n + i)))
    dt = (time.perf_counter() - t0) / n_steps
    return {"decode_tok_s": round(1.0 / dt, 3), "decode_ms_per_tok": round(dt * 1e3, 2), "cores": os.cpu_count() or 1,
            "kind": "port", "cpu": cpu_model(), "isa": ISA_NOTES["baseline"],
            "sample": f"{n_steps} greedy steps at positions {n}..{n + n_steps - 1} (the GPU run's context; KV cache "
                      f"filled to {n} positions)"}


def decode_model(name, max_seq, seed):
    """The host weights of a decode case: TinyLlama-1.1B's shape with its
    Q4_K_M mix (config 2), or SmolLM-135M's with the Q4_K_M fallback types."""
    from arm_ai_amd import synth
    from arm_ai_amd.llama import LlamaConfig, fallback_q4km_types, smollm_135m_config, synthetic_weights

    if name == "tinyllama":
        cfg = LlamaConfig(max_seq=max_seq)
        desc = "TinyLlama-1.1B shape (22 layers, hidden 2048, FFN 5632, 32/4 heads, vocab 32000), Q4_K_M types"
        return desc, synthetic_weights(cfg, seed, unit=True)
    cfg = smollm_135m_config(max_seq=max_seq)
    desc = ("SmolLM-135M shape (30 layers, hidden 576, FFN 1536, 9/3 heads, vocab 49152, tied output), Q4_K_M "
            "types with the fallbacks of rows of 576 (Q5_0, Q8_0)")
    return desc, synthetic_weights(cfg, seed, types=fallback_q4km_types, output_type=synth.TYPE_Q8_0, unit=True)


def measure_decode(ctx, model_name, n_prompt, n_new, seed, with_cpu=True):
    """A Llama-shaped model with random weights (config 2: TinyLlama-1.1B's
    Q4_K_M shape), a prompt of uniform-random ids, greedy decode with the
    decode step replayed from a HIP graph; statistics as
    ArmAI.LlamaCandle.generate reports them."""
    from arm_ai_amd.llama import Llama

    t0 = time.perf_counter()
    desc, hw = decode_model(model_name, n_prompt + n_new, seed)
    cfg = hw.cfg
    wbytes = sum(qt.data.size for layer in hw.layers for qt in layer.values()) + hw.output.data.size
    model = Llama(ctx, hw)
    log(f"{model_name} model ready in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, cfg.vocab, size=n_prompt).tolist()
    model.generate(prompt[:16], 4, graph=True)  # capture the step, first-call set-up
    res = model.generate(prompt, n_new, graph=True)
    st = res.stats(n_prompt)
    eager = model.generate(prompt, 16)
    est = eager.stats(n_prompt)
    model.free()
    cpu = cpu_decode_baseline(hw, prompt) if with_cpu else None
    del hw
    out = {
        "model": desc + ", random unit-scaled weights (activations of order one through every layer)",
        "n_prompt": n_prompt,
        "n_new": st["n_new"],
        "decode_tok_s": round(1e3 / st["decode_ms_per_tok"], 1),
        "decode_ms_per_tok": round(st["decode_ms_per_tok"], 4),
        "prefill_ms": round(st["prefill_ms"], 3),
        "prefill_tok_s": round(st["prefill_tokens_per_sec"], 1),
        # the same prompt again (the eager run's prefill): no first-call allocations at this length
        "prefill_ms_warm": round(est["prefill_ms"], 3),
        "eager_decode_tok_s": round(1e3 / est["decode_ms_per_tok"], 1),
        "matmul_weight_bytes_per_token": int(wbytes),
        "weight_GBps_at_decode": round(wbytes / (st["decode_ms_per_tok"] / 1e3) / 1e9, 1),
        # greedy paths on random weights part where a top-2 logit margin is
        # below the graph step's rounding difference from the eager step
        # (tests/test_llama_fullsize.py holds them teacher-forced to the margin)
        "graph_eager_tokens_equal_before": next(
            (i for i, (a, b) in enumerate(zip(res.tokens, eager.tokens)) if a != b), len(eager.tokens)),
        "graph_eager_tokens_compared": len(eager.tokens),
        "timing": "wall clock around generate (llama_candle.rs:80-139 points); decode step replayed from a HIP graph",
    }
    if cpu is not None:
        out["cpu_baseline"] = cpu
    return out


def measure_crate(ctx, kind, m, n, k, steps, warmup):
    """One of the NIF crate's kernels on device memory (weights rotated over
    enough copies to exceed the Infinity Cache); GB/s of algorithmic bytes, or
    int8 TOPS for the int8 x int8 matmul."""
    import arm_ai_amd as A
    from arm_ai_amd import hip

    L = A._lib.load()
    rng = np.random.default_rng(11)
    if kind in ("q4_x_q8", "q4_0"):
        wbytes = n * (k // 2) + n * (k // 32) * 4
    elif kind == "i8w":
        wbytes = n * k + n * 4
    else:
        wbytes = n * k + n * 4
    copies = copies_for(wbytes)
    ws = []
    for _ in range(copies):
        if kind in ("q4_x_q8", "q4_0"):
            ws.append((hip.to_device(rng.integers(0, 256, (n, k // 2)).astype(np.uint8)),
                       hip.to_device(rng.uniform(1e-3, 0.05, (n, k // 32)).astype(np.float32))))
        else:
            ws.append((hip.to_device(rng.integers(-127, 128, (n, k)).astype(np.int8)),
                       hip.to_device(rng.uniform(1e-3, 0.05, n).astype(np.float32))))
    dout = hip.DeviceBuffer(m * n * 4)
    if kind == "i8i8":
        da = hip.to_device(rng.integers(-127, 128, (m, k)).astype(np.int8))
        das = hip.to_device(rng.uniform(1e-3, 0.05, m).astype(np.float32))
        fn = lambda i: L.aq_int8_matmul_f32_device(ctx.handle, da.ptr, ws[i % copies][0].ptr, das.ptr, 0.0,
                                                   ws[i % copies][1].ptr, m, n, k, dout.ptr)
    else:
        da = hip.to_device(rng.standard_normal((m, k)).astype(np.float32))
        if kind == "q4_x_q8":
            act = hip.DeviceBuffer(int(L.aq_q4_x_q8_act_bytes(k)))
            fn = lambda i: L.aq_int4_matmul_gemv_q4_x_q8_device(ctx.handle, da.ptr, ws[i % copies][0].ptr,
                                                                ws[i % copies][1].ptr, n, k, dout.ptr, act.ptr, None, None)
        else:
            fmt = 0 if kind == "q4_0" else 1
            fn = lambda i: L.aq_weight_only_matmul_device(ctx.handle, fmt, da.ptr, ws[i % copies][0].ptr,
                                                          ws[i % copies][1].ptr, m, n, k, dout.ptr)
    assert fn(0) == 0
    ms, _ = time_graph(ctx, fn, min(steps, 100), min(warmup, 10))
    out = {"kind": kind, "m": m, "n": n, "k": k, "us": round(ms * 1e3, 3), "rotating_weight_copies": copies}
    if kind == "i8i8":
        out["TOPS"] = round(2.0 * m * n * k / (ms / 1e3) / 1e12, 1)
        out["frac_int8_peak"] = round(out["TOPS"] / INT8_PEAK_TOPS, 4)
    else:
        nbytes = wbytes + m * k * 4 + m * n * 4
        out["GBps"] = round(nbytes / (ms / 1e3) / 1e9, 1)
        out["frac_hbm"] = round(out["GBps"] / HBM_PEAK_GBS, 4)
    return out


def measure_vendor_int8(m, n, k, steps, warmup):
    """torch._int_mm (hipBLASLt) on int8 operands of the given shape, the weight
    rotated over enough copies to exceed the Infinity Cache; HIP events around
    `steps` back-to-back calls."""
    import torch

    dev = torch.device("cuda:0")
    copies = copies_for(n * k)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev)
    bs = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev).t() for _ in range(copies)]
    for i in range(warmup):
        torch._int_mm(a, bs[i % copies])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        torch._int_mm(a, bs[i % copies])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    tops = 2.0 * m * n * k / us / 1e6
    return {"library": "hipBLASLt via torch._int_mm (int8 x int8 -> int32, no dequantisation)", "m": m, "n": n,
            "k": k, "us": round(us, 3), "TOPS": round(tops, 1), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
            "rotating_weight_copies": copies}


def measure_read_family(ctx, nbytes, steps, warmup, pattern=None):
    """The read rate of kernels that only stream nbytes (the read-only family of
    libaq_bench.so, a measurement aid outside the product library), each over
    enough rotating buffers to exceed the Infinity Cache and timed like the
    matvec.  The fastest member is the practical ceiling for a single launch
    of that many bytes on this GPU.  pattern = (rows, groups): also time
    loads-only kernels in the Q4_K row-per-lane matvec's own access pattern
    (56-row chunks, a wavefront per group) over that weight's bytes, and
    variants of it (workgroup size, pieces in flight, chunk-major storage),
    reported under "matvec_pattern"."""
    import ctypes

    from arm_ai_amd import hip

    lib = ctypes.CDLL(os.path.join(ROOT, "arm_ai_amd", "libaq_bench.so"))
    lib.aq_bench_read_name.restype = ctypes.c_char_p
    lib.aq_bench_read_name.argtypes = [ctypes.c_int]
    lib.aq_bench_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    nbytes = nbytes // 16 * 16
    copies = copies_for(nbytes)
    bufs = [hip.DeviceBuffer(nbytes) for _ in range(copies)]  # contents do not matter to a read
    out = hip.DeviceBuffer(4 * 1024)
    members = []
    for mb in range(lib.aq_bench_read_members()):
        fn = lambda i, mb=mb: lib.aq_bench_read(mb, ctx.stream, bufs[i % copies].ptr, nbytes, out.ptr)
        assert fn(0) == 0
        ms, _ = time_graph(ctx, fn, steps, warmup)
        gbps = nbytes / (ms / 1e3) / 1e9
        members.append({"kernel": lib.aq_bench_read_name(mb).decode(), "us": round(ms * 1e3, 3),
                        "GBps": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBS, 4)})
    best = min(members, key=lambda r: r["us"])
    res = {"kernel": best["kernel"], "bytes": nbytes, "us": best["us"], "GBps": best["GBps"],
           "frac_hbm": best["frac_hbm"], "rotating_copies": copies, "family": members}
    if pattern is not None:
        rows, ng = pattern
        wbytes = rows * ng * 144
        assert wbytes <= nbytes
        lib.aq_bench_read_pattern_name.restype = ctypes.c_char_p
        lib.aq_bench_read_pattern_name.argtypes = [ctypes.c_int]
        lib.aq_bench_read_pattern.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_void_p]
        pats = []
        for v in range(lib.aq_bench_read_patterns()):
            fn = lambda i, v=v: lib.aq_bench_read_pattern(v, ctx.stream, bufs[i % copies].ptr, rows, ng, out.ptr)
            assert fn(0) == 0
            ms, _ = time_graph(ctx, fn, steps, warmup)
            gbps = wbytes / (ms / 1e3) / 1e9
            pats.append({"kernel": lib.aq_bench_read_pattern_name(v).decode(), "bytes": wbytes,
                         "us": round(ms * 1e3, 3), "GBps": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBS, 4)})
        res["matvec_pattern"] = pats
    return res


def measure_mfma_rates(ctx):
    """The rate the matrix cores sustain for the GEMMs' MFMA shapes in a
    register-only loop (libaq_bench.so, k_mfma.hip): 1024 workgroups of four
    wavefronts, four independent accumulator chains each, one launch of a few
    ms timed with HIP events on the context's stream."""
    import ctypes

    from arm_ai_amd import hip

    lib = ctypes.CDLL(os.path.join(ROOT, "arm_ai_amd", "libaq_bench.so"))
    lib.aq_bench_mfma.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.aq_bench_mfma_macs.restype = ctypes.c_longlong
    grid, iters = 1024, 20000
    out = hip.DeviceBuffer(grid * 256 * 4)
    rows = {}
    for kind, name, peak in ((0, "v_mfma_i32_32x32x32_i8", INT8_PEAK_TOPS), (1, "v_mfma_i32_16x16x64_i8", INT8_PEAK_TOPS),
                             (2, "v_mfma_f32_32x32x16_f16", F16_PEAK_TFLOPS)):
        assert lib.aq_bench_mfma(kind, ctx.stream, grid, iters, out.ptr) == 0  # warm-up
        e0, e1 = hip.Event(), hip.Event()
        e0.record(ctx.stream)
        assert lib.aq_bench_mfma(kind, ctx.stream, grid, iters, out.ptr) == 0
        e1.record(ctx.stream)
        e1.synchronize()
        ms = e0.elapsed_ms(e1)
        ops = 2.0 * lib.aq_bench_mfma_macs(kind) * 4 * iters * grid * 4  # 4 wavefronts, 4 chains
        tops = ops / (ms / 1e3) / 1e12
        rows[name] = {"TOPS": round(tops, 1), "frac_of_published_peak": round(tops / peak, 4), "ms": round(ms, 3)}
    out.close()
    rows["coexec_i8_random_operands"] = measure_coexec(ctx)
    rows["coexec_f16_random_operands"] = measure_coexec(ctx, f16=True)
    return rows


def measure_coexec(ctx, f16=False):
    """What VALU work costs next to v_mfma_i32_32x32x32_i8 (f16: next to
    v_mfma_f32_32x32x16_f16 on integer values as a Q4_K GEMM without the
    scale split would feed it) (libaq_bench.so, k_mfma.hip coexec_loop): two
    wavefronts per SIMD, four accumulator chains each on random operands,
    each MFMA followed by nv independent f32 fmas; time per MFMA per SIMD for
    nv = 0, 4, 8, 16.  The slope is the time each VALU instruction adds, i.e.
    how much of it the matrix core does not hide."""
    import ctypes

    from arm_ai_amd import hip

    lib = ctypes.CDLL(os.path.join(ROOT, "arm_ai_amd", "libaq_bench.so"))
    fn = lib.aq_bench_coexec_f16 if f16 else lib.aq_bench_coexec
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    rng = np.random.default_rng(1)
    src = hip.to_device(rng.integers(-2**31, 2**31 - 1, size=8192, dtype=np.int64).astype(np.int32))
    out = hip.DeviceBuffer(512 * 256 * 4)
    iters = 2000
    ns = {}
    for nv in (0, 4, 8, 16):
        assert fn(nv, ctx.stream, 50, src.ptr, out.ptr) == 0  # warm-up
        e0, e1 = hip.Event(), hip.Event()
        e0.record(ctx.stream)
        assert fn(nv, ctx.stream, iters, src.ptr, out.ptr) == 0
        e1.record(ctx.stream)
        e1.synchronize()
        ns[nv] = e0.elapsed_ms(e1) * 1e6 / (4 * iters * 2)  # 4 MFMAs per iteration, 2 wavefronts per SIMD
    out.close()
    src.close()
    slope = (ns[16] - ns[4]) / 12.0
    kk = 16 if f16 else 32  # the MFMA's k
    return {"ns_per_mfma_per_simd": {f"valu_per_mfma_{nv}": round(v, 3) for nv, v in ns.items()},
            "ns_per_valu_beyond_4": round(slope, 3),
            "mfma_TOPS_random_operands": round(2.0 * 32 * 32 * kk / (ns[0] * 1e-9) * 1024 / 1e12, 1)}


def measure_launch_floor(ctx):
    """The cost of one dependent kernel launch: a HIP graph of 200 launches of
    an empty kernel (libaq_bench.so, k_launch.hip) timed with HIP events, at
    one workgroup and at 256 (one per CU)."""
    import ctypes

    from arm_ai_amd import hip

    lib = ctypes.CDLL(os.path.join(ROOT, "arm_ai_amd", "libaq_bench.so"))
    lib.aq_bench_empty.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    out = hip.DeviceBuffer(4)
    rows = {}
    for grid in (1, 256):
        ms, _ = time_graph(ctx, lambda i: lib.aq_bench_empty(ctx.stream, grid, out.ptr), 200, 5)
        rows[f"grid_{grid}"] = {"us_per_launch": round(ms * 1e3, 3)}
    out.close()
    return rows


def run_decode_child(name, no_cpu=False):
    """Run a decode (or vendor reference) case in a child process: the driver's
    torch glue needs torch imported before this library is loaded (one HIP
    runtime per process)."""
    import subprocess

    cmd = [sys.executable, "-u", os.path.abspath(__file__), "--case", name] + (["--no-cpu"] if no_cpu else [])
    r = subprocess.run(cmd,
                       stdout=subprocess.PIPE, text=True, cwd=ROOT)
    if r.returncode != 0:
        raise RuntimeError(f"{name} failed in its child process (exit {r.returncode})")
    out = json.loads(r.stdout.strip().splitlines()[-1])
    out.pop("case", None)
    return out


def run_case(ctx, name, steps, warmup, with_cpu=False):
    if name in CRATE_CASES:
        out = measure_crate(ctx, *CRATE_CASES[name], steps, warmup)
        log(f"{name}: {out['us']} us ({out.get('GBps', out.get('TOPS'))} {'GB/s' if 'GBps' in out else 'TOPS'})")
        return out
    if name in VENDOR_CASES:
        out = measure_vendor_int8(*VENDOR_CASES[name], min(steps, 50), min(warmup, 5))
        log(f"{name}: {out['us']} us ({out['TOPS']} TOPS, {out['frac_int8_peak']} of int8 peak)")
        return out
    if name in DECODE_CASES:
        model_name, n_prompt, n_new, seed = DECODE_CASES[name]
        out = measure_decode(ctx, model_name, n_prompt, n_new, seed, with_cpu=with_cpu)
        log(f"{name}: decode {out['decode_tok_s']} tok/s ({out['decode_ms_per_tok']} ms/tok; eager {out['eager_decode_tok_s']} tok/s), prefill {out['prefill_ms']} ms ({out['prefill_tok_s']} tok/s; warm {out['prefill_ms_warm']} ms)")
        return out
    if name in MATVEC_CASES:
        wt, n_, k_, m_, seed = MATVEC_CASES[name]
        w2, *_, out = measure(ctx, wt, n_, k_, m_, min(steps, 100), min(warmup, 10), seed)
        w2.free()
        log(f"{name}: step {out['step_us']} us ({out['step_GBps']} GB/s), pre-quantised matvec {out['matvec_us']} us ({out['matvec_GBps']} GB/s)")
        return out
    wt, n_, k_, m_, seed = PREFILL_CASES[name]
    out = measure_prefill(ctx, wt, n_, k_, m_, min(steps, 50), min(warmup, 5), seed, cpu=with_cpu and name.startswith("c3_"))
    log(f"{name}: step {out['step_us']} us ({out['step_TOPS']} TOPS), gemm {out['gemm_us']} us ({out['gemm_TOPS']} TOPS, {out['gemm_frac_int8_peak']} of int8 peak)")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-extra", action="store_true", help="skip the other configurations")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--case", default=None, help="run only this extra configuration and print its JSON")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run ten 64 MiB device-to-device copies (known-size kernel for PMC scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the quantized-matmul path runs on a single MI355X "
              "(it would shard by weight rows, one slice per GPU; not run here). Use --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        return 2

    if args.case in DECODE_CASES or args.case in VENDOR_CASES:
        import torch  # noqa: F401  (before the library: one HIP runtime per process)

    import arm_ai_amd as A

    if args.copy_calibration:
        from arm_ai_amd import hip

        nbytes = 64 << 20
        src, dst = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
        for _ in range(10):
            hip.check(hip.rt().hipMemcpy(dst.ptr, src.ptr, nbytes, hip.D2D), "D2D copy")
        hip.synchronize()
        print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 10}), flush=True)
        return 0

    all_cases = list(MATVEC_CASES) + list(PREFILL_CASES) + list(CRATE_CASES) + list(DECODE_CASES) + list(VENDOR_CASES)
    if args.case is not None and args.case not in all_cases:
        print(f"unknown case {args.case!r}; cases: {', '.join(all_cases)}", file=sys.stderr)
        return 2

    ctx = A.Context(0)
    log("context ready on device 0")
    if args.case is not None:
        out = run_case(ctx, args.case, args.steps, args.warmup, with_cpu=not args.no_cpu)
        ctx.close()
        print(json.dumps({"case": args.case, **out}), flush=True)
        return 0
    n, k, m = 14336, 4096, 1
    wl, step_ms, step_wall, kern_ms, head = measure(ctx, 12, n, k, m, args.steps, args.warmup, seed=4)
    log(f"headline: step {step_ms*1e3:.2f} us ({wl.step_bytes / step_ms / 1e6:.1f} GB/s), pre-quantised matvec {kern_ms*1e3:.2f} us ({head['matvec_GBps']} GB/s)")
    value = wl.step_bytes / (step_ms / 1e3) / 1e9
    achieved = value
    head_extra = {k2: head[k2] for k2 in ("matvec_us", "matvec_GBps", "matvec_frac_hbm")}
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b ffn_up Q4_K matvec, batch 1 (Q8_K quantise + matvec in one kernel)",
            "n": n, "k": k, "m": m, "weight_type": "Q4_K", "activation_type": "Q8_K",
            "rotating_weight_copies": wl.copies,
            "timing": "HIP graph of `steps` steps, events on the library stream",
            "wall_ms_per_step": round(step_wall, 6),
            "bytes_per_step": wl.step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profile(),
            "kernel": "rl_kernel<12, 56, 16, 1, 6, true, true, false, false, 0, false> (Q4_K, batch 1, one weight row per lane, Q8_K quantisation fused)",
            "bytes_per_launch": wl.step_bytes,
            "avg_launch_us": round(step_ms * 1e3, 3),
        },
    }
    ref = measure_read_family(ctx, wl.step_bytes, args.steps, args.warmup, pattern=(wl.n, wl.k // 256))
    log(f"fastest of {len(ref['family'])} read-only kernels on the same {ref['bytes']} bytes: {ref['kernel']}, {ref['us']} us ({ref['GBps']} GB/s, {ref['frac_hbm']} of peak)")
    result["roofline"]["read_only_reference"] = ref
    result["roofline"]["frac_of_read_only_reference"] = round(achieved / ref["GBps"], 4)
    if not args.no_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(wl)
        log(f"cpu baseline {result['cpu_baseline']['value']} GB/s")
        import oracle as O

        if O.cpu_has_v3():
            v3 = cpu_baseline(wl, isa="v3")
            log(f"cpu x86-64-v3 upper bound {v3['value']} GB/s")
        else:
            v3 = {"skipped": "this host CPU cannot run x86-64-v3 code"}
    wl.free()

    if not args.no_extra:
        extra = {}
        for name in MATVEC_CASES:
            extra[name] = run_case(ctx, name, args.steps, args.warmup)
        for name in PREFILL_CASES:
            extra[name] = run_case(ctx, name, args.steps, args.warmup, with_cpu=not args.no_cpu)
        for name in CRATE_CASES:
            extra[name] = run_case(ctx, name, args.steps, args.warmup)
        for name in DECODE_CASES:
            extra[name] = run_decode_child(name, no_cpu=args.no_cpu)
        for name in VENDOR_CASES:
            extra[name] = run_decode_child(name, no_cpu=True)
        extra["ref_mfma_rate"] = measure_mfma_rates(ctx)
        log(f"matrix cores, register-only loop: {extra['ref_mfma_rate']}")
        extra["ref_launch_floor"] = measure_launch_floor(ctx)
        log(f"dependent launch of an empty kernel in a graph: {extra['ref_launch_floor']}")
        result["extra"] = extra
    else:
        result["extra"] = {}
    result["extra"]["c4_q4k_14336x4096_b1_prequantised"] = head_extra
    if not args.no_cpu:
        result["extra"]["cpu_baseline_x86_64_v3"] = v3
    ctx.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
