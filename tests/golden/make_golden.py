"""Writes tests/golden/golden.npz: small known-answer vectors for the hot path.

The reference holds no golden vectors for its quantized matmul (its only
model test needs a network download), so these vectors are made here, by two
implementations that share no code:

  * this script's own numpy restatement of the GGUF block formats (the
    public GGML layouts of Q4_K, Q6_K, Q8_0, Q8_K), of candle-core 0.8.4's
    activation quantizers (BlockQ8K::from_float, BlockQ8_0::from_float) and
    of the crate's quantizers (shape_ops.rs:1273-1292, :2936-2954,
    :3242-3275), written from those descriptions with element-by-element
    loops;
  * the C oracle (oracle/), a separate restatement.

The script refuses to write unless both agree bit for bit on every integer
and byte output; the f32 matmul outputs are the oracle's (candle's
vec_dot_unopt order).  Tests compare the oracle and the GPU library with the
stored vectors (tests/test_golden.py).  Inputs are seeded and include the
edge cases the quantizers branch on (all-zero blocks, ties at .5, the
first-maximum rule, NaN, f32 subnormals, saturation).

Run from the repository root:  python tests/golden/make_golden.py
"""
import math
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402
from arm_ai_amd import synth as S  # noqa: E402

OUT = os.path.join(HERE, "golden.npz")
F32 = np.float32


# ----------------------------------------------------------- scalar helpers
def round_away(v: float) -> float:
    """Rust f32::round: half away from zero (exact for |v| < 2^23)."""
    if v != v:
        return v
    a = abs(v)
    r = math.floor(a)
    if a - r >= 0.5:
        r += 1.0
    return math.copysign(r, v)


def sat_int(v: float, lo: int, hi: int) -> int:
    """Rust `v as iN` for a float: NaN -> 0, saturating at the type's range."""
    if v != v:
        return 0
    return int(max(lo, min(hi, math.trunc(v))))


def f16_bits(v) -> int:
    return int(np.array([v], np.float32).astype(np.float16).view(np.uint16)[0])


def f16_val(bits: int) -> float:
    return float(np.array([bits], np.uint16).view(np.float16)[0])


# ------------------------------------------------- activation quantizers
def q8k_block(x: np.ndarray) -> bytes:
    """candle BlockQ8K::from_float on 256 f32 values."""
    amax, mx = F32(0.0), F32(0.0)
    for v in x:
        a = F32(abs(v))
        if amax < a:  # first element of largest |x|; NaN never compares greater
            amax, mx = a, v
    if amax == 0:
        d, q = F32(0.0), [0] * 256
    else:
        iscale = F32(F32(-128.0) / mx)
        q = []
        for v in x:
            t = round_away(float(F32(iscale * v)))
            t = 127.0 if t != t else min(t, 127.0)  # f32::min returns the non-NaN operand
            q.append(sat_int(t, -128, 127))
        d = F32(F32(1.0) / iscale)
    bsums = [sum(q[16 * g:16 * g + 16]) for g in range(16)]
    return struct.pack("<f", d) + bytes(np.array(q, np.int8).view(np.uint8)) + struct.pack("<16h", *bsums)


def q8_0_block(x: np.ndarray) -> bytes:
    """candle BlockQ8_0::from_float on 32 f32 values (d stored as f16, RNE)."""
    amax = F32(0.0)
    for v in x:
        a = F32(abs(v))
        if a == a and a > amax:  # f32::max ignores a NaN operand
            amax = a
    d = F32(amax / F32(127.0))
    iv = F32(1.0) / d if d != 0 else F32(0.0)
    q = [sat_int(round_away(float(F32(v * iv))), -128, 127) for v in x]
    return struct.pack("<H", f16_bits(d)) + bytes(np.array(q, np.int8).view(np.uint8))


def quantize_rows(x: np.ndarray, block) -> np.ndarray:
    n = 256 if block is q8k_block else 32
    out = b"".join(block(row[i:i + n]) for row in x for i in range(0, x.shape[1], n))
    return np.frombuffer(out, np.uint8).copy()


# ------------------------------------------------------- weight decoding
def q4k_fields(blk: bytes):
    """GGML block_q4_K: d, dmin (f16), 12 bytes of 6-bit scales/mins, 128 qs."""
    d, dmin = f16_val(blk[0] | blk[1] << 8), f16_val(blk[2] | blk[3] << 8)
    sb = blk[4:16]
    sc, mn = [], []
    for j in range(8):  # get_scale_min_k4
        if j < 4:
            sc.append(sb[j] & 63)
            mn.append(sb[j + 4] & 63)
        else:
            sc.append((sb[j + 4] & 0xF) | ((sb[j - 4] >> 6) << 4))
            mn.append((sb[j + 4] >> 4) | ((sb[j] >> 6) << 4))
    qs = blk[16:144]
    q = [0] * 256
    for c in range(4):
        for i in range(32):
            q[64 * c + i] = qs[32 * c + i] & 0xF
            q[64 * c + 32 + i] = qs[32 * c + i] >> 4
    return d, dmin, sc, mn, q


def q6k_fields(blk: bytes):
    """GGML block_q6_K: ql[128], qh[64], int8 scales[16], d (f16); q in [-32, 31]."""
    ql, qh = blk[0:128], blk[128:192]
    sc = list(np.frombuffer(blk[192:208], np.int8).astype(int))
    d = f16_val(blk[208] | blk[209] << 8)
    q = [0] * 256
    for h in range(2):
        for i in range(32):
            a, b, hb = ql[64 * h + i], ql[64 * h + 32 + i], qh[32 * h + i]
            q[128 * h + i] = ((a & 0xF) | ((hb & 3) << 4)) - 32
            q[128 * h + 32 + i] = ((b & 0xF) | (((hb >> 2) & 3) << 4)) - 32
            q[128 * h + 64 + i] = ((a >> 4) | (((hb >> 4) & 3) << 4)) - 32
            q[128 * h + 96 + i] = ((b >> 4) | (((hb >> 6) & 3) << 4)) - 32
    return d, sc, q


def block_sums(wtype: int, w: np.ndarray, n: int, k: int, xq: np.ndarray, m: int):
    """Integer parts of every (row of x, weight row, block) product:
    Q4_K: S = sum_j sc_j * sum_32 q*x, Smin = sum_g bsums[g] * m[g/2];
    Q6_K: S = sum_j sc_j * sum_16 q*x (q - 32 included), Smin = 0;
    Q8_0: S = sum_32 qw*qx, Smin = 0."""
    wb, bb = O.BLOCK_BYTES[wtype], O.BLOCK_ELEMS[wtype]
    nblk = k // bb
    w = w.reshape(n, nblk * wb)
    xq = xq.reshape(m, -1)
    S = np.zeros((m, n, nblk), np.int32)
    Sm = np.zeros((m, n, nblk), np.int32)
    for r in range(m):
        if wtype == O.Q8_0:
            xs = [np.frombuffer(bytes(xq[r, 34 * b + 2:34 * b + 34]), np.int8).astype(int) for b in range(nblk)]
        else:
            xs = [np.frombuffer(bytes(xq[r, 292 * b + 4:292 * b + 260]), np.int8).astype(int) for b in range(nblk)]
            bs = [np.frombuffer(bytes(xq[r, 292 * b + 260:292 * b + 292]), np.int16).astype(int) for b in range(nblk)]
        for j in range(n):
            for b in range(nblk):
                blk = bytes(w[j, wb * b:wb * (b + 1)])
                if wtype == O.Q4_K:
                    _, _, sc, mn, q = q4k_fields(blk)
                    S[r, j, b] = sum(sc[s] * int(np.dot(q[32 * s:32 * s + 32], xs[b][32 * s:32 * s + 32])) for s in range(8))
                    Sm[r, j, b] = sum(int(bs[b][g]) * mn[g // 2] for g in range(16))
                elif wtype == O.Q6_K:
                    _, sc, q = q6k_fields(blk)
                    S[r, j, b] = sum(sc[s] * int(np.dot(q[16 * s:16 * s + 16], xs[b][16 * s:16 * s + 16])) for s in range(16))
                else:
                    qw = np.frombuffer(blk[2:34], np.int8).astype(int)
                    S[r, j, b] = int(np.dot(qw, xs[b]))
    return S, Sm


# --------------------------------------------------- crate quantizers
def crate_int8_per_token(x: np.ndarray):
    q = np.zeros(x.shape, np.int8)
    sc = np.zeros(x.shape[0], np.float32)
    for i, row in enumerate(x):
        mx = F32(0.0)
        for v in row:
            a = F32(abs(v))
            if a == a and a > mx:
                mx = a
        s = F32(mx / F32(127.0)) if mx > 0 else F32(1.0)
        sc[i] = s
        for jj, v in enumerate(row):
            q[i, jj] = max(-127, min(127, sat_int(round_away(float(F32(v / s))), -2**31, 2**31 - 1)))
    return q, sc


def crate_q8_groups(a: np.ndarray):
    q = np.zeros(a.shape, np.int8)
    sc = np.zeros(a.size // 32, np.float32)
    for g in range(a.size // 32):
        grp = a[32 * g:32 * g + 32]
        mx = F32(0.0)
        for v in grp:
            if F32(abs(v)) > mx:
                mx = F32(abs(v))
        s = F32(mx / F32(127.0)) if mx > 0 else F32(1.0)
        sc[g] = s
        inv = F32(F32(1.0) / s)
        for i, v in enumerate(grp):
            t = round_away(float(F32(v * inv)))
            q[32 * g + i] = 0 if t != t else int(max(-128.0, min(127.0, t)))
    return q, sc


def crate_q4_0(w: np.ndarray):
    n, k = w.shape
    packed = np.zeros((n, k // 2), np.uint8)
    sc = np.zeros((n, k // 32), np.float32)
    for i in range(n):
        for g in range(k // 32):
            grp = w[i, 32 * g:32 * g + 32]
            mx = F32(0.0)
            for v in grp:
                a = F32(abs(v))
                if a == a and a > mx:
                    mx = a
            s = F32(mx / F32(7.0)) if mx > 0 else F32(1.0)
            sc[i, g] = s
            qv = [max(-8, min(7, sat_int(round_away(float(F32(v / s))), -2**31, 2**31 - 1))) + 8 for v in grp]
            for jj in range(16):
                packed[i, 16 * g + jj] = (qv[2 * jj + 1] << 4) | qv[2 * jj]
    return packed, sc


# ------------------------------------------------------------------ inputs
def act_rows(k: int, rng) -> np.ndarray:
    rows = [rng.standard_normal(k).astype(np.float32), np.zeros(k, np.float32)]
    r = np.zeros(k, np.float32)
    r[:8] = [127.0, -63.5, 0.5, 2.5, -2.5, 1.49, -126.5, 3.0]
    r[8] = -127.0  # same |x| as r[0], later: r[0] stays the first maximum
    rows.append(r)
    r = rng.standard_normal(k).astype(np.float32) * 1e3
    r[3] = np.nan
    r[300 % k] = np.float32(1e-40)
    rows.append(r)
    r = np.full(k, -2.0, np.float32)  # every element equal: the first is the maximum
    r[::7] = np.float32(1e-39)
    rows.append(r)
    return np.stack(rows)


def main():
    rng = np.random.default_rng(20240607)
    data = {}
    k = 512
    x = act_rows(k, rng)
    data["act_x"] = x
    data["act_q8k"] = quantize_rows(x, q8k_block)
    data["act_q8_0"] = quantize_rows(x, q8_0_block)
    assert np.array_equal(data["act_q8k"], O.quantize(x, O.Q8_K).reshape(-1)), "Q8_K quantizer disagrees"
    assert np.array_equal(data["act_q8_0"], O.quantize(x, O.Q8_0).reshape(-1)), "Q8_0 quantizer disagrees"

    for name, wtype in (("q4k", O.Q4_K), ("q6k", O.Q6_K), ("q8_0", O.Q8_0)):
        n, m = 20, 3
        W = S.make_weight(wtype, n, k, seed=wtype)
        xm = x[[0, 2, 3]]
        xq = O.quantize(xm, O.act_type(wtype))
        Sg, Smg = block_sums(wtype, W.blocks, n, k, xq, m)
        So, Smo = O.block_sums(wtype, k, W.blocks, xq)
        assert np.array_equal(Sg, So) and np.array_equal(Smg, Smo), f"{name}: block sums disagree"
        data[f"{name}_w"] = np.asarray(W.blocks, np.uint8).reshape(-1)
        data[f"{name}_x"] = xm
        data[f"{name}_S"] = Sg
        data[f"{name}_Smin"] = Smg
        data[f"{name}_y"] = O.matmul_preq(wtype, xq, W.blocks, n, k)

    a = x[[0, 2, 3], :100].copy()
    q, sc = crate_int8_per_token(a)
    qo, sco = O.quantize_int8_per_token(a, 3, 100)
    assert np.array_equal(q, qo) and np.array_equal(sc, sco), "int8 per-token quantizer disagrees"
    data["crate_i8_x"], data["crate_i8_q"], data["crate_i8_s"] = a, q, sc

    g = x[[0, 2, 3]].reshape(-1)[:256].copy()
    g[64:96] = 0.0
    q, sc = crate_q8_groups(g)
    qo, sco = O.quantize_q8_groups(g, 256)
    assert np.array_equal(q, qo) and np.array_equal(sc, sco), "q8 group quantizer disagrees"
    data["crate_q8g_x"], data["crate_q8g_q"], data["crate_q8g_s"] = g, q, sc

    w4 = (rng.standard_normal((4, 64)) * 3).astype(np.float32)
    w4[1, :8] = [7.0, -7.0, 3.5, -3.5, 0.5, -0.5, 2.49, 6.51]
    w4[1, 8:32] = 0.0
    w4[2, 32:] = 0.0
    p4, s4 = crate_q4_0(w4)
    po, so = O.quantize_int4_q4_0(w4, 4, 64)
    assert np.array_equal(p4, po) and np.array_equal(s4, so), "Q4_0 quantizer disagrees"
    data["crate_q4_x"], data["crate_q4_p"], data["crate_q4_s"] = w4, p4, s4

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: {len(data)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
