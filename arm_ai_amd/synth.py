"""Seeded synthetic GGUF block data for the quantized-matmul hot path.

The reference publishes no fixture data for this path (its only model test
needs a downloaded TinyLlama GGUF, test/llama_candle_model_test.exs:2-4), so
every workload here is synthetic, with the value distributions the benchmark
configurations prescribe:

* Q4_K: d, dmin = f16(|N(0, 0.02)|); 6-bit scales and mins ~ U[0, 63];
  4-bit quants ~ U[0, 15].
* Q5_K: as Q4_K with 5-bit quants ~ U[0, 31].
* Q6_K: d = f16(|N(0, 0.02)|); int8 sub-scales ~ U[-32, 31]; 6-bit quants
  ~ U[0, 63] (value q - 32).
* Q8_0: d = f16(|N(0, 0.02)|); int8 quants ~ U[-127, 127].
* Q4_0: d = f16(|N(0, 0.02)|); 4-bit quants ~ U[0, 15] (value q - 8).
* Q5_0: d = f16(|N(0, 0.02)|); 5-bit quants ~ U[0, 31] (value q - 16).
* Q2_K: d, dmin = f16(|N(0, 0.02)|); 4-bit scales and mins ~ U[0, 15];
  2-bit quants ~ U[0, 3].
* Q3_K: d = f16(|N(0, 0.02)|); 6-bit scales ~ U[0, 63] (value s - 32);
  3-bit quants ~ U[-4, 3].
* activations: f32 N(0, 1).

Generators draw element-level arrays from ``numpy.random.default_rng(seed)``
(PCG64) and pack them into GGUF block bytes with the GGUF layout (block
formats: Q4_K 144 B, Q5_K 176 B, Q6_K 210 B, Q8_0 34 B, Q4_0 18 B, Q5_0 22 B,
Q2_K 84 B, Q3_K 110 B).  The element arrays are kept so
tests can compute exact answers without going through any unpacking code.
f32 -> f16 uses numpy's IEEE round-to-nearest-even conversion, the same
rounding the reference's `half` crate uses (shape_ops.rs:1492-1503).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

QK_K = 256
QK8_0 = 32
TYPE_Q4_0 = 2
TYPE_Q5_0 = 6
TYPE_Q8_0 = 8
TYPE_Q2_K = 10
TYPE_Q3_K = 11
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_Q8_K = 15

BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210, TYPE_Q8_0: 34, TYPE_Q4_0: 18, TYPE_Q5_0: 22, TYPE_Q2_K: 84,
               TYPE_Q3_K: 110, TYPE_Q8_K: 292}
BLOCK_ELEMS = {TYPE_Q4_K: QK_K, TYPE_Q5_K: QK_K, TYPE_Q6_K: QK_K, TYPE_Q8_0: QK8_0, TYPE_Q4_0: QK8_0,
               TYPE_Q5_0: QK8_0, TYPE_Q2_K: QK_K, TYPE_Q3_K: QK_K, TYPE_Q8_K: QK_K}
TYPE_NAMES = {TYPE_Q4_K: "q4_k", TYPE_Q5_K: "q5_k", TYPE_Q6_K: "q6_k", TYPE_Q8_0: "q8_0", TYPE_Q4_0: "q4_0",
              TYPE_Q5_0: "q5_0", TYPE_Q2_K: "q2_k", TYPE_Q3_K: "q3_k", TYPE_Q8_K: "q8_k"}


@dataclass
class QWeight:
    """A packed GGUF weight of `n` rows by `k` columns plus its element arrays."""

    type: int
    n: int
    k: int
    blocks: np.ndarray  # uint8 [n, nb * block_bytes], GGUF AoS layout
    d: np.ndarray  # float16 [n, nb]
    dmin: np.ndarray | None  # float16 [n, nb] (Q2_K, Q4_K, Q5_K)
    sc: np.ndarray | None  # Q4_K / Q5_K uint8 [n, nb, 8]; Q2_K uint8 [n, nb, 16]; Q3_K (value), Q6_K int8 [n, nb, 16]
    mn: np.ndarray | None  # Q4_K / Q5_K uint8 [n, nb, 8]; Q2_K uint8 [n, nb, 16]
    q: np.ndarray  # Q4_K uint8 [n,nb,256] in [0,15]; Q5_K in [0,31]; Q6_K int8 in [-32,31]; Q8_0 int8 [n,nb,32];
    #               Q4_0 uint8 [n,nb,32] in [0,15] (value q - 8); Q5_0 in [0,31] (value q - 16); Q2_K uint8 in [0,3]; Q3_K int8 in [-4,3]

    @property
    def nbytes(self) -> int:
        return int(self.blocks.nbytes)

    def dequantize(self) -> np.ndarray:
        """f64 [n, k] element values from the element arrays (GGML formulas)."""
        d = self.d.astype(np.float64)[..., None]
        if self.type in (TYPE_Q4_K, TYPE_Q5_K):
            sc = np.repeat(self.sc.astype(np.float64), 32, axis=-1)
            mn = np.repeat(self.mn.astype(np.float64), 32, axis=-1)
            v = d * sc * self.q.astype(np.float64) - self.dmin.astype(np.float64)[..., None] * mn
        elif self.type == TYPE_Q2_K:
            sc = np.repeat(self.sc.astype(np.float64), 16, axis=-1)
            mn = np.repeat(self.mn.astype(np.float64), 16, axis=-1)
            v = d * sc * self.q.astype(np.float64) - self.dmin.astype(np.float64)[..., None] * mn
        elif self.type in (TYPE_Q3_K, TYPE_Q6_K):
            sc = np.repeat(self.sc.astype(np.float64), 16, axis=-1)
            v = d * sc * self.q.astype(np.float64)
        elif self.type == TYPE_Q4_0:
            v = d * (self.q.astype(np.float64) - 8.0)
        elif self.type == TYPE_Q5_0:
            v = d * (self.q.astype(np.float64) - 16.0)
        else:
            v = d * self.q.astype(np.float64)
        return v.reshape(self.n, self.k)


def _half_abs_normal(rng: np.random.Generator, shape, sigma: float = 0.02) -> np.ndarray:
    return np.abs(rng.normal(0.0, sigma, size=shape)).astype(np.float32).astype(np.float16)


def pack_q4k(d, dmin, sc, mn, q) -> np.ndarray:
    """Pack Q4_K element arrays into 144-byte blocks.

    6-bit scale/min packing (inverse of GGML's get_scale_min_k4), j < 4:
      s[j]   = sc[j] | (sc[j+4] >> 4) << 6
      s[j+4] = m[j]  | (m[j+4]  >> 4) << 6
      s[j+8] = (sc[j+4] & 15) | (m[j+4] & 15) << 4
    quants: qs[32c+l] = q[64c+l] | q[64c+32+l] << 4.
    """
    n, nb = d.shape
    out = np.empty((n, nb, 144), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    out[..., 2:4] = dmin.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    s = out[..., 4:16]
    s[..., 0:4] = sc[..., 0:4] | ((sc[..., 4:8] >> 4) << 6)
    s[..., 4:8] = mn[..., 0:4] | ((mn[..., 4:8] >> 4) << 6)
    s[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
    qq = q.astype(np.uint8).reshape(n, nb, 4, 2, 32)  # [c][lo/hi][l]
    out[..., 16:144] = (qq[..., 0, :] | (qq[..., 1, :] << 4)).reshape(n, nb, 128)
    return out.reshape(n, nb * 144)


def pack_q5k(d, dmin, sc, mn, q) -> np.ndarray:
    """Pack Q5_K element arrays (q in [0, 31]) into 176-byte blocks:
    d f16 @0, dmin f16 @2, the 12 scale/min bytes @4 packed as Q4_K's,
    qh @16: bit s of qh[l] = bit 4 of element 32s + l,
    qs @48: qs[32c+l] = (q[64c+l] & 15) | (q[64c+32+l] & 15) << 4.
    """
    n, nb = d.shape
    q = q.astype(np.uint8)
    q4 = pack_q4k(d, dmin, sc, mn, q & 15).reshape(n, nb, 144)
    out = np.empty((n, nb, 176), dtype=np.uint8)
    out[..., 0:16] = q4[..., 0:16]
    hb = ((q >> 4) & 1).reshape(n, nb, 8, 32)  # [sub-block s][l]
    qh = np.zeros((n, nb, 32), dtype=np.uint8)
    for s_ in range(8):
        qh |= hb[..., s_, :] << s_
    out[..., 16:48] = qh
    out[..., 48:176] = q4[..., 16:144]
    return out.reshape(n, nb * 176)


def pack_q6k(d, sc, q) -> np.ndarray:
    """Pack Q6_K element arrays (q in [-32, 31]) into 210-byte blocks.

    For half h, l < 32, u = q + 32:
      ql[64h+l]    = u[128h+l]    & 15 | (u[128h+64+l] & 15) << 4
      ql[64h+32+l] = u[128h+32+l] & 15 | (u[128h+96+l] & 15) << 4
      qh[32h+l]    = u[128h+l]>>4 | u[128h+32+l]>>4 << 2 | u[128h+64+l]>>4 << 4 | u[128h+96+l]>>4 << 6
    """
    n, nb = d.shape
    out = np.empty((n, nb, 210), dtype=np.uint8)
    u = (q.astype(np.int16) + 32).astype(np.uint8).reshape(n, nb, 2, 4, 32)  # [h][g][l]
    ql = out[..., 0:128].reshape(n, nb, 2, 2, 32)  # [h][first/second 32][l]
    ql[..., 0, :] = (u[..., 0, :] & 15) | ((u[..., 2, :] & 15) << 4)
    ql[..., 1, :] = (u[..., 1, :] & 15) | ((u[..., 3, :] & 15) << 4)
    qh = out[..., 128:192].reshape(n, nb, 2, 32)
    qh[...] = (u[..., 0, :] >> 4) | ((u[..., 1, :] >> 4) << 2) | ((u[..., 2, :] >> 4) << 4) | ((u[..., 3, :] >> 4) << 6)
    out[..., 192:208] = sc.astype(np.int8).view(np.uint8)
    out[..., 208:210] = d.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    return out.reshape(n, nb * 210)


def pack_q5_0(d, q) -> np.ndarray:
    """Pack Q5_0 element arrays (q in [0, 31]) into 22-byte blocks: f16 d @0,
    qh @2 (u32, bit e = bit 4 of element e), qs @6 with qs[j] = q[j] & 15 |
    (q[j + 16] & 15) << 4."""
    n, nb = d.shape
    out = np.empty((n, nb, 22), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    q = q.astype(np.uint32)
    qh = ((q >> 4) & 1) << np.arange(32, dtype=np.uint32)
    out[..., 2:6] = qh.sum(axis=-1, dtype=np.uint32).astype("<u4").view(np.uint8).reshape(n, nb, 4)
    out[..., 6:22] = ((q[..., 0:16] & 15) | ((q[..., 16:32] & 15) << 4)).astype(np.uint8)
    return out.reshape(n, nb * 22)


def pack_q2k(d, dmin, sc, mn, q) -> np.ndarray:
    """Pack Q2_K element arrays (sc, mn in [0, 15] per 16-element group, q in
    [0, 3]) into 84-byte blocks: scales[g] = sc[g] | mn[g] << 4 @0,
    qs @16 with qs[32hf + l] = sum_j q[128hf + 32j + l] << 2j, d f16 @80,
    dmin f16 @82."""
    n, nb = d.shape
    out = np.empty((n, nb, 84), dtype=np.uint8)
    out[..., 0:16] = (sc.astype(np.uint8) & 15) | ((mn.astype(np.uint8) & 15) << 4)
    qq = q.astype(np.uint8).reshape(n, nb, 2, 4, 32)  # [hf][j][l]
    qs = np.zeros((n, nb, 2, 32), dtype=np.uint8)
    for j in range(4):
        qs |= (qq[..., j, :] & 3) << (2 * j)
    out[..., 16:80] = qs.reshape(n, nb, 64)
    out[..., 80:82] = d.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    out[..., 82:84] = dmin.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    return out.reshape(n, nb * 84)


def pack_q3k(d, sc, q) -> np.ndarray:
    """Pack Q3_K element arrays (sc in [-32, 31] per 16-element group, q in
    [-4, 3]) into 110-byte blocks.  With u = q + 4: hmask @0, bit 4hf + j of
    hmask[l] = u[128hf + 32j + l] >> 2; qs @32, qs[32hf + l] = sum_j
    (u[128hf + 32j + l] & 3) << 2j; the 6-bit s = sc + 32 @96: byte i < 4 =
    s[i] & 15 | (s[8+i] & 15) << 4, byte 4 + i = s[4+i] & 15 | (s[12+i] & 15)
    << 4, byte 8 + i = s[i] >> 4 | s[4+i] >> 4 << 2 | s[8+i] >> 4 << 4 |
    s[12+i] >> 4 << 6; d f16 @108."""
    n, nb = d.shape
    out = np.empty((n, nb, 110), dtype=np.uint8)
    u = (q.astype(np.int16) + 4).astype(np.uint8).reshape(n, nb, 2, 4, 32)  # [hf][j][l]
    hm = np.zeros((n, nb, 32), dtype=np.uint8)
    qs = np.zeros((n, nb, 2, 32), dtype=np.uint8)
    for hf in range(2):
        for j in range(4):
            hm |= (u[..., hf, j, :] >> 2) << (4 * hf + j)
            qs[..., hf, :] |= (u[..., hf, j, :] & 3) << (2 * j)
    out[..., 0:32] = hm
    out[..., 32:96] = qs.reshape(n, nb, 64)
    s6 = (sc.astype(np.int16) + 32).astype(np.uint8)
    b = out[..., 96:108]
    b[..., 0:4] = (s6[..., 0:4] & 15) | ((s6[..., 8:12] & 15) << 4)
    b[..., 4:8] = (s6[..., 4:8] & 15) | ((s6[..., 12:16] & 15) << 4)
    b[..., 8:12] = (s6[..., 0:4] >> 4) | ((s6[..., 4:8] >> 4) << 2) | ((s6[..., 8:12] >> 4) << 4) | ((s6[..., 12:16] >> 4) << 6)
    out[..., 108:110] = d.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    return out.reshape(n, nb * 110)


def pack_q8_0(d, q) -> np.ndarray:
    n, nb = d.shape
    out = np.empty((n, nb, 34), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    out[..., 2:34] = q.astype(np.int8).view(np.uint8)
    return out.reshape(n, nb * 34)


def pack_q4_0(d, q) -> np.ndarray:
    """Pack Q4_0 element arrays (q in [0, 15]) into 18-byte blocks: f16 d @0,
    qs @2 with qs[j] = q[j] | q[j + 16] << 4."""
    n, nb = d.shape
    out = np.empty((n, nb, 18), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    q = q.astype(np.uint8)
    out[..., 2:18] = (q[..., 0:16] & 15) | ((q[..., 16:32] & 15) << 4)
    return out.reshape(n, nb * 18)


def make_weight(type_: int, n: int, k: int, seed: int = 0, rng: np.random.Generator | None = None) -> QWeight:
    """A seeded random weight of `n` rows by `k` columns in GGUF block format."""
    if rng is None:
        rng = np.random.default_rng(seed)
    blk = BLOCK_ELEMS[type_]
    if k % blk:
        raise ValueError(f"k={k} is not a multiple of the block size {blk}")
    nb = k // blk
    if type_ == TYPE_Q4_K:
        d = _half_abs_normal(rng, (n, nb))
        dmin = _half_abs_normal(rng, (n, nb))
        sc = rng.integers(0, 64, size=(n, nb, 8), dtype=np.uint8)
        mn = rng.integers(0, 64, size=(n, nb, 8), dtype=np.uint8)
        q = rng.integers(0, 16, size=(n, nb, 256), dtype=np.uint8)
        return QWeight(type_, n, k, pack_q4k(d, dmin, sc, mn, q), d, dmin, sc, mn, q)
    if type_ == TYPE_Q5_K:
        d = _half_abs_normal(rng, (n, nb))
        dmin = _half_abs_normal(rng, (n, nb))
        sc = rng.integers(0, 64, size=(n, nb, 8), dtype=np.uint8)
        mn = rng.integers(0, 64, size=(n, nb, 8), dtype=np.uint8)
        q = rng.integers(0, 32, size=(n, nb, 256), dtype=np.uint8)
        return QWeight(type_, n, k, pack_q5k(d, dmin, sc, mn, q), d, dmin, sc, mn, q)
    if type_ == TYPE_Q6_K:
        d = _half_abs_normal(rng, (n, nb))
        sc = rng.integers(-32, 32, size=(n, nb, 16), dtype=np.int8)
        q = (rng.integers(0, 64, size=(n, nb, 256), dtype=np.uint8).astype(np.int16) - 32).astype(np.int8)
        return QWeight(type_, n, k, pack_q6k(d, sc, q), d, None, sc, None, q)
    if type_ == TYPE_Q8_0:
        d = _half_abs_normal(rng, (n, nb))
        q = rng.integers(-127, 128, size=(n, nb, 32), dtype=np.int8)
        return QWeight(type_, n, k, pack_q8_0(d, q), d, None, None, None, q)
    if type_ == TYPE_Q4_0:
        d = _half_abs_normal(rng, (n, nb))
        q = rng.integers(0, 16, size=(n, nb, 32), dtype=np.uint8)
        return QWeight(type_, n, k, pack_q4_0(d, q), d, None, None, None, q)
    if type_ == TYPE_Q5_0:
        d = _half_abs_normal(rng, (n, nb))
        q = rng.integers(0, 32, size=(n, nb, 32), dtype=np.uint8)
        return QWeight(type_, n, k, pack_q5_0(d, q), d, None, None, None, q)
    if type_ == TYPE_Q2_K:
        d = _half_abs_normal(rng, (n, nb))
        dmin = _half_abs_normal(rng, (n, nb))
        sc = rng.integers(0, 16, size=(n, nb, 16), dtype=np.uint8)
        mn = rng.integers(0, 16, size=(n, nb, 16), dtype=np.uint8)
        q = rng.integers(0, 4, size=(n, nb, 256), dtype=np.uint8)
        return QWeight(type_, n, k, pack_q2k(d, dmin, sc, mn, q), d, dmin, sc, mn, q)
    if type_ == TYPE_Q3_K:
        d = _half_abs_normal(rng, (n, nb))
        sc = rng.integers(-32, 32, size=(n, nb, 16), dtype=np.int8)
        q = rng.integers(-4, 4, size=(n, nb, 256), dtype=np.int8)
        return QWeight(type_, n, k, pack_q3k(d, sc, q), d, None, sc, None, q)
    raise ValueError(f"unsupported weight type {type_}")


def make_weight_unit(type_: int, n: int, k: int, seed: int = 0, rng: np.random.Generator | None = None) -> QWeight:
    """A random weight whose dequantised values have mean about 0 and standard
    deviation about 1/sqrt(k), so a stack of layers keeps activations of order
    one (the block distributions of make_weight give every element a mean of
    about +3, which saturates a deep model).  Same block formats:

    * Q4_K / Q5_K: sub-block scales sc ~ U[1, 8], mins m = round(sc * mid) with
      mid the centre of the quant range (7.5 or 15.5; m <= 63 for Q4_K, Q5_K
      uses sc ~ U[1, 4]), dmin = d, so a value d*sc*q - dmin*m is centred on
      zero; d = f16(U[0.5, 1.5] / (sqrt(k) * rms(sc) * std(q))).
    * Q6_K: sub-scales ~ U[-8, 8] without 0, q6 ~ U[0, 63] (value q - 32),
      d = f16(U[0.5, 1.5] / (sqrt(k) * rms(sc) * std(q))).
    * Q3_K: sub-scales +-U[1, 8], q3 ~ U[-4, 3]; Q2_K: sc ~ U[1, 8],
      m = round(1.5 sc), dmin = d; Q8_0, Q4_0, Q5_0: d * (q - centre) with d
      scaled the same way."""
    if rng is None:
        rng = np.random.default_rng(seed)
    if type_ in (TYPE_Q8_0, TYPE_Q4_0, TYPE_Q5_0):  # value d * (q - centre), blocks of 32
        if k % QK8_0:
            raise ValueError(f"k={k} is not a multiple of {QK8_0}")
        nb = k // QK8_0
        spread = rng.uniform(0.5, 1.5, size=(n, nb))
        if type_ == TYPE_Q8_0:
            q = rng.integers(-127, 128, size=(n, nb, 32), dtype=np.int8)
            std_q, pack = np.sqrt((255 * 255 - 1) / 12.0), pack_q8_0
        else:
            top = 16 if type_ == TYPE_Q4_0 else 32
            q = rng.integers(0, top, size=(n, nb, 32), dtype=np.uint8)
            std_q, pack = np.sqrt((top * top - 1) / 12.0), (pack_q4_0 if top == 16 else pack_q5_0)
        d = (spread / (np.sqrt(k) * std_q)).astype(np.float32).astype(np.float16)
        return QWeight(type_, n, k, pack(d, q), d, None, None, None, q)
    if k % QK_K:
        raise ValueError(f"k={k} is not a multiple of {QK_K}")
    nb = k // QK_K
    spread = rng.uniform(0.5, 1.5, size=(n, nb))
    if type_ in (TYPE_Q4_K, TYPE_Q5_K):
        five = type_ == TYPE_Q5_K
        top = 32 if five else 16
        smax = 4 if five else 8
        sc = rng.integers(1, smax + 1, size=(n, nb, 8), dtype=np.uint8)
        mn = np.minimum(np.rint(sc.astype(np.float64) * (top - 1) / 2.0), 63).astype(np.uint8)
        q = rng.integers(0, top, size=(n, nb, 256), dtype=np.uint8)
        rms_sc = np.sqrt(np.mean(np.arange(1, smax + 1) ** 2))
        std_q = np.sqrt((top * top - 1) / 12.0)
        d = (spread / (np.sqrt(k) * rms_sc * std_q)).astype(np.float32).astype(np.float16)
        pack = pack_q5k if five else pack_q4k
        return QWeight(type_, n, k, pack(d, d, sc, mn, q), d, d.copy(), sc, mn, q)
    if type_ == TYPE_Q6_K:
        mag = rng.integers(1, 9, size=(n, nb, 16))
        sc = (mag * np.where(rng.integers(0, 2, size=mag.shape) == 1, 1, -1)).astype(np.int8)
        q = (rng.integers(0, 64, size=(n, nb, 256), dtype=np.uint8).astype(np.int16) - 32).astype(np.int8)
        rms_sc = np.sqrt(np.mean(np.arange(1, 9) ** 2))
        std_q = np.sqrt((64 * 64 - 1) / 12.0)
        d = (spread / (np.sqrt(k) * rms_sc * std_q)).astype(np.float32).astype(np.float16)
        return QWeight(type_, n, k, pack_q6k(d, sc, q), d, None, sc, None, q)
    if type_ == TYPE_Q3_K:  # value d * sc * q, sc = +-U[1, 8], q ~ U[-4, 3]
        mag = rng.integers(1, 9, size=(n, nb, 16))
        sc = (mag * np.where(rng.integers(0, 2, size=mag.shape) == 1, 1, -1)).astype(np.int8)
        q = rng.integers(-4, 4, size=(n, nb, 256), dtype=np.int8)
        d = (spread / (np.sqrt(k) * np.sqrt(np.mean(np.arange(1, 9) ** 2)) * np.sqrt(5.25))).astype(np.float32).astype(np.float16)
        return QWeight(type_, n, k, pack_q3k(d, sc, q), d, None, sc, None, q)
    if type_ == TYPE_Q2_K:  # value d * sc * q - dmin * m, sc ~ U[1, 8], m = round(1.5 sc), dmin = d
        sc = rng.integers(1, 9, size=(n, nb, 16), dtype=np.uint8)
        mn = np.rint(sc.astype(np.float64) * 1.5).astype(np.uint8)
        q = rng.integers(0, 4, size=(n, nb, 256), dtype=np.uint8)
        d = (spread / (np.sqrt(k) * np.sqrt(np.mean(np.arange(1, 9) ** 2)) * np.sqrt(1.25))).astype(np.float32).astype(np.float16)
        return QWeight(type_, n, k, pack_q2k(d, d, sc, mn, q), d, d.copy(), sc, mn, q)
    raise ValueError(f"make_weight_unit has no distribution for type {type_}")


def make_activation(m: int, k: int, seed: int = 0, rng: np.random.Generator | None = None) -> np.ndarray:
    """f32 [m, k] drawn from N(0, 1)."""
    if rng is None:
        rng = np.random.default_rng(seed)
    return rng.standard_normal(size=(m, k), dtype=np.float32)


def weight_bytes(type_: int, n: int, k: int) -> int:
    return n * (k // BLOCK_ELEMS[type_]) * BLOCK_BYTES[type_]


def act_bytes(type_: int, m: int, k: int) -> int:
    """Bytes of the quantised activation a weight of `type_` is dotted with."""
    if type_ in (TYPE_Q8_0, TYPE_Q4_0, TYPE_Q5_0):
        return m * (k // QK8_0) * 34
    return m * (k // QK_K) * 292
