"""Error measures used by the parity tests.

The GPU kernels compute every integer block sum exactly and differ from
candle's `vec_dot_unopt` only in the order of the f32 combination.  With
N(0, 1) activations some outputs are close to zero, so a plain per-element
relative error is ill-conditioned (it is unbounded for any change of
summation order).  Two measures are used instead, both gated at the
tolerance the task fixes (1e-5, or 1e-4 for K >= 14336):

* ``rel_max``  = max_i |y_i - r_i| / max_i |r_i|   (norm-wise relative error)
* ``rel_cond`` = max_i |y_i - r_i| / D_i, with D_i = sum_e |w_e| |x_e| taken
  over the two halves of each dequantised weight (|d*sc*q| + |dmin*m|), i.e.
  the error relative to the magnitude of the terms being summed -- the
  quantity any reordering of an f32 sum is bounded by.
"""
from __future__ import annotations

import numpy as np


def tol_for_k(k: int) -> float:
    return 1e-4 if k >= 14336 else 1e-5


def rel_max(y: np.ndarray, r: np.ndarray) -> float:
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    den = np.abs(r).max()
    return float(np.abs(y - r).max() / den) if den > 0 else float(np.abs(y - r).max())


def abs_weight_magnitude(W) -> np.ndarray:
    """f32 [n, k]: |d*sc*q| + |dmin*m| per element, from the generator's element arrays."""
    d = np.abs(W.d.astype(np.float32))[..., None]
    if W.dmin is not None:
        per = W.k // W.d.shape[1] // W.sc.shape[-1]  # elements per scale: 32 (Q4_K, Q5_K) or 16 (Q2_K)
        sc = np.repeat(W.sc.astype(np.float32), per, axis=-1)
        mn = np.repeat(W.mn.astype(np.float32), per, axis=-1)
        v = d * sc * W.q.astype(np.float32) + np.abs(W.dmin.astype(np.float32))[..., None] * mn
    elif W.sc is not None:
        sc = np.repeat(np.abs(W.sc.astype(np.float32)), 16, axis=-1)
        v = d * sc * np.abs(W.q.astype(np.float32))
    else:
        v = d * np.abs(W.q.astype(np.float32))
    return v.reshape(W.n, W.k)


def rel_cond(y: np.ndarray, r: np.ndarray, W, xdeq_abs: np.ndarray) -> float:
    """xdeq_abs: f32 [m, k] = |d_x * q_x| of the quantised activation."""
    D = xdeq_abs.astype(np.float32) @ abs_weight_magnitude(W).T  # [m, n]
    D = np.maximum(D.astype(np.float64), np.finfo(np.float32).tiny)
    return float((np.abs(np.asarray(y, np.float64) - np.asarray(r, np.float64)) / D).max())
