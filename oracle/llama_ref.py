"""CPU restatement of candle-transformers 0.8.4 quantized_llama's forward:
numpy f32 for the glue, the oracle's k_quants::matmul for every quantized
projection.  Test infrastructure only (the driver tests' reference, and the
CPU decode baseline bench.py times beside the GPU's).

Follows the call sequence the reference reaches from
native/arm_ai_nif/src/llama_candle.rs:93 (prefill) and :119 (decode); candle's
source is not in the container, so the glue semantics (rope_i pairing,
repeat_kv grouping, causal mask j > i, rms_norm, silu) are restated, not
pinned against candle itself.
"""
from __future__ import annotations

import numpy as np

import oracle as O


class RefLlama:
    def __init__(self, hw):
        self.hw = hw
        cfg = hw.cfg
        self.cfg = cfg
        hd = cfg.hidden // cfg.n_head
        self.hd = hd
        inv = np.float32(1.0) / (np.float32(cfg.rope_theta) ** (np.arange(0, hd, 2, dtype=np.float32) / np.float32(hd)))
        ang = np.arange(cfg.max_seq, dtype=np.float32)[:, None] * inv[None, :].astype(np.float32)
        self.cos, self.sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        self.k = [np.zeros((cfg.n_kv_head, 0, hd), np.float32) for _ in range(cfg.n_layer)]
        self.v = [np.zeros((cfg.n_kv_head, 0, hd), np.float32) for _ in range(cfg.n_layer)]

    def mm(self, qt, x):
        n, k = qt.shape
        return O.matmul(int(qt.dtype), np.ascontiguousarray(x, np.float32), qt.data, n, k).astype(np.float32)

    def rms(self, x, w):
        eps = np.float32(self.cfg.rms_eps)
        ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
        return (x / np.sqrt(ms + eps)) * w

    def rope(self, x, pos0):
        # x [L, H, D]; pairs (2i, 2i+1) rotated by angle pos * theta_i
        L, H, D = x.shape
        c = self.cos[pos0:pos0 + L][:, None, :]
        s = self.sin[pos0:pos0 + L][:, None, :]
        a, b = x[..., 0::2], x[..., 1::2]
        out = np.empty_like(x)
        out[..., 0::2] = a * c - b * s
        out[..., 1::2] = a * s + b * c
        return out

    def embed(self, tokens, index_pos):
        tokens = np.asarray(tokens, np.int64)
        if index_pos == 0:
            cfg, hd = self.cfg, self.hd
            self.k = [np.zeros((cfg.n_kv_head, 0, hd), np.float32) for _ in range(cfg.n_layer)]
            self.v = [np.zeros((cfg.n_kv_head, 0, hd), np.float32) for _ in range(cfg.n_layer)]
        return self.hw.tok_embeddings[tokens].astype(np.float32)

    def layer(self, li, x, index_pos):
        """Layer li on the residual stream x [L, hidden] at positions index_pos..;
        appends the layer's k, v to its cache and returns the new residual stream."""
        cfg, hw, hd = self.cfg, self.hw, self.hd
        L = x.shape[0]
        H, Hkv = cfg.n_head, cfg.n_kv_head
        lw = hw.layers[li]
        n = self.rms(x, hw.attn_norm[li])
        q = self.rope(self.mm(lw["wq"], n).reshape(L, H, hd), index_pos).transpose(1, 0, 2)
        k = self.rope(self.mm(lw["wk"], n).reshape(L, Hkv, hd), index_pos).transpose(1, 0, 2)
        v = self.mm(lw["wv"], n).reshape(L, Hkv, hd).transpose(1, 0, 2)
        self.k[li] = np.concatenate([self.k[li][:, :index_pos], k], axis=1)
        self.v[li] = np.concatenate([self.v[li][:, :index_pos], v], axis=1)
        T = self.k[li].shape[1]
        y = np.empty((H, L, hd), np.float32)
        grp = H // Hkv
        for h in range(H):
            kk, vv = self.k[li][h // grp], self.v[li][h // grp]
            att = (q[h] @ kk.T) / np.float32(np.sqrt(hd))
            if L > 1:
                i = np.arange(L)[:, None] + index_pos
                j = np.arange(T)[None, :]
                att = np.where(j > i, -np.inf, att)
            att = att - att.max(axis=-1, keepdims=True)
            e = np.exp(att)
            y[h] = (e / e.sum(axis=-1, keepdims=True)) @ vv
        x = x + self.mm(lw["wo"], y.transpose(1, 0, 2).reshape(L, H * hd))
        n = self.rms(x, hw.ffn_norm[li])
        g = self.mm(lw["w1"], n)
        u = self.mm(lw["w3"], n)
        return x + self.mm(lw["w2"], (g / (1.0 + np.exp(-g))) * u)

    def head(self, x):
        """Final norm and output head on the last position of x -> logits [vocab]."""
        last = self.rms(x[-1:], self.hw.norm)
        return self.mm(self.hw.output, last)[0]

    def forward(self, tokens, index_pos):
        x = self.embed(tokens, index_pos)
        for li in range(self.cfg.n_layer):
            x = self.layer(li, x, index_pos)
        return self.head(x)
