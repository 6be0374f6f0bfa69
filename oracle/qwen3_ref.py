"""Test infrastructure only (never shipped, never on the product path): float64 restatement of
the reference's Qwen3 text encoder forward (app/models/qwen3.js:38-78) and of its 1D RoPE table
(app/models/common.js:3-22), for the parity test of js/qwen3.mjs.

Pinned by: RMSNorm and SiLU are closed forms (ops.js:111-117, kernels.js:19); the causal GQA
softmax is the oracle's brute force with the causal limit min(Lk, row + 1) of kernels.js:49;
attention is additionally pinned against the C oracle in tests/test_attention_gpu.py.
"""

import numpy as np

CFG = dict(hidden=1024, heads=16, kv_heads=8, head_dim=128, theta=1e6)


def rope_table(L, Dh, theta):
    """(cos, sin) [L][Dh/2] as common.js builds them: angle = l * fround(1 / theta^(2i/Dh)),
    cos / sin in float64, stored as float32 (common.js:3-22)."""
    half = Dh // 2
    inv = np.array([np.float32(1.0 / theta ** ((2 * i) / Dh)) for i in range(half)], np.float64)
    ang = (np.arange(L, dtype=np.float64)[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    return np.cos(ang).astype(np.float32).astype(np.float64), np.sin(ang).astype(np.float32).astype(np.float64)


def rmsnorm(x, w, eps=1e-6):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def rope(x, cos, sin):
    """split-half rotation per head: x [L, H, Dh] (ops.js:148; kernels.js rope)"""
    h = x.shape[-1] // 2
    a, b = x[..., :h], x[..., h:]
    c, s = cos[:, None, :], sin[:, None, :]
    return np.concatenate([a * c - b * s, b * c + a * s], -1)


def causal_gqa(q, k, v, group):
    """q [L, H, Dh], k / v [L, KH, Dh]: softmax over keys j <= i (kernels.js:49) per head."""
    L, H, Dh = q.shape
    o = np.zeros_like(q)
    mask = np.triu(np.ones((L, L), bool), 1)
    for h in range(H):
        s = q[:, h] @ k[:, h // group].T / np.sqrt(Dh)
        s[mask] = -np.inf
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        o[:, h] = (p / p.sum(-1, keepdims=True)) @ v[:, h // group]
    return o


def encode(W, ids, layers):
    """W: dict name -> float64 array ('{i}.q' [N, K] etc., 'embed' [V, 1024], 'norm')."""
    D, H, KH, Dh = CFG["hidden"], CFG["heads"], CFG["kv_heads"], CFG["head_dim"]
    L = len(ids)
    x = W["embed"][np.asarray(ids)]
    cos, sin = rope_table(L, Dh, CFG["theta"])
    for i in range(layers):
        g = lambda n: W[f"{i}.{n}"]
        h = rmsnorm(x, g("ln1"))
        q = (h @ g("q").T).reshape(L, H, Dh)
        k = (h @ g("k").T).reshape(L, KH, Dh)
        v = (h @ g("v").T).reshape(L, KH, Dh)
        q = rope(rmsnorm(q, g("qn")), cos, sin)
        k = rope(rmsnorm(k, g("kn")), cos, sin)
        a = causal_gqa(q, k, v, H // KH).reshape(L, H * Dh)
        x = x + a @ g("o").T
        h2 = rmsnorm(x, g("ln2"))
        gt, up = h2 @ g("gate").T, h2 @ g("up").T
        x = x + (gt / (1.0 + np.exp(-gt)) * up) @ g("down").T
    return rmsnorm(x, W["norm"])
