"""Test infrastructure only (never shipped, never on the product path): float64 restatement of
the LLM adapter (app/models/dit.js:136-190; tools/reference.py:141-169) for the parity test of
js/dit.mjs adapt.  RoPE tables as app/models/common.js builds them (qwen3_ref.rope_table).

Pinned by: RMSNorm, the split-half rotation and erf-GELU are closed forms; the softmax attention
is a brute force (the kernels' own D = 64 path is pinned against the C oracle in
tests/test_attention_gpu.py)."""

import math

import numpy as np

from .qwen3_ref import rmsnorm, rope, rope_table

H, HD, D = 16, 64, 1024


def _attn(q, k, v):
    o = np.zeros_like(q)
    for h in range(H):
        s = q[:, h] @ k[:, h].T / math.sqrt(HD)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        o[:, h] = (p / p.sum(-1, keepdims=True)) @ v[:, h]
    return o


def adapt(W, hidden, ids, weights, blocks):
    gelu = np.vectorize(lambda z: 0.5 * z * (1.0 + math.erf(z / math.sqrt(2.0))))
    x = W["embed"][np.asarray(ids)]
    Lt, Ls = x.shape[0], hidden.shape[0]
    cT, sT = rope_table(Lt, HD, 1e4)
    cS, sS = rope_table(Ls, HD, 1e4)

    def attn(p, xq, ctx, cq, sq, ck, sk):
        q = rope(rmsnorm((xq @ W[p + "q"].T).reshape(-1, H, HD), W[p + "qn"]), cq, sq)
        k = rope(rmsnorm((ctx @ W[p + "k"].T).reshape(-1, H, HD), W[p + "kn"]), ck, sk)
        v = (ctx @ W[p + "v"].T).reshape(-1, H, HD)
        return _attn(q, k, v).reshape(-1, D) @ W[p + "o"].T

    for i in range(blocks):
        p = f"{i}."
        n = rmsnorm(x, W[p + "nSelf"])
        x = x + attn(p + "self.", n, n, cT, sT, cT, sT)
        x = x + attn(p + "cross.", rmsnorm(x, W[p + "nCross"]), hidden, cT, sT, cS, sS)
        h = gelu(rmsnorm(x, W[p + "nMlp"]) @ W[p + "mlp0"].T + W[p + "mlp0.bias"])
        x = x + h @ W[p + "mlp2"].T + W[p + "mlp2.bias"]
    out = rmsnorm(x @ W["out"].T + W["out.bias"], W["norm"]) * np.asarray(weights, np.float64)[:, None]
    return np.concatenate([out, np.zeros((max(512, Lt) - Lt, D))])
