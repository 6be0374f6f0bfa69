"""PyTorch fp32 CPU restatement of the reference's attention math -- TEST/BASELINE ONLY.

Restates tools/reference.py's DiT self-attention in torch fp32 on the CPU: rms_norm
(reference.py:93-94), rotate_half RoPE with the 3D Cosmos angles (97-99, 174-187, 214-229)
and F.scaled_dot_product_attention (109-111).  bench.py times it on the host cores as the
CPU baseline; tests use it as an independent formulation of the fused norm+RoPE+attention.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def rms_norm(x, w, eps=1e-6):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def dit_rope(Hp, Wp):
    """cos, sin [L, 128] (split-half duplicated), reference.py:174-187 and 214-216."""
    head_dim = 128
    dim_h = head_dim // 6 * 2
    dim_t = head_dim - 2 * dim_h
    sp = torch.arange(0, dim_h, 2)[: dim_h // 2].float() / dim_h
    tp = torch.arange(0, dim_t, 2)[: dim_t // 2].float() / dim_t
    h_theta = 10000.0 * 4.0 ** (dim_h / (dim_h - 2))
    hf = 1.0 / h_theta ** sp
    tf = 1.0 / 10000.0 ** tp
    hh, ww = torch.meshgrid(torch.arange(Hp).float(), torch.arange(Wp).float(), indexing="ij")
    ang = torch.cat([torch.zeros(Hp * Wp, tf.numel()) * tf, hh.reshape(-1, 1) * hf, ww.reshape(-1, 1) * hf], 1)
    cos, sin = ang.cos(), ang.sin()
    return torch.cat([cos, cos], -1), torch.cat([sin, sin], -1)


def self_attention(qkv, qn, kn, cos, sin, H=16, D=128):
    """qkv [B, L, 3*H*D] -> O [B, L, H*D]: q/k RMSNorm + RoPE + SDPA (reference.py:222-230)."""
    B, L, _ = qkv.shape
    x = qkv.view(B, L, 3, H, D)
    q = rms_norm(x[:, :, 0], qn).transpose(1, 2)
    k = rms_norm(x[:, :, 1], kn).transpose(1, 2)
    v = x[:, :, 2].transpose(1, 2)
    q = q * cos + rotate_half(q) * sin
    k = k * cos + rotate_half(k) * sin
    o = F.scaled_dot_product_attention(q, k, v)
    return o.transpose(1, 2).reshape(B, L, H * D)


def attention_flops(B, H, Lq, Lk, D=128):
    """4*Lq*Lk*D*H per batch element (app/gpu/ops.js:174)."""
    return 4.0 * B * H * Lq * Lk * D


def seconds(fn, reps=3, warmup=1):
    import time

    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    ts.sort()
    return ts[len(ts) // 2]


def attention_baseline(B=2, Hp=64, Wp=64, H=16, D=128):
    """Times self_attention at the bench workload on every host core; returns the
    cpu_baseline record (TFLOP/s with the GPU's algorithmic FLOP count)."""
    import os

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    L = Hp * Wp
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(B, L, 3 * H * D, generator=g)
    qn = 1 + 0.02 * torch.randn(D, generator=g)
    kn = 1 + 0.02 * torch.randn(D, generator=g)
    cos, sin = dit_rope(Hp, Wp)
    with torch.no_grad():
        t = seconds(lambda: self_attention(qkv, qn, kn, cos, sin, H, D), reps=3, warmup=1)
    fl = attention_flops(B, H, L, L, D)
    return {"value": round(fl / t / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"full step: torch fp32 q/k RMSNorm + RoPE + SDPA (tools/reference.py math), B={B} H={H} "
                      f"N={L} D={D}; median of 3 after 1 warm-up = {t * 1e3:.0f} ms/step"}


if __name__ == "__main__":
    import json
    import sys

    if "--attention" in sys.argv:
        print(json.dumps(attention_baseline()))
