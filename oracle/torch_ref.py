"""PyTorch fp32 CPU restatement of the reference's attention math -- TEST/BASELINE ONLY.

Restates tools/reference.py's DiT math in torch fp32 on the CPU: rms_norm (reference.py:93-94),
rotate_half RoPE with the 3D Cosmos angles (97-99, 174-187, 214-229),
F.scaled_dot_product_attention (109-111), the LayerNorm + adaLN modulation and gated residuals of
the block (231-242), and the ConvRot int8 linears in two semantics: W8A32 (the reference's own:
dequantized weights, fp32 activations) and W8A8 (this build's: activations quantized per token
after the rotation, emulated in fp32).  bench.py times it on the host cores as the CPU baseline
(attention, the quantized projections, the full 28-block step); tests/test_oracle_torchref.py
checks its RoPE table and attention against the C oracle.
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


def cpu_model():
    """The host CPU as /proc/cpuinfo names it, with its family / model numbers (a virtualized host may
    report only "AMD EPYC"; family 0x1A is Zen 5, 0x19 Zen 3 / Zen 4) and thread counts."""
    import os

    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (t.strip() for t in line.split(":", 1))
                if k in ("model name", "cpu family", "model", "stepping") and k not in info:
                    info[k] = v
    except OSError:
        pass
    name = info.get("model name", "unknown")
    arch = {"23": "Zen / Zen 2", "25": "Zen 3 / Zen 4", "26": "Zen 5"}.get(info.get("cpu family", ""), "")
    fam = f"family {info.get('cpu family', '?')} model {info.get('model', '?')} stepping {info.get('stepping', '?')}"
    return (f"{name} ({fam}{', ' + arch if arch and 'AMD' in name else ''}; {os.cpu_count()} host threads, "
            f"{len(os.sched_getaffinity(0))} usable)")


def hadamard256(x):
    """ConvRot rotation (tools/quant.py:30-45): x @ kron(H4, H4, H4, H4) / 16 per group of 256."""
    h4 = torch.tensor([[1., 1., 1., -1.], [1., 1., -1., 1.], [1., -1., 1., 1.], [-1., 1., 1., 1.]])
    h = torch.kron(torch.kron(h4, h4), torch.kron(h4, h4)) / 16
    return (x.reshape(-1, 256) @ h).reshape(x.shape)


def token_fake_quant(x):
    """W8A8's per-token int8 activations (s = amax/127, q = rint(x/s) clamped), returned dequantized."""
    s = x.abs().amax(-1, keepdim=True) / 127
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.clamp(torch.round(x / s), -127, 127) * s


def qlinear(x, w_deq, mode):
    """ConvRot int8 linear: y = H(x) @ W^T with W the dequantized rotated-domain weight; W8A8 also
    quantizes the rotated activations per token."""
    xr = hadamard256(x)
    if mode == "w8a8":
        xr = token_fake_quant(xr)
    return xr @ w_deq.T


def int8_weight(g, N, K):
    """comfy_quant int8 weight of the configs: round(40 N(0,1)) clipped to +-127, per-row scale."""
    q = torch.clamp(torch.round(40 * torch.randn(N, K, generator=g)), -127, 127)
    s = (0.5 + torch.rand(N, 1, generator=g)) / (127 * math.sqrt(K))
    return q * s


def linears_baseline(mode):
    """The attention sublayer's quantized projections of the 1024x1024 CFG batch (x [2*4096, 2048]:
    QKV 2048 -> 6144 and out 2048 -> 2048, 275 GOP) with the rotation and, for W8A8, the activation
    quantization; median of 3 after 1 warm-up."""
    import os

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2 * 4096, 2048, generator=g)
    wq, wo = int8_weight(g, 6144, 2048), int8_weight(g, 2048, 2048)
    with torch.no_grad():
        t = seconds(lambda: (qlinear(x, wq, mode), qlinear(x, wo, mode)), reps=3, warmup=1)
    ops = 2.0 * 8192 * 2048 * (6144 + 2048)
    return {"value": round(ops / t / 1e12, 4), "unit": "TOP/s", "cores": cores, "kind": "port", "cpu": cpu_model(),
            "ms": round(t * 1e3, 1),
            "sample": f"QKV (2048->6144) + out (2048->2048) int8 ConvRot linears on x [2*4096, 2048], {mode.upper()} "
                      f"semantics, torch fp32; median of 3 after 1 warm-up"}


def dit_step_baseline(mode="w8a32", blocks=28):
    """One full DiT step at 1024x1024, B=2 CFG (reference.py:231-242 per block, batched), run once:
    the patch embedding, every block -- self-attention with q/k RMSNorm + RoPE, cross-attention to
    the prompt pair's 512-token K/V, GELU MLP, adaLN modulation and gated residuals, quantized
    linears in `mode` -- and the final layer.  Each block has its own weight tensors (row-rotated
    copies of one seeded draw: the work does not depend on the values) and its own cross K/V,
    projected from the contexts before the timed step as the pipeline prepares them once per prompt
    (app/models/dit.js:232-249)."""
    import os
    import time

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B, Hp, Wp, H, D, C, CTX = 2, 64, 64, 16, 128, 2048, 1024
    L, Lk = Hp * Wp, 512
    g = torch.Generator().manual_seed(4)
    base = {n: int8_weight(g, N, K) for n, N, K in (("qkv", 3 * C, C), ("o", C, C), ("cq", C, C), ("co", C, C),
                                                     ("m1", 4 * C, C), ("m2", C, 4 * C))}
    Wk, Wv = int8_weight(g, C, CTX), int8_weight(g, C, CTX)
    Ws = [{n: torch.roll(w, i, 0) for n, w in base.items()} for i in range(blocks)]
    norms = [1 + 0.02 * torch.randn(D, generator=g) for _ in range(3)]
    ctx = torch.randn(B * Lk, CTX, generator=g)
    with torch.no_grad():
        kv = [(rms_norm(qlinear(ctx, torch.roll(Wk, i, 0), mode).view(B, Lk, H, D), norms[2]).transpose(1, 2),
               qlinear(ctx, torch.roll(Wv, i, 0), mode).view(B, Lk, H, D).transpose(1, 2)) for i in range(blocks)]
    mods = 0.1 * torch.randn(blocks, 3, 3 * C, generator=g)
    w_emb = 0.02 * torch.randn(C, 68, generator=g)
    w_fin = 0.02 * torch.randn(64, C, generator=g)
    cos, sin = dit_rope(Hp, Wp)
    lat = torch.randn(B, 16, 2 * Hp, 2 * Wp, generator=g)

    def ln_mod(x, m):
        return F.layer_norm(x, (C,), eps=1e-6) * (1 + m[C:2 * C]) + m[:C]

    def block(x, W, kc, vc, md):
        m = md[0]
        qkv = qlinear(ln_mod(x, m), W["qkv"], mode).view(B, L, 3, H, D)
        q = rms_norm(qkv[:, :, 0], norms[0]).transpose(1, 2)
        k = rms_norm(qkv[:, :, 1], norms[1]).transpose(1, 2)
        v = qkv[:, :, 2].transpose(1, 2)
        q = q * cos + rotate_half(q) * sin
        k = k * cos + rotate_half(k) * sin
        a = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(B * L, C)
        x = x + m[2 * C:] * qlinear(a, W["o"], mode)
        m = md[1]
        q = rms_norm(qlinear(ln_mod(x, m), W["cq"], mode).view(B, L, H, D), norms[0]).transpose(1, 2)
        a = F.scaled_dot_product_attention(q, kc, vc).transpose(1, 2).reshape(B * L, C)
        x = x + m[2 * C:] * qlinear(a, W["co"], mode)
        m = md[2]
        h = F.gelu(qlinear(ln_mod(x, m), W["m1"], mode))
        return x + m[2 * C:] * qlinear(h, W["m2"], mode)

    def step():
        # patchify 2x2 (16 channels -> 64 + 4 padding-mask features, dit.js:55-78) and embed
        p = lat.view(B, 16, Hp, 2, Wp, 2).permute(0, 2, 4, 3, 5, 1).reshape(B * L, 64)
        x = torch.cat([p, torch.zeros(B * L, 4)], 1) @ w_emb.T
        for i in range(blocks):
            x = block(x, Ws[i], kv[i][0], kv[i][1], mods[i])
        return F.layer_norm(x, (C,), eps=1e-6) @ w_fin.T

    with torch.no_grad():
        block(torch.randn(512, C, generator=g).repeat(16, 1), Ws[0], kv[0][0], kv[0][1], mods[0])  # kernel warm-up
        t = time.perf_counter()
        step()
        t = time.perf_counter() - t
    M = B * L
    flops = blocks * (2 * M * C * (3 * C + C + C + C + 8 * C) + 4 * B * H * L * L * D + 4 * B * H * L * Lk * D)
    return {"value": round(t * 1e3, 1), "unit": "ms", "tflops": round(flops / t / 1e12, 4), "cores": cores, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"one full {blocks}-block DiT step at 1024x1024, B=2 CFG, {mode.upper()} linears, torch fp32, "
                      f"run once (every block its own weights and cross K/V; the K/V projected before the step, "
                      f"once per prompt pair as on the GPU path)"}


if __name__ == "__main__":
    import json
    import sys

    if "--attention" in sys.argv:
        out = attention_baseline()
        out["cpu"] = cpu_model()
        print(json.dumps(out))
    if "--linears" in sys.argv:
        print(json.dumps({m: linears_baseline(m) for m in ("w8a8", "w8a32")}))
    if "--dit-step" in sys.argv:
        print(json.dumps(dit_step_baseline("w8a32", blocks=28)))
