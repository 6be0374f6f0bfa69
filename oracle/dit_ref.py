"""CPU oracle of one Anima DiT step -- TEST INFRASTRUCTURE ONLY.

numpy (+ the C oracle for the exact row ops, quantization and attention) restatement of
tools/reference.py:194-249 / app/models/dit.js:196-325 for B prompts at once, in two semantics:
  * "w8a8": this build's arithmetic (per-token int8 activations after the ConvRot rotation, exact
    integer GEMMs, bf16 attention numerics model);
  * "ref":  the reference's own (W8A32 on the dequantized weights, fp64 attention).
Weights come as a dict of numpy arrays in the comfy_quant layout (tools/quant.py).
"""

from __future__ import annotations

import math

import numpy as np

import oracle as orc

D, HEADS, HD = 2048, 16, 128


def bf16_to_f32(u16):
    import torch

    u = torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).to(torch.int32)
    return (u << 16).view(torch.float32).numpy()


def timestep_embedding(sigma):
    """app/models/dit.js:41-51 (float32 rounding at the same points)."""
    half = D // 2
    i = np.arange(half, dtype=np.float64)
    f = np.exp((-math.log(10000) * i / half).astype(np.float32).astype(np.float64)).astype(np.float32)
    a = (np.float64(sigma) * f.astype(np.float64)).astype(np.float32).astype(np.float64)
    return np.concatenate([np.cos(a), np.sin(a)]).astype(np.float32)


def patchify(lat, h, w):
    Hp, Wp = h // 2, w // 2
    x = np.concatenate([lat, np.zeros((1, h, w), np.float32)], 0).reshape(17, Hp, 2, Wp, 2)
    return x.transpose(1, 3, 0, 2, 4).reshape(Hp * Wp, 68)


def unpatchify(o, h, w):
    Hp, Wp = h // 2, w // 2
    return o.reshape(Hp, Wp, 2, 2, 16).transpose(4, 0, 2, 1, 3).reshape(16, h, w)


class Linear:
    def __init__(self, W, base):
        self.kind = "bf16"
        if base + "comfy_quant" in W:
            fmt = bytes(W[base + "comfy_quant"].tolist()).decode()
            if "int8_tensorwise" in fmt:
                self.kind = "i8"
                self.grid = W[base + "weight"].astype(np.int8)
                self.scale = W[base + "weight_scale"].reshape(-1).astype(np.float32)
            else:
                self.kind = "w4"
                codes = W[base + "weight"].view(np.uint8)
                N, K2 = codes.shape
                self.grid = orc.w4_decode(codes, W[base + "weight_s_rel"].view(np.uint8), W[base + "weight_codebook"], N, 2 * K2)
                self.scale = W[base + "weight_s_channel"].astype(np.float32)
        else:
            self.w = bf16_to_f32(W[base + "weight"])

    def deq(self):
        """Dense fp32 weight in the rotated input domain (x_r @ deq^T), tools/quant.py:81-83."""
        return self.grid.astype(np.float64) * self.scale[:, None].astype(np.float64)


def stack(lins):
    out = Linear.__new__(Linear)
    out.kind = lins[0].kind
    out.grid = np.concatenate([l.grid for l in lins])
    out.scale = np.concatenate([l.scale for l in lins])
    return out


def gelu_as(x):
    """erf-GELU with Abramowitz-Stegun 7.1.26 (app/gpu/kernels.js:9-20), float64."""
    z = x * 0.7071067811865476
    a = np.abs(z)
    t = 1.0 / (1.0 + 0.3275911 * a)
    y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t * np.exp(-a * a)
    return 0.5 * x * (1.0 + np.sign(z) * y)


def imatmul(q, g, chunk=1024):
    """Exact int64 q [M,K] @ g [N,K]^T of int8 operands in |v| <= 128: float32 products over K-chunks
    of 1024, each of whose partial sums (whatever order the BLAS adds in) is an integer below
    128 * 127 * 1024 < 2^24, so every float32 step is exact; the chunks add in int64."""
    import torch

    qt, gt = torch.from_numpy(np.ascontiguousarray(q)), torch.from_numpy(np.ascontiguousarray(g))
    acc = torch.zeros((q.shape[0], g.shape[0]), dtype=torch.int64)
    for k0 in range(0, q.shape[1], chunk):
        acc += (qt[:, k0:k0 + chunk].float() @ gt[:, k0:k0 + chunk].float().T).to(torch.int64)
    assert int(acc.abs().max()) < 2 ** 31
    return acc.to(torch.int32).numpy()


def qlinear(mode, x_rot, L, epi_c=None, gate=None, g_off=0, act=0, xq=None):
    """y = x_r @ dec(W)^T with this build's W8A8 arithmetic or the reference's W8A32."""
    if mode == "w8a8":
        q, s = xq if xq is not None else orc.token_quant(x_rot)
        acc = imatmul(q, L.grid)
        return orc.linear_epilogue(acc, s, L.scale, act=act, epi=2 if gate is not None else 0,
                                   gate=gate, g_off=g_off, c=epi_c)
    y = (x_rot.astype(np.float64) @ L.deq().T)
    if act == 1:
        y = gelu_as(y)
    if gate is not None:
        return (epi_c.astype(np.float64) + gate[g_off:g_off + y.shape[1]] * y).astype(np.float32)
    return y.astype(np.float32)


def bf16_linear(x, L, act=None):
    import torch

    y = (torch.from_numpy(np.ascontiguousarray(x)).double() @ torch.from_numpy(L.w).double().T).numpy()
    if act == "silu":
        y = y / (1 + np.exp(-y))
    return y.astype(np.float32)


def attention(mode, q, k, v, B, Lq, Lk, ldq, ldk, ldv, q_off=0, k_off=0, v_off=0):
    kind = "bf16" if mode == "w8a8" else "f64"
    return orc.attention(kind, q, k, v, B=B, Lq=Lq, Lk=Lk, H=HEADS, D=HD, ldq=ldq, ldk=ldk, ldv=ldv, q_off=q_off,
                         k_off=k_off, v_off=v_off).reshape(B * Lq, HEADS * HD)


def _f32(W, name):
    return (bf16_to_f32(W[name]) if W[name].dtype == np.uint16 else W[name]).astype(np.float32)


def time_cond(W, nblocks, sigma):
    """timeCond (app/models/dit.js:196-225; tools/reference.py:203-213, 218-220, 244): per block the
    modulation vectors [3D] of the self-attention, cross-attention and MLP sublayers (shift, scale,
    gate chunks), plus the final layer's [2D] (shift, scale).  mod = adaln_lora[:n] + W2 W1 silu(emb)."""
    temb = timestep_embedding(sigma)[None]
    lora = bf16_linear(bf16_linear(temb, Linear(W, "t_embedder.1.linear_1."), "silu"), Linear(W, "t_embedder.1.linear_2."))
    emb = orc.rmsnorm(temb, _f32(W, "t_embedding_norm.weight"), D)
    semb = (emb.astype(np.float64) / (1 + np.exp(-emb.astype(np.float64)))).astype(np.float32)

    def mod(p, n):
        hh = bf16_linear(semb, Linear(W, p + ".1."))
        return (lora[0, :n].astype(np.float64) + bf16_linear(hh, Linear(W, p + ".2."))[0]).astype(np.float32)

    blocks = [tuple(mod(f"blocks.{i}.{nm}", 3 * D) for nm in
                    ("adaln_modulation_self_attn", "adaln_modulation_cross_attn", "adaln_modulation_mlp"))
              for i in range(nblocks)]
    return blocks, mod("final_layer.adaln_modulation", 2 * D)


def prepare_context(ctxs):
    """prepareContext's shared part (dit.js:232-249): the stacked contexts, rotated once, and their
    per-token int8 form."""
    ctx = np.concatenate(ctxs).astype(np.float32)
    ctx_r = orc.hadamard256(ctx)
    return ctx_r, orc.token_quant(ctx_r), ctxs[0].shape[0]


def dit_block(mode, W, i, x, mods, cs, ctx, B, L):
    """One DiT block (dit.js:261-315; reference.py:231-242): x [B*L, D] -> x.  mods = (self, cross,
    mlp) modulation vectors, each (shift | scale | gate) chunks of D; ctx = prepare_context(...)."""
    p = f"blocks.{i}."
    ms, mc, mm = mods
    ctx_r, ctx_q, Lk = ctx
    # self-attention
    n = orc.layernorm_mod(x, ms, 0, D, D, rotate=True)
    qkv_w = stack([Linear(W, p + f"self_attn.{t}_proj.") for t in "qkv"])
    qkv = qlinear(mode, n, qkv_w)
    qn, kn = _f32(W, p + "self_attn.q_norm.weight"), _f32(W, p + "self_attn.k_norm.weight")
    qkv = np.concatenate([orc.qk_norm_rope(qkv[b * L:(b + 1) * L], L, HEADS, HD, 3 * D, qn, kn, cs, L * 64)
                          for b in range(B)])
    a = attention(mode, qkv, qkv, qkv, B, L, L, 3 * D, 3 * D, 3 * D, 0, D, 2 * D)
    x = qlinear(mode, orc.hadamard256(a), Linear(W, p + "self_attn.output_proj."), epi_c=x, gate=ms, g_off=2 * D)
    # cross-attention (no RoPE; q and k RMSNorm per head)
    n = orc.layernorm_mod(x, mc, 0, D, D, rotate=True)
    q = qlinear(mode, n, Linear(W, p + "cross_attn.q_proj."))
    q = orc.rmsnorm(q.reshape(-1, HD), _f32(W, p + "cross_attn.q_norm.weight"), HD).reshape(B * L, D)
    kx = qlinear(mode, ctx_r, Linear(W, p + "cross_attn.k_proj."), xq=ctx_q if mode == "w8a8" else None)
    k = orc.rmsnorm(kx.reshape(-1, HD), _f32(W, p + "cross_attn.k_norm.weight"), HD).reshape(B * Lk, D)
    v = qlinear(mode, ctx_r, Linear(W, p + "cross_attn.v_proj."), xq=ctx_q if mode == "w8a8" else None)
    a = attention(mode, q, k, v, B, L, Lk, D, D, D)
    x = qlinear(mode, orc.hadamard256(a), Linear(W, p + "cross_attn.output_proj."), epi_c=x, gate=mc, g_off=2 * D)
    # MLP
    n = orc.layernorm_mod(x, mm, 0, D, D, rotate=True)
    hdn = qlinear(mode, n, Linear(W, p + "mlp.layer1."), act=1)
    return qlinear(mode, orc.hadamard256(hdn), Linear(W, p + "mlp.layer2."), epi_c=x, gate=mm, g_off=2 * D)


def dit_step(W, nblocks, latents, h, w, ctxs, sigma, mode="w8a8"):
    """Returns (velocities [B][16,h,w], x after block 0 [B*L, 2048])."""
    B = len(latents)
    Hp, Wp = h // 2, w // 2
    L = Hp * Wp
    mods, mf = time_cond(W, nblocks, sigma)
    ctx = prepare_context(ctxs)
    x = bf16_linear(np.concatenate([patchify(l, h, w) for l in latents]), Linear(W, "x_embedder.proj.1."))
    cs = orc.dit_rope_table(Hp, Wp)
    block0 = None
    for i in range(nblocks):
        x = dit_block(mode, W, i, x, mods[i], cs, ctx, B, L)
        if i == 0:
            block0 = x.copy()
    n = orc.layernorm_mod(x, mf, 0, D, D, rotate=False)
    o = bf16_linear(n, Linear(W, "final_layer.linear."))
    return [unpatchify(o[b * L:(b + 1) * L], h, w) for b in range(B)], block0
