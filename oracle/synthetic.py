"""Synthetic DiT weights for the oracle -- TEST INFRASTRUCTURE ONLY.

Restates, on the CPU, the seeded random-init weights that the JS host builds on the device
(js/weights.mjs SyntheticWeights, js/dit.mjs AnimaDiT.synthetic): every tensor is
anima_fill_random over its element count with the seed (seed * 1000003 + fnv1a32(name)) mod
(2^53 - 111), restated by the C oracle's orc_fill_random.  The result is a dict in the comfy_quant
layout of tools/quant.py (the one oracle/dit_ref.py reads), so a full-depth DiT step can be checked
without writing a checkpoint file: the stacked self-attention q/k/v weight is split back into its
three row blocks.
"""

from __future__ import annotations

import json
import math

import numpy as np

import oracle as orc

D, HD, MLP, CTX, R = 2048, 128, 8192, 1024, 256
FIXED_LUT = np.array([-0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
                      0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671], np.float32)


def fnv1a32(s: str) -> int:
    h = 0x811C9DC5
    for ch in s:
        h ^= ord(ch)
        h = (h * 0x01000193) & 0xFFFFFFFF
    return h


def meta(fmt, **kw):
    return np.frombuffer(json.dumps({"format": fmt, **kw}).encode(), np.uint8)


class Source:
    """The per-name fills of SyntheticWeights (js/weights.mjs)."""

    def __init__(self, seed, mode="w4a8", blocks=28):
        self.seed, self.mode, self.blocks = seed, mode, blocks

    def seed_of(self, name):
        return (self.seed * 1000003 + fnv1a32(name)) % 9007199254740881

    def fill(self, n, kind, name, lo, hi):
        return orc.fill_random(n, kind, self.seed_of(name), np.float32(lo), np.float32(hi))

    def vector(self, name, n, lo=0.98, hi=1.02):
        return self.fill(n, "f32", name, lo, hi)

    def bf16(self, name, N, K, gain=1.0):
        a = gain * math.sqrt(3.0 / K)
        return self.fill(N * K, "bf16", name, -a, a).reshape(N, K)

    def quant_kind(self, block):
        if self.mode == "int8":
            return "i8"
        return "w4" if 0 < block < self.blocks - 1 else "i8"

    def block_linear(self, name, N, K, block):
        """(kind, arrays): i8 (grid [N,K], scale [N]); w4 (codes [N,K/2], srel [N,K/16], scale [N])."""
        kind = self.quant_kind(block)
        scale = self.fill(N, "f32", name + ".scale", 0.5 / (127 * math.sqrt(K)), 1.5 / (127 * math.sqrt(K)))
        if kind == "i8":
            return kind, (self.fill(N * K, "i8n", name, 40, 0).reshape(N, K), scale)
        codes = self.fill(N * K // 2, "u8", name, 0, 255).reshape(N, K // 2)
        srel = self.fill(N * K // 16, "u8", name + ".srel", 0x60, 0x6F).reshape(N, K // 16)
        return kind, (codes, srel, scale)


def _put_linear(W, base, kind, arrs, rows=None):
    sl = slice(None) if rows is None else rows
    if kind == "i8":
        grid, scale = arrs
        W[base + "weight"] = grid[sl]
        W[base + "weight_scale"] = scale[sl].reshape(-1, 1)
        W[base + "comfy_quant"] = meta("int8_tensorwise", convrot=True, convrot_groupsize=256)
    else:
        codes, srel, scale = arrs
        W[base + "weight"] = codes[sl].view(np.int8)
        W[base + "weight_s_rel"] = srel[sl]
        W[base + "weight_s_channel"] = scale[sl]
        W[base + "weight_codebook"] = FIXED_LUT
        W[base + "comfy_quant"] = meta("asym_w4a8_int8", group_size=16, convrot=True, convrot_groupsize=256)


def dit_weights(seed, mode="w4a8", blocks=28):
    """The weights of AnimaDiT.synthetic(gpu, new SyntheticWeights(gpu, seed, {mode, blocks})) in the
    dict layout of oracle/dit_ref.py (names of the reference checkpoint)."""
    src = Source(seed, mode, blocks)
    W = {}
    W["x_embedder.proj.1.weight"] = src.bf16("x_embedder.proj.1", D, 68)
    W["t_embedder.1.linear_1.weight"] = src.bf16("t_embedder.1.linear_1", D, D)
    W["t_embedder.1.linear_2.weight"] = src.bf16("t_embedder.1.linear_2", 3 * D, D)
    W["t_embedding_norm.weight"] = src.vector("t_embedding_norm.weight", D)
    for i in range(blocks):
        p = f"blocks.{i}."
        for nm in ("adaln_modulation_self_attn", "adaln_modulation_cross_attn", "adaln_modulation_mlp"):
            W[p + nm + ".1.weight"] = src.bf16(p + nm + ".1", R, D)
            W[p + nm + ".2.weight"] = src.bf16(p + nm + ".2", 3 * D, R, 0.1)
        kind, arrs = src.block_linear(p + "self_attn.qkv", 3 * D, D, i)
        for j, t in enumerate("qkv"):
            _put_linear(W, p + f"self_attn.{t}_proj.", kind, arrs, slice(j * D, (j + 1) * D))
        for nm, N, K in (("self_attn.output_proj", D, D), ("cross_attn.q_proj", D, D), ("cross_attn.k_proj", D, CTX),
                         ("cross_attn.v_proj", D, CTX), ("cross_attn.output_proj", D, D), ("mlp.layer1", MLP, D),
                         ("mlp.layer2", D, MLP)):
            kind, arrs = src.block_linear(p + nm, N, K, i)
            _put_linear(W, p + nm + ".", kind, arrs)
        for a in ("self_attn", "cross_attn"):
            W[p + a + ".q_norm.weight"] = src.vector(p + a + ".q_norm.weight", HD)
            W[p + a + ".k_norm.weight"] = src.vector(p + a + ".k_norm.weight", HD)
    W["final_layer.adaln_modulation.1.weight"] = src.bf16("final_layer.adaln_modulation.1", R, D)
    W["final_layer.adaln_modulation.2.weight"] = src.bf16("final_layer.adaln_modulation.2", 2 * D, R, 0.1)
    W["final_layer.linear.weight"] = src.bf16("final_layer.linear", 64, D)
    return W


# Wan 2.1 VAE decoder stages after the middle blocks (js/vae.mjs VAE_UPSAMPLES): residual blocks
# (cin, cout) or resamples (2x upsample + conv3x3 dim -> dim / 2)
VAE_UPSAMPLES = [(384, 384), (384, 384), (384, 384), ("up", 384),
                 (192, 384), (384, 384), (384, 384), ("up", 384),
                 (192, 192), (192, 192), (192, 192), ("up", 192),
                 (96, 96), (96, 96), (96, 96)]


def _bf16(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


def vae_weights(seed):
    """The weights of VAEDecoder.synthetic(gpu, new SyntheticWeights(gpu, seed)) (js/vae.mjs): a dict
    name -> float32 array in the checkpoint's names (OHWI convolution weights flattened to [N, 9*cin],
    1x1 convolutions [N, cin])."""
    src = Source(seed)
    W = {}

    def lin(name, N, K, gain):
        W[name + ".weight"] = _bf16(src.bf16(name, N, K, gain))
        W[name + ".bias"] = src.fill(N, "f32", name + ".bias", -0.05, 0.05)

    def gamma(name, n):
        W[name] = src.fill(n, "f32", name, 0.9, 1.1)

    def res(p, cin, cout):
        gamma(p + ".residual.0.gamma", cin)
        lin(p + ".residual.2", cout, 9 * cin, 1.0)
        gamma(p + ".residual.3.gamma", cout)
        lin(p + ".residual.6", cout, 9 * cout, 0.5)
        if cin != cout:
            lin(p + ".shortcut", cout, cin, 1.0)

    lin("conv2", 16, 16, 1.0)
    lin("decoder.conv1", 384, 9 * 16, 1.0)
    res("decoder.middle.0", 384, 384)
    gamma("decoder.middle.1.norm.gamma", 384)
    lin("decoder.middle.1.to_qkv", 3 * 384, 384, 1.0)
    lin("decoder.middle.1.proj", 384, 384, 0.5)
    res("decoder.middle.2", 384, 384)
    for i, s in enumerate(VAE_UPSAMPLES):
        p = f"decoder.upsamples.{i}"
        if s[0] == "up":
            lin(p + ".resample.1", s[1] // 2, 9 * s[1], 1.0)
        else:
            res(p, s[0], s[1])
    gamma("decoder.head.0.gamma", 96)
    lin("decoder.head.2", 3, 9 * 96, 1.0)
    return W
