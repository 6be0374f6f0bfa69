"""CPU oracle of the Qwen-Image (Wan 2.1) VAE decoder -- TEST INFRASTRUCTURE ONLY.

torch float64 restatement of app/models/vae.js:40-113 and its ops: conv3x3 with zero padding 1 and
the optional 2x nearest upsample of the input (app/gpu/gemm.js:56-80; torch.nn.functional.conv2d, a
library routine, pinned against a direct loop in tests/test_oracle_vae.py), the channel norm
y = x / max(||x||, 1e-12) * sqrt(C) * gamma (+ SiLU) (app/gpu/kernels.js:62-89 mode 1), the
single-head attention of the middle block (softmax(q k^T / sqrt(C)) v, app/models/vae.js:71-76),
and the RGBA conversion (vae.js:104-112).  Weights: a dict of float32 arrays in the checkpoint's
names, convolution weights OHWI flattened to [N, 9*cin].
"""

from __future__ import annotations

import math

import numpy as np

LATENT_MEAN = [-0.7571, -0.7089, -0.9113, 0.1075, -0.1745, 0.9653, -0.1517, 1.5508, 0.4134, -0.0715, 0.5517,
               -0.3632, -0.1922, -0.9497, 0.2503, -0.2921]
LATENT_STD = [2.8184, 1.4541, 2.3275, 2.6558, 1.2196, 1.7708, 2.6052, 2.0743, 3.2687, 2.1526, 2.8652, 1.5579,
              1.6382, 1.1253, 2.8251, 1.916]


def _t(a):
    import torch

    return torch.as_tensor(np.asarray(a), dtype=torch.float64)


def conv3x3(x, w, bias=None, up=False):
    """x NHWC [B, H, W, cin] (float64 tensor), w [cout, 9*cin] (OHWI) -> [B, H', W', cout]."""
    import torch
    import torch.nn.functional as F

    B, H, Wd, cin = x.shape
    if up:
        x = x.repeat_interleave(2, 1).repeat_interleave(2, 2)
    wk = _t(w).reshape(-1, 3, 3, cin).permute(0, 3, 1, 2)
    y = F.conv2d(x.permute(0, 3, 1, 2), wk, None if bias is None else _t(bias), padding=1)
    return y.permute(0, 2, 3, 1)


def conv3x3_direct(x, w, bias=None, up=False):
    """The same convolution as an explicit loop over output pixels and taps (numpy float64)."""
    x = np.asarray(x, np.float64)
    if up:
        x = x.repeat(2, 1).repeat(2, 2)
    B, H, Wd, cin = x.shape
    cout = w.shape[0]
    wk = np.asarray(w, np.float64).reshape(cout, 3, 3, cin)
    y = np.zeros((B, H, Wd, cout))
    for b in range(B):
        for oy in range(H):
            for ox in range(Wd):
                acc = np.zeros(cout) if bias is None else np.asarray(bias, np.float64).copy()
                for ty in range(3):
                    for tx in range(3):
                        iy, ix = oy + ty - 1, ox + tx - 1
                        if 0 <= iy < H and 0 <= ix < Wd:
                            acc += wk[:, ty, tx, :] @ x[b, iy, ix]
                y[b, oy, ox] = acc
    return y


def channel_norm(x, g, silu):
    """Channel norm over the last axis (float64)."""
    import torch

    C = x.shape[-1]
    n = torch.clamp(torch.sqrt((x * x).sum(-1, keepdim=True)), min=1e-12)
    y = x / n * math.sqrt(C) * _t(g)
    return y * torch.sigmoid(y) if silu else y


def linear(x, W, name):
    y = x @ _t(W[name + ".weight"]).T
    return y + _t(W[name + ".bias"]) if name + ".bias" in W else y


def resblock(x, W, p):
    """app/models/vae.js:42-56: norm + SiLU, conv, norm + SiLU, conv, plus the (1x1) shortcut."""
    t = channel_norm(x, W[p + ".residual.0.gamma"], True)
    t = conv3x3(t, W[p + ".residual.2.weight"], W[p + ".residual.2.bias"])
    t = channel_norm(t, W[p + ".residual.3.gamma"], True)
    t = conv3x3(t, W[p + ".residual.6.weight"], W[p + ".residual.6.bias"])
    sc = linear(x, W, p + ".shortcut") if p + ".shortcut.weight" in W else x
    return sc + t


def attention_block(x, W, p="decoder.middle.1"):
    import torch

    B, H, Wd, C = x.shape
    n = channel_norm(x, W[p + ".norm.gamma"], False).reshape(B, H * Wd, C)
    qkv = linear(n, W, p + ".to_qkv")
    q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
    s = q @ k.transpose(1, 2) / math.sqrt(C)
    a = torch.softmax(s, -1) @ v
    return x + linear(a, W, p + ".proj").reshape(B, H, Wd, C)


def decode(W, latent, upsamples):
    """latent [16, h, w] (normalized space) -> (float64 output [8h, 8w, 3] before clamping, RGBA
    uint8 [8h, 8w, 4]).  upsamples: the stage list (synthetic.VAE_UPSAMPLES layout)."""
    import torch

    lat = np.asarray(latent, np.float64)
    z = lat * np.asarray(LATENT_STD)[:, None, None] + np.asarray(LATENT_MEAN)[:, None, None]
    x = _t(z.transpose(1, 2, 0)[None].astype(np.float32))  # the device input is float32
    with torch.no_grad():
        x = linear(x, W, "conv2")
        x = conv3x3(x, W["decoder.conv1.weight"], W["decoder.conv1.bias"])
        x = resblock(x, W, "decoder.middle.0")
        x = attention_block(x, W)
        x = resblock(x, W, "decoder.middle.2")
        for i, s in enumerate(upsamples):
            p = f"decoder.upsamples.{i}"
            if s[0] == "up":
                x = conv3x3(x, W[p + ".resample.1.weight"], W[p + ".resample.1.bias"], up=True)
            else:
                x = resblock(x, W, p)
        x = channel_norm(x, W["decoder.head.0.gamma"], True)
        x = conv3x3(x, W["decoder.head.2.weight"], W["decoder.head.2.bias"])
    out = x[0].numpy()
    return out, to_rgba(out)


def to_rgba(out):
    """RGBA bytes of the decoder output [H, W, 3] (app/models/vae.js:104-112): float32 values promoted
    to double, clamp to [-1, 1], (v + 1) / 2 * 255, JS Math.round (nearest, ties toward +inf), a NaN
    stored as 0 by Uint8ClampedArray; alpha 255."""
    out = np.asarray(out, np.float32)
    t = (np.clip(out.astype(np.float64), -1.0, 1.0) + 1.0) / 2.0 * 255.0
    r = np.floor(t)
    r = np.where(t - r >= 0.5, r + 1.0, r)
    r = np.where(np.isnan(t), 0.0, r)
    img = np.full(out.shape[:2] + (4,), 255, np.uint8)
    img[..., :3] = r.astype(np.uint8)
    return img
