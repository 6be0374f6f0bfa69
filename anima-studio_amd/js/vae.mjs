// Qwen-Image (Wan 2.1) VAE decoder for single images on the gfx950 op layer, NHWC activations.
// Restates app/models/vae.js (load 10-36, resblock 42-56, decode 59-113) on this build's ops:
// conv3x3 as an implicit GEMM on the bf16 matrix cores (fused 2x nearest upsample and residual),
// the channel norm kernel, the 1x1 convolutions as bf16-weight linears, and the single-head
// 384-dim spatial attention on the chunked attention path.  The causal 3D convolutions arrive
// collapsed to 2D in OHWI layout (tools/build_assets.py:160-180).
// Node-12 syntax only.

import * as ops from "./ops.mjs";
import { native } from "./gpu.mjs";

// latent denormalization constants of the Qwen-Image VAE (app/models/vae.js:6-7)
export const LATENT_MEAN = [-0.7571, -0.7089, -0.9113, 0.1075, -0.1745, 0.9653, -0.1517, 1.5508, 0.4134, -0.0715, 0.5517,
  -0.3632, -0.1922, -0.9497, 0.2503, -0.2921];
export const LATENT_STD = [2.8184, 1.4541, 2.3275, 2.6558, 1.2196, 1.7708, 2.6052, 2.0743, 3.2687, 2.1526, 2.8652, 1.5579,
  1.6382, 1.1253, 2.8251, 1.916];

// The decoder's stages (Wan 2.1 Decoder3d with dim 96, dim_mult [1, 2, 4, 4], 2 residual blocks per
// level + 1): after the middle blocks at 384 channels, entries of decoder.upsamples are residual
// blocks [cin, cout] or resamples (2x nearest upsample + conv3x3 cin -> cin / 2).
export const VAE_UPSAMPLES = [
  [384, 384], [384, 384], [384, 384], { up: 384 },
  [192, 384], [384, 384], [384, 384], { up: 384 },
  [192, 192], [192, 192], [192, 192], { up: 192 },
  [96, 96], [96, 96], [96, 96],
];
export const VAE_DIM = 384;

export class VAEDecoder {
  // From the decoder checkpoint in the web-asset layout (app/models/vae.js:10-36).
  static load(gpu, st) {
    const v = new VAEDecoder(gpu);
    const res = (p) => ({
      n1: st.vector(gpu, p + ".residual.0.gamma"),
      c1: st.linear(gpu, p + ".residual.2."),
      n2: st.vector(gpu, p + ".residual.3.gamma"),
      c2: st.linear(gpu, p + ".residual.6."),
      sc: st.has(p + ".shortcut.weight") ? st.linear(gpu, p + ".shortcut.") : null,
    });
    v.conv2 = st.linear(gpu, "conv2.");
    v.conv1 = st.linear(gpu, "decoder.conv1.");
    v.mid0 = res("decoder.middle.0");
    v.attn = {
      norm: st.vector(gpu, "decoder.middle.1.norm.gamma"),
      qkv: st.linear(gpu, "decoder.middle.1.to_qkv."),
      proj: st.linear(gpu, "decoder.middle.1.proj."),
    };
    v.mid2 = res("decoder.middle.2");
    v.ups = [];
    for (let i = 0; i < 15; i++) {
      const p = `decoder.upsamples.${i}`;
      if (st.has(p + ".resample.1.weight")) v.ups.push({ up: st.linear(gpu, p + ".resample.1.") });
      else v.ups.push({ res: res(p) });
    }
    v.headNorm = st.vector(gpu, "decoder.head.0.gamma");
    v.head = st.linear(gpu, "decoder.head.2.");
    return v;
  }

  // Seeded random-init weights of the same architecture (SyntheticWeights), under the checkpoint's
  // names: convolutions U(-a, a), a = gain sqrt(3 / K), biases U(-0.05, 0.05), gammas U(0.9, 1.1).
  static synthetic(gpu, src) {
    const v = new VAEDecoder(gpu);
    const lin = (name, N, K, gain) => {
      const W = src.bf16Linear(gpu, name, N, K, gain);
      W.bias = src.vector(gpu, name + ".bias", N, -0.05, 0.05);
      return W;
    };
    const gamma = (name, n) => src.vector(gpu, name, n, 0.9, 1.1);
    const res = (p, cin, cout) => ({
      n1: gamma(p + ".residual.0.gamma", cin), c1: lin(p + ".residual.2", cout, 9 * cin, 1.0),
      n2: gamma(p + ".residual.3.gamma", cout), c2: lin(p + ".residual.6", cout, 9 * cout, 0.5),
      sc: cin !== cout ? lin(p + ".shortcut", cout, cin, 1.0) : null,
    });
    v.conv2 = lin("conv2", 16, 16, 1.0);
    v.conv1 = lin("decoder.conv1", VAE_DIM, 9 * 16, 1.0);
    v.mid0 = res("decoder.middle.0", VAE_DIM, VAE_DIM);
    v.attn = { norm: gamma("decoder.middle.1.norm.gamma", VAE_DIM), qkv: lin("decoder.middle.1.to_qkv", 3 * VAE_DIM, VAE_DIM, 1.0),
      proj: lin("decoder.middle.1.proj", VAE_DIM, VAE_DIM, 0.5) };
    v.mid2 = res("decoder.middle.2", VAE_DIM, VAE_DIM);
    v.ups = VAE_UPSAMPLES.map((s, i) => {
      const p = `decoder.upsamples.${i}`;
      return s.up ? { up: lin(p + ".resample.1", s.up / 2, 9 * s.up, 1.0) } : { res: res(p, s[0], s[1]) };
    });
    v.headNorm = gamma("decoder.head.0.gamma", 96);
    v.head = lin("decoder.head.2", 3, 9 * 96, 1.0);
    return v;
  }

  constructor(gpu) {
    this.gpu = gpu;
    // conv / attention arithmetic: "fp32" (the reference's: fp32-level results from the bf16 matrix
    // cores, activations as two bf16 terms) or "bf16" (activations rounded to bf16)
    this.precision = "fp32";
    this.keepRaw = false; // decode() also returns the float output before clamping as `raw`
  }

  // residual block (app/models/vae.js:42-56): norm + SiLU -> conv -> norm + SiLU -> conv + shortcut
  resblock(x, r, h, w) {
    const gpu = this.gpu;
    const o = { precision: this.precision };
    const cin = x.shape[1];
    let t = ops.channelNorm(gpu, x, r.n1, cin, true);
    const a = ops.conv3x3(gpu, t, r.c1, h, w, false, null, o);
    t.release();
    t = ops.channelNorm(gpu, a, r.n2, r.c1.N, true);
    a.release();
    const out = r.sc ? ops.linear(gpu, x, r.sc) : x;
    ops.conv3x3Into(gpu, t, r.c2, h, w, out, o);
    t.release();
    if (out !== x) x.release();
    return out;
  }

  // The decoder on a device tensor z [h*w, 16] (NHWC, denormalized): returns the [8h*8w, 3] output
  // before clamping (a new tensor).  onStage(frac) is awaited after the middle blocks and after
  // every up-stage.
  async decodeDevice(z, h, w, onStage) {
    const gpu = this.gpu;
    const o = { precision: this.precision };
    let t = ops.linear(gpu, z, this.conv2);
    let x = ops.conv3x3(gpu, t, this.conv1, h, w, false, null, o);
    t.release();
    x = this.resblock(x, this.mid0, h, w);

    // single-head spatial attention (app/models/vae.js:71-76)
    const C = VAE_DIM, hw = h * w;
    const n = ops.channelNorm(gpu, x, this.attn.norm, C, false);
    const qkv = ops.linear(gpu, n, this.attn.qkv);
    n.release();
    const a = ops.attention(gpu, { q: qkv, k: qkv, v: qkv, Lq: hw, Lk: hw, H: 1, D: C, ldq: 3 * C, ldk: 3 * C, ldv: 3 * C,
      qOff: 0, kOff: C, vOff: 2 * C, precision: this.precision });
    qkv.release();
    ops.linear(gpu, a, this.attn.proj, { out: x, resid: true });
    a.release();
    x = this.resblock(x, this.mid2, h, w);
    if (onStage) await onStage(0);

    let H = h, W = w;
    for (let i = 0; i < this.ups.length; i++) {
      const u = this.ups[i];
      if (u.up) {
        const y = ops.conv3x3(gpu, x, u.up, H, W, true, null, o);
        x.release();
        x = y;
        H *= 2;
        W *= 2;
      } else {
        x = this.resblock(x, u.res, H, W);
      }
      if (onStage) await onStage((i + 1) / this.ups.length);
    }
    t = ops.channelNorm(gpu, x, this.headNorm, x.shape[1], true);
    x.release();
    const rgb = ops.conv3x3(gpu, t, this.head, H, W, false, null, o);
    t.release();
    return rgb;
  }

  // latent: Float32Array [16, h, w] in the model's normalized space -> RGBA image
  // (app/models/vae.js:59-113).  onStage(frac) after the middle blocks and after every up-stage;
  // the device queue is drained there, as the reference does to keep the caller responsive.
  async decode(latent, h, w, onStage) {
    const gpu = this.gpu;
    const hw = h * w;
    const z = new Float32Array(hw * 16);
    for (let c = 0; c < 16; c++) for (let i = 0; i < hw; i++) z[i * 16 + c] = latent[c * hw + i] * LATENT_STD[c] + LATENT_MEAN[c];
    const zt = gpu.fromArray(z, [hw, 16]);
    const rgb = await this.decodeDevice(zt, h, w, async (f) => {
      await gpu.sync();
      if (onStage) onStage(f);
    });
    zt.release();
    const H = 8 * h, W = 8 * w;
    // RGBA on the device (vae.js:104-112's loop, same arithmetic), one read of 4 bytes per pixel
    const rgba = gpu.empty([H * W * 4], "u8");
    native.toRgba(gpu.ctx, rgb.buf, H * W, rgba.buf);
    const bytes = await gpu.read(rgba);
    rgba.release();
    const img = new Uint8ClampedArray(bytes.buffer, bytes.byteOffset, bytes.length);
    const out = { data: img, width: W, height: H };
    if (this.keepRaw) out.raw = await gpu.read(rgb);
    rgb.release();
    return out;
  }
}
