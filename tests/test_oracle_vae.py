"""Pins of the VAE oracle (oracle/vae_ref.py) and the channel norm restatement (oracle.c):

  * conv3x3 through torch's conv2d in float64 against an explicit loop over pixels and taps, with
    and without the fused 2x nearest upsample, and against the defining property of the upsample
    (the same as convolving the nearest-upsampled image, which the loop restates directly);
  * the channel norm of the C oracle (the shader's fp32 reduction order) against the float64 closed
    form, its scale invariance, and the norm of the output (sqrt(C) * gamma per pixel);
  * the decoder's stage list: 15 up-stages, three resamples that halve the channels, 8x the latent
    size at the end.
"""

import math

import numpy as np
import pytest

import oracle as orc
from oracle import synthetic, vae_ref

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("up", [False, True])
def test_conv3x3_library_matches_direct_loop(up):
    rng = np.random.default_rng(1 + up)
    B, H, W, cin, cout = 2, 5, 4, 16, 3
    x = rng.standard_normal((B, H, W, cin))
    w = rng.standard_normal((cout, 9 * cin))
    b = rng.standard_normal(cout)
    got = vae_ref.conv3x3(torch.tensor(x), w, b, up=up).numpy()
    ref = vae_ref.conv3x3_direct(x, w, b, up=up)
    assert got.shape == ref.shape == (B, 2 * H if up else H, 2 * W if up else W, cout)
    assert np.max(np.abs(got - ref)) <= 1e-12 * np.abs(ref).max()


def test_conv3x3_tap_layout():
    # OHWI: weight k = (ky * 3 + kx) * cin + ci; a single tap at (ky, kx) = (0, 2) with an impulse
    # input at pixel (2, 1) lands at output pixel (2 - 0 + 1, 1 - 2 + 1) = (3, 0)
    cin = 16
    x = np.zeros((1, 5, 5, cin))
    x[0, 2, 1, 3] = 1.0
    w = np.zeros((1, 9 * cin))
    w[0, (0 * 3 + 2) * cin + 3] = 2.0
    y = vae_ref.conv3x3(torch.tensor(x), w).numpy()[0, :, :, 0]
    assert y[3, 0] == 2.0 and np.count_nonzero(y) == 1


def test_channel_norm_closed_form_and_invariants():
    rng = np.random.default_rng(3)
    for cols in (16, 96, 384):
        x = (rng.standard_normal((500, cols)) * rng.uniform(0.01, 100, (500, 1))).astype(np.float32)
        g = rng.uniform(0.9, 1.1, cols).astype(np.float32)
        y = orc.channel_norm(x, g, cols).astype(np.float64)
        x64 = x.astype(np.float64)
        ref = x64 / np.linalg.norm(x64, axis=1, keepdims=True) * math.sqrt(cols) * g
        assert np.max(np.abs(y - ref)) <= 2e-6 * np.abs(ref).max()
        # per pixel, ||y / gamma|| = sqrt(C); a scaled input gives the same output
        assert np.allclose(np.linalg.norm(y / g, axis=1), math.sqrt(cols), rtol=2e-6)
        assert np.max(np.abs(orc.channel_norm(4.0 * x, g, cols) - y)) <= 2e-6 * np.abs(y).max()
        ys = orc.channel_norm(x, g, cols, silu=True).astype(np.float64)
        assert np.max(np.abs(ys - ref / (1 + np.exp(-ref)))) <= 4e-6 * np.abs(ref).max()
    # an all-zero row stays zero (the 1e-12 floor of the norm)
    assert np.all(orc.channel_norm(np.zeros((2, 96), np.float32), np.ones(96, np.float32), 96) == 0)


def test_vae_stage_list():
    ups = [s for s in synthetic.VAE_UPSAMPLES if s[0] == "up"]
    assert len(synthetic.VAE_UPSAMPLES) == 15 and len(ups) == 3
    # channel widths chain: each block's cin is the previous output (halved after a resample)
    c = 384
    for s in synthetic.VAE_UPSAMPLES:
        if s[0] == "up":
            assert s[1] == c
            c //= 2
        else:
            assert s[0] == c
            c = s[1]
    assert c == 96


def test_vae_oracle_decode_runs():
    W = synthetic.vae_weights(21)
    lat = orc.randn(9, 16 * 4 * 4).reshape(16, 4, 4)
    out, img = vae_ref.decode(W, lat, synthetic.VAE_UPSAMPLES)
    assert out.shape == (32, 32, 3) and img.shape == (32, 32, 4) and np.all(np.isfinite(out))
    assert np.all(img[..., 3] == 255)


def test_to_rgba_matches_js_semantics():
    # Math.round: nearest, ties toward +inf (x = 0 -> 127.5 -> 128; np.round would agree there, so
    # ties are also pinned directly below); clamp to [-1, 1]; NaN -> 0 (Uint8ClampedArray); alpha 255
    x = np.array([[[0.0, -1.0, 1.0], [5.0, -7.0, np.nan], [-0.5, 0.5, 0.999]]], np.float32)
    img = vae_ref.to_rgba(x)
    assert img.tolist() == [[[128, 0, 255, 255], [255, 0, 0, 255], [64, 191, 255, 255]]]

    def js_round(t):  # the spec's definition, one value at a time
        f = math.floor(t)
        return f + 1 if t - f >= 0.5 else f

    rng = np.random.default_rng(5)
    v = rng.uniform(-1.2, 1.2, (1, 4000, 3)).astype(np.float32)
    got = vae_ref.to_rgba(v)[0, :, :3]
    ref = [[js_round((min(1.0, max(-1.0, float(a))) + 1.0) / 2.0 * 255.0) for a in row] for row in v[0]]
    assert got.tolist() == ref
    # ties: the helper rounds 2.5 -> 3 and 3.5 -> 4 (banker's rounding would give 2 and 4)
    assert js_round(2.5) == 3 and js_round(3.5) == 4
