"""GPU parity of the VAE decoder's ops and of the whole decoder (the last rank-4 "next" component):

  * channel norm (app/gpu/kernels.js:62-89 mode 1) bit-exact against the C oracle, and within 1e-6
    with the SiLU (exp rounding);
  * conv3x3 (implicit GEMM on the bf16 matrix cores, fused 2x upsample, bias, residual) against the
    float64 convolution (oracle/vae_ref.py, pinned by a direct loop): fp32 precision (activations as
    two bf16 terms) rel L2 <= 3e-5, bf16 <= 1e-2;
  * attention with head dim 384 on the chunked path (app/gpu/ops.js:177-207) against float64,
    including several score chunks, B = 2 with valid key lengths and GQA heads;
  * VAEDecoder.decode through the JS host against the float64 decoder on the same seeded weights:
    fp32 precision rel L2 <= 1e-3 with RGBA bytes within 1, bf16 precision reported and <= 5e-2.
"""

import json
import math
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from helpers import RUN_CASE, amd, report

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def bf16_bits(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bits(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("cols", [16, 96, 192, 384, 500])
def test_channel_norm_matches_oracle(cols):
    m = amd()
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((1000, cols)) * rng.uniform(0.1, 10, (1000, 1))).astype(np.float32)
    x[7] = 0.0
    g = rng.uniform(0.9, 1.1, cols).astype(np.float32)
    with m.Context() as ctx:
        dx, dg, dy = ctx.upload(x), ctx.upload(g), ctx.empty(x.shape)
        for silu in (False, True):
            print(f"[case] channel_norm cols={cols} silu={silu}", flush=True)
            ctx.channel_norm(dx, dg, dy, 1000, cols, silu)
            got, ref = dy.numpy(), orc.channel_norm(x, g, cols, silu)
            if silu:
                assert report(f"channel_norm+silu cols={cols}", got, ref)[1] <= 1e-6 * np.abs(ref).max()
            else:
                assert np.array_equal(got, ref)
        for b in (dx, dg, dy):
            b.release()


CONV_CASES = [  # B, H, W (output), cin, cout, up, resid
    (1, 16, 16, 16, 384, False, False),
    (2, 13, 11, 96, 3, False, True),
    (1, 32, 24, 192, 96, True, False),
    (1, 20, 20, 384, 192, True, True),
    # spatial tiles (16 x 32 pixels x 96 channels, input halo in LDS): borders, several tiles and
    # images, residual, upsample, several channel steps and column tiles
    (2, 32, 64, 96, 96, False, True),
    (1, 32, 32, 192, 192, True, False),
    (1, 16, 32, 384, 384, False, False),
    (1, 16, 32, 96, 3, False, True),  # one 32-wide column tile for 3 channels (the head)
    (1, 32, 64, 64, 32, True, False),
]


@pytest.mark.parametrize("case", CONV_CASES)
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_conv3x3_matches_float64(case, precision):
    from oracle import vae_ref

    m = amd()
    B, H, W, cin, cout, up, resid = case
    rng = np.random.default_rng(hash(case) % 1000)
    Hi, Wi = (H // 2, W // 2) if up else (H, W)
    x = rng.standard_normal((B, Hi, Wi, cin)).astype(np.float32)
    w = from_bits(bf16_bits(rng.uniform(-1, 1, (cout, 9 * cin)) * math.sqrt(3.0 / (9 * cin))))
    bias = rng.uniform(-0.1, 0.1, cout).astype(np.float32)
    c0 = rng.standard_normal((B, H, W, cout)).astype(np.float32)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    print(f"[case] conv3x3 {case} {precision}", flush=True)
    with m.Context() as ctx:
        dx, dw, db = ctx.upload(x), ctx.upload(bf16_bits(w)), ctx.upload(bias)
        do = ctx.upload(c0) if resid else ctx.empty((B, H, W, cout))
        ctx.conv3x3(dx, dw, do, B=B, H=H, W=W, cin=cin, cout=cout, up=up, bias=db, resid=resid, precision=prec)
        got = do.numpy()
        for b in (dx, dw, db, do):
            b.release()
    ref = vae_ref.conv3x3(torch.tensor(x, dtype=torch.float64), w, bias, up=up).numpy()
    if resid:
        ref = ref + c0
    r, _ = report(f"conv3x3 {case} {precision} vs float64", got, ref)
    assert r <= (3e-5 if precision == "fp32" else 1e-2)


ATTN_CASES = [  # B, Lq, Lk, H, group, D, kv_len
    (1, 300, 300, 1, 1, 384, None),
    (2, 256, 200, 2, 2, 384, [200, 77]),
    (1, 2304, 16384, 1, 1, 384, None),  # one 2304 x 16384 score chunk
    (1, 96, 150, 3, 1, 96, None),
]


@pytest.mark.parametrize("case", ATTN_CASES)
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_chunked_attention_matches_float64(case, precision):
    m = amd()
    B, Lq, Lk, H, group, D, kv_len = case
    Hk = H // group
    rng = np.random.default_rng(Lq + Lk)
    q = rng.standard_normal((B, Lq, H * D)).astype(np.float32)
    k = rng.standard_normal((B, Lk, Hk * D)).astype(np.float32)
    v = rng.standard_normal((B, Lk, Hk * D)).astype(np.float32)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    print(f"[case] chunked attention {case} {precision}", flush=True)
    with m.Context() as ctx:
        dq, dk, dv, do = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((B, Lq, H * D))
        ctx.attention(q=dq, k=dk, v=dv, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D, ldk=Hk * D, ldv=Hk * D,
                      group=group, kv_len=kv_len, precision=prec)
        got = do.numpy()
        for b in (dq, dk, dv, do):
            b.release()
    for b in range(B):
        n = kv_len[b] if kv_len else Lk
        for h in range(H):
            hk = h // group
            qh = torch.tensor(q[b, :, h * D:(h + 1) * D], dtype=torch.float64)
            kh = torch.tensor(k[b, :n, hk * D:(hk + 1) * D], dtype=torch.float64)
            vh = torch.tensor(v[b, :n, hk * D:(hk + 1) * D], dtype=torch.float64)
            ref = (torch.softmax(qh @ kh.T / math.sqrt(D), -1) @ vh).numpy()
            r, _ = report(f"chunked attention b={b} h={h} {precision} vs float64", got[b, :, h * D:(h + 1) * D], ref)
            assert r <= (2e-5 if precision == "fp32" else 1e-2)


def _attn_rows_f64(q, k, v, rows, D, causal, n=None):
    """float64 softmax(q k^T / sqrt(D)) v for the given query rows of one head (keys < n; with
    causal, keys <= row as well)."""
    n = k.shape[0] if n is None else n
    out = []
    for i in rows:
        lim = min(n, i + 1) if causal else n
        s = (k[:lim].astype(np.float64) @ q[i].astype(np.float64)) / math.sqrt(D)
        p = np.exp(s - s.max())
        out.append(p @ v[:lim].astype(np.float64) / p.sum())
    return np.array(out)


@pytest.mark.parametrize("D", [64, 96])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_chunked_attention_causal_gqa(D, precision):
    """The causal mask (app/gpu/ops.js:196, kernels.js:49: limit = min(cols, row + 1)) on the
    chunked path (D = 96) and on the flash kernels with zero-padded operands (D = 64), with GQA (4
    query heads over 2 kv heads), B = 2 with a ragged valid key length, and Lq != Lk: every query
    row against a float64 restatement."""
    m = amd()
    B, Lq, Lk, H, group = 2, 150, 190, 4, 2
    Hk = H // group
    kv_len = [190, 120]
    rng = np.random.default_rng(D)
    q = rng.standard_normal((B, Lq, H * D)).astype(np.float32)
    k = rng.standard_normal((B, Lk, Hk * D)).astype(np.float32)
    v = rng.standard_normal((B, Lk, Hk * D)).astype(np.float32)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    print(f"[case] chunked causal GQA attention D={D} {precision}", flush=True)
    with m.Context() as ctx:
        dq, dk, dv, do = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((B, Lq, H * D))
        ctx.attention(q=dq, k=dk, v=dv, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D, ldk=Hk * D, ldv=Hk * D,
                      group=group, kv_len=kv_len, precision=prec, causal=1)
        got = do.numpy()
        for b_ in (dq, dk, dv, do):
            b_.release()
    for b in range(B):
        for h in range(H):
            hk = h // group
            sl, kl = slice(h * D, (h + 1) * D), slice(hk * D, (hk + 1) * D)
            ref = _attn_rows_f64(q[b, :, sl], k[b, :, kl], v[b, :, kl], range(Lq), D, True, kv_len[b])
            r, _ = report(f"causal b={b} h={h} D={D} {precision} vs float64", got[b, :, sl], ref)
            assert r <= (2e-5 if precision == "fp32" else 1e-2)
    # query 0 sees key 0 only
    for h in range(H):
        hk = h // group
        assert np.allclose(got[:, 0, h * D:(h + 1) * D], v[:, 0, hk * D:(hk + 1) * D], rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("causal", [0, 1])
def test_chunked_attention_two_score_chunks(causal):
    """Lq = 4500 queries over Lk = 65536 keys: 4096 score rows fit the 1 GiB chunk, so the product
    runs in two chunks (4096 + 404 rows).  Rows on both sides of the boundary and the last ones
    against float64, plain and causal (the causal limit follows the absolute query index)."""
    m = amd()
    B, Lq, Lk, H, D = 1, 4500, 65536, 1, 8
    rng = np.random.default_rng(7 + causal)
    q = rng.standard_normal((Lq, D)).astype(np.float32)
    k = rng.standard_normal((Lk, D)).astype(np.float32)
    v = rng.standard_normal((Lk, D)).astype(np.float32)
    print(f"[case] chunked attention two score chunks causal={causal}", flush=True)
    with m.Context() as ctx:
        dq, dk, dv, do = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((Lq, D))
        ctx.attention(q=dq, k=dk, v=dv, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=D, ldq=D, ldk=D, ldv=D,
                      precision=m.PREC_FP32, causal=causal)
        got = do.numpy()
        for b_ in (dq, dk, dv, do):
            b_.release()
    rows = [0, 1, 2, 4094, 4095, 4096, 4097, Lq - 2, Lq - 1]
    ref = _attn_rows_f64(q, k, v, rows, D, bool(causal))
    r, _ = report(f"two chunks causal={causal} vs float64", got[rows], ref)
    assert r <= 2e-5


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
@pytest.mark.timeout(600)
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_vae_decode_through_js_matches_float64(tmp_path, precision):
    from oracle import synthetic, vae_ref

    h = w = 16
    seed = 21
    lat = orc.randn(31, 16 * h * w).reshape(16, h, w)
    lp = str(tmp_path / "lat.bin")
    lat.tofile(lp)
    out = str(tmp_path / "vae")
    spec = {"case": "vae", "seed": seed, "latent": lp, "h": h, "w": w, "precision": precision, "out": out}
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print(f"[case] js vae decode 16x16 -> 128x128 {precision}", flush=True)
    r = subprocess.run(["node", RUN_CASE, str(tmp_path / "case.json")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"vae"' in ln))["vae"]
    assert info["width"] == 8 * w and info["height"] == 8 * h and len(info["stages"]) == 16
    raw = np.fromfile(out + ".raw", np.float32).reshape(8 * h, 8 * w, 3)
    img = np.fromfile(out + ".img", np.uint8).reshape(8 * h, 8 * w, 4)
    ref, ref_img = vae_ref.decode(synthetic.vae_weights(seed), lat, synthetic.VAE_UPSAMPLES)
    rr, _ = report(f"vae decode ({precision}) vs float64", raw, ref)
    d = np.abs(img.astype(int) - ref_img.astype(int))
    print(f"vae image bytes: max |d| {d.max()}, {np.count_nonzero(d)} of {d.size} differ", flush=True)
    assert np.all(np.isfinite(raw))
    # the device's RGBA conversion is the reference loop's arithmetic: exact on the device's own output
    assert np.array_equal(img, vae_ref.to_rgba(raw))
    if precision == "fp32":
        assert rr <= 1e-3 and d.max() <= 1
    else:
        assert rr <= 5e-2


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
@pytest.mark.timeout(600)
def test_pipeline_generate_decodes_reports_progress_and_cancels(tmp_path):
    """LatentPipeline.generate with a VAE (app/pipeline.js:225-292): per-block sampling progress
    with increasing fractions, decode progress, the image of the final latent (equal to a separate
    decode of it), and an AbortError when the signal is raised mid-generation."""
    from oracle import synthetic, vae_ref

    out = str(tmp_path / "p")
    spec = {"case": "pipeline", "blocks": 2, "size": 128, "steps": 3, "Lk": 64, "out": out}
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print("[case] js pipeline generate + decode 128x128, 2 blocks, 3 steps", flush=True)
    r = subprocess.run(["node", RUN_CASE, str(tmp_path / "case.json")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"pipeline"' in ln))["pipeline"]
    ev = info["events"]
    sample = [e for e in ev if e["phase"] == "sample"]
    decode = [e for e in ev if e["phase"] == "decode"]
    assert len(sample) == 3 * 2 and [e["frac"] for e in sample] == sorted(e["frac"] for e in sample)
    assert abs(sample[-1]["frac"] - 1.0) < 1e-9 and decode[0]["frac"] == 0 and decode[-1]["frac"] == 1
    assert info["image"] == [128, 128]
    assert info["cancel"] is not None and info["cancel"]["name"] == "AbortError"
    lat = np.fromfile(out + ".latent", np.float32).reshape(16, 16, 16)
    img = np.fromfile(out + ".img", np.uint8).reshape(128, 128, 4)
    _, ref_img = vae_ref.decode(synthetic.vae_weights(21), lat, synthetic.VAE_UPSAMPLES)
    assert np.abs(img.astype(int) - ref_img.astype(int)).max() <= 1
