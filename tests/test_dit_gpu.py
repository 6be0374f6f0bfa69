"""Full DiT step parity through the JavaScript host (js/dit.mjs -> N-API -> libanima.so).

A 3-block Anima DiT (block 0 and 2 int8, block 1 W4 -- the "mixed" layout of
tools/build_assets.py:119 at 3 blocks) is written as a comfy_quant safetensors checkpoint with
seeded random weights, loaded by js/weights.mjs, and run for one B=2 step (cond + uncond contexts)
at 256x256 (32x32 latent, 256 tokens).  The velocities and the residual stream after block 0 are
compared with the numpy/C oracle of the same step (oracle/dit_ref.py):
  * W8A8 semantics (this build's arithmetic): rel L2 <= 5e-3, the reference's own bar for
    dit_block0 / denoised0 (tools/check.js:103, 109);
  * the reference's W8A32 + fp32-attention semantics: reported, bounded by 5e-2.
"""

import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from helpers import RUN_CASE, report

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]

D, CTX, MLP, R = 2048, 1024, 8192, 256
FIXED_LUT = np.array([-0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
                      0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671], np.float32)


def save_safetensors(path, tensors):
    """Minimal safetensors writer (8-byte header size, JSON header, raw little-endian data)."""
    header, chunks, off = {}, [], 0
    for name, (dtype, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        chunks.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for c in chunks:
            f.write(c)


def meta(fmt, **kw):
    return np.frombuffer(json.dumps({"format": fmt, **kw}).encode(), np.uint8)


def fitted_codebook(rng):
    """A 16-level codebook of the shape tools/quant.py:98-113 fits (sorted, spanning about [-1, 1]);
    its values differ from FIXED_LUT, so linears carrying it cannot share a stacked W4 weight."""
    cb = np.sort(rng.uniform(-0.95, 0.95, 16)).astype(np.float32)
    cb[0], cb[-1] = -1.0, 1.0
    return cb


def make_checkpoint(path, nblocks, seed=0, distinct_qkv_codebooks=False):
    """comfy_quant checkpoint of an nblocks DiT (int8 first / last block, W4 between).  With
    distinct_qkv_codebooks the W4 blocks give self-attention q FIXED_LUT and k, v two different
    fitted codebooks (tools/quant.py:116-124 picks a codebook per linear), so concatLinears cannot
    stack them (app/weights.js:155-158)."""
    rng = np.random.default_rng(seed)
    T = {}
    W = {}

    def bf16(name, N, K, gain=1.0):
        a = gain * np.sqrt(3.0 / K)
        w = orc.bf16_round(rng.uniform(-a, a, size=(N, K)).astype(np.float32))
        u = (w.view(np.uint32) >> 16).astype(np.uint16)
        T[name] = ("BF16", u)
        W[name] = u

    def f32(name, arr):
        T[name] = ("F32", arr.astype(np.float32))
        W[name] = arr.astype(np.float32)

    def quant(base, N, K, kind, codebook=FIXED_LUT):
        scale = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
        if kind == "i8":
            q = np.clip(np.rint(40 * rng.standard_normal((N, K))), -127, 127).astype(np.int8)
            T[base + "weight"], W[base + "weight"] = ("I8", q), q
            f32(base + "weight_scale", scale.reshape(N, 1))
            m = meta("int8_tensorwise", convrot=True, convrot_groupsize=256)
        else:
            codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
            srel = rng.integers(0x60, 0x70, size=(N, K // 16), dtype=np.uint8)
            T[base + "weight"], W[base + "weight"] = ("I8", codes.view(np.int8)), codes.view(np.int8)
            T[base + "weight_s_rel"], W[base + "weight_s_rel"] = ("F8_E4M3", srel), srel
            f32(base + "weight_s_channel", scale)
            f32(base + "weight_codebook", codebook)
            m = meta("asym_w4a8_int8", group_size=16, convrot=True, convrot_groupsize=256)
        T[base + "comfy_quant"], W[base + "comfy_quant"] = ("U8", m), m

    bf16("x_embedder.proj.1.weight", D, 68)
    bf16("t_embedder.1.linear_1.weight", D, D)
    bf16("t_embedder.1.linear_2.weight", 3 * D, D)
    f32("t_embedding_norm.weight", 1 + 0.02 * rng.standard_normal(D))
    for i in range(nblocks):
        p = f"blocks.{i}."
        kind = "i8" if i in (0, nblocks - 1) else "w4"
        for nm in ("adaln_modulation_self_attn", "adaln_modulation_cross_attn", "adaln_modulation_mlp"):
            bf16(p + nm + ".1.weight", R, D)
            bf16(p + nm + ".2.weight", 3 * D, R, 0.5)
        for t in "qkv":
            cb = fitted_codebook(rng) if distinct_qkv_codebooks and t != "q" else FIXED_LUT
            quant(p + f"self_attn.{t}_proj.", D, D, kind, cb)
        quant(p + "self_attn.output_proj.", D, D, kind)
        quant(p + "cross_attn.q_proj.", D, D, kind)
        quant(p + "cross_attn.k_proj.", D, CTX, kind)
        quant(p + "cross_attn.v_proj.", D, CTX, kind)
        quant(p + "cross_attn.output_proj.", D, D, kind)
        for a in ("self_attn", "cross_attn"):
            f32(p + a + ".q_norm.weight", 1 + 0.02 * rng.standard_normal(128))
            f32(p + a + ".k_norm.weight", 1 + 0.02 * rng.standard_normal(128))
        quant(p + "mlp.layer1.", MLP, D, kind)
        quant(p + "mlp.layer2.", D, MLP, kind)
    bf16("final_layer.adaln_modulation.1.weight", R, D)
    bf16("final_layer.adaln_modulation.2.weight", 2 * D, R, 0.5)
    bf16("final_layer.linear.weight", 64, D)
    save_safetensors(path, T)
    return W


def run_dit_case(tmp_path, W, ck, nblocks, h, w, Lk, sigma):
    """Writes seeded latents / contexts, runs AnimaDiT.load -> timeCond -> prepareContext -> forward
    through js (tests/js/run_case.mjs), returns (latents, contexts, velocities, block-0 residual,
    per-block stacked flags)."""
    lat = [orc.randn(201 + b, 16 * h * w).reshape(16, h, w) for b in range(2)]
    ctx = [orc.randn(211 + b, Lk * CTX).reshape(Lk, CTX) for b in range(2)]
    files = {}
    for b in range(2):
        files[f"lat{b}"] = str(tmp_path / f"lat{b}.bin")
        lat[b].tofile(files[f"lat{b}"])
        files[f"ctx{b}"] = str(tmp_path / f"ctx{b}.bin")
        ctx[b].tofile(files[f"ctx{b}"])
    out = str(tmp_path / "v")
    spec = {"case": "dit", "weights": ck, "blocks": nblocks, "sigma": sigma, "Lk": Lk, "h": h, "w": w,
            "ctx": [files["ctx0"], files["ctx1"]], "latents": [files["lat0"], files["lat1"]], "out": out}
    (tmp_path / "case.json").write_text(json.dumps(spec))
    r = subprocess.run(["node", RUN_CASE, str(tmp_path / "case.json")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    got = [np.fromfile(out + f".{b}", np.float32).reshape(16, h, w) for b in range(2)]
    got_b0 = np.fromfile(out + ".block0", np.float32)
    stacked = json.loads(open(out + ".stacked.json").read())
    return lat, ctx, got, got_b0, stacked


def test_dit_step_unstacked_qkv_through_js_matches_oracle(tmp_path):
    """The unstacked self-attention projection (app/models/dit.js:274-288): the W4 block's q, k and v
    carry three different codebooks, so they load as three linears writing column slices of one
    QKV buffer; the step still matches the oracle at the reference's bar (tools/check.js:103,109)."""
    nblocks, h, w, Lk, sigma = 3, 32, 32, 512, 0.9
    print("[case] dit 3 blocks, W4 block with distinct q/k/v codebooks, 256x256 B=2 via js", flush=True)
    ck = str(tmp_path / "dit.safetensors")
    W = make_checkpoint(ck, nblocks, seed=3, distinct_qkv_codebooks=True)
    cbs = [W[f"blocks.1.self_attn.{t}_proj.weight_codebook"] for t in "qkv"]
    assert not np.array_equal(cbs[0], cbs[1]) and not np.array_equal(cbs[1], cbs[2])
    lat, ctx, got, got_b0, stacked = run_dit_case(tmp_path, W, ck, nblocks, h, w, Lk, sigma)
    assert stacked == [True, False, True]

    from oracle import dit_ref

    ref, ref_b0 = dit_ref.dit_step(W, nblocks, lat, h, w, ctx, sigma, mode="w8a8")
    assert np.all(np.isfinite(np.stack(got)))
    rb0, _ = report("dit_block0 vs W8A8 oracle", got_b0, ref_b0.reshape(-1))
    rv, _ = report("velocity (unstacked W4 q/k/v in block 1) vs W8A8 oracle", np.stack(got), np.stack(ref))
    assert rb0 < 5e-3 and rv < 5e-3


def test_dit_step_through_js_matches_oracle(tmp_path):
    nblocks, h, w, Lk, sigma = 3, 32, 32, 512, 0.9
    print("[case] dit 3 blocks (int8/W4/int8) 256x256 B=2 via js", flush=True)
    ck = str(tmp_path / "dit.safetensors")
    W = make_checkpoint(ck, nblocks)
    lat, ctx, got, got_b0, stacked = run_dit_case(tmp_path, W, ck, nblocks, h, w, Lk, sigma)
    assert stacked == [True, True, True]

    from oracle import dit_ref

    ref, ref_b0 = dit_ref.dit_step(W, nblocks, lat, h, w, ctx, sigma, mode="w8a8")
    assert np.all(np.isfinite(np.stack(got)))
    rb0, _ = report("dit_block0 vs W8A8 oracle", got_b0, ref_b0.reshape(-1))
    rv, _ = report("velocity vs W8A8 oracle", np.stack(got), np.stack(ref))
    assert rb0 < 5e-3 and rv < 5e-3
    sem, sem_b0 = dit_ref.dit_step(W, nblocks, lat, h, w, ctx, sigma, mode="ref")
    rs, _ = report("velocity vs reference W8A32 + fp32 attention", np.stack(got), np.stack(sem))
    report("dit_block0 vs reference W8A32 + fp32 attention", got_b0, sem_b0.reshape(-1))
    assert rs < 5e-2
