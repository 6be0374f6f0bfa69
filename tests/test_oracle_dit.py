"""Pins of the DiT-step oracle (oracle/dit_ref.py) and of the synthetic-weight restatement
(oracle/synthetic.py), independent of the oracle's own formulas:

  * timestep_embedding (app/models/dit.js:41-51) against the float64 closed form, torch's float32
    evaluation of tools/reference.py:203-206, and the JS host's common.mjs through node;
  * the block composition (dit.js:261-315, reference.py:231-242) by invariants a wrong shift /
    scale / gate chunk offset would break: all gates 0 => the block is the identity; shift 0 and
    scale -1 (a zero modulated row) => the self-attention and MLP sublayers add nothing and the
    cross-attention sublayer adds one row per batch element (uniform attention over the context);
  * time_cond's sum adaln_lora[:n] + W2 W1 silu(emb): W2 = 0 leaves the lora chunks, and the final
    layer takes the first 2D entries;
  * the seeded fill: splitmix64 against Vigna's published outputs for state 0, and the documented
    value ranges / moments of each kind.
"""

import json
import math
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from helpers import PKG_DIR
from oracle import dit_ref, synthetic

D = 2048


def test_timestep_embedding_closed_form():
    for sigma in (0.0, 0.03, 0.5, 0.9, 1.0):
        t = dit_ref.timestep_embedding(sigma).astype(np.float64)
        i = np.arange(1024, dtype=np.float64)
        a = sigma * np.exp(-math.log(10000.0) * i / 1024)
        ref = np.concatenate([np.cos(a), np.sin(a)])
        # the reference rounds f and sigma*f to float32 (two roundings of |a| <= 1): <= 3e-7
        assert np.max(np.abs(t - ref)) <= 3e-7
        # cos half first, sin half second, frequency 1 at index 0 (a swapped half or a shifted
        # index fails by O(sigma))
        assert abs(t[0] - math.cos(sigma)) <= 1e-7 and abs(t[1024] - math.sin(sigma)) <= 1e-7


def test_timestep_embedding_torch_reference_formula():
    torch = pytest.importorskip("torch")
    for sigma in (0.1, 0.77, 1.0):
        freqs = torch.exp(-math.log(10000) * torch.arange(1024).float() / 1024)
        temb = sigma * freqs
        ref = torch.cat([temb.cos(), temb.sin()]).numpy()
        assert np.max(np.abs(dit_ref.timestep_embedding(sigma) - ref)) <= 2.5e-7


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_timestep_embedding_matches_js_host():
    js = (f"import {{ timestepEmbedding }} from '{PKG_DIR}/js/common.mjs';"
          "console.log(JSON.stringify(Array.from(timestepEmbedding(0.6180339887))));")
    r = subprocess.run(["node", "--input-type=module", "-e", js], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    got = np.array(json.loads(r.stdout), np.float32)
    ref = dit_ref.timestep_embedding(0.6180339887)
    # the same rounding points; Math.exp / Math.cos may differ from libm by an ulp of float64
    assert np.max(np.abs(got.view(np.int32) - ref.view(np.int32))) <= 1


@pytest.fixture(scope="module")
def one_block():
    """Synthetic one-block W (int8), B=2 prompts of 16 tokens, 8 context tokens."""
    W = synthetic.dit_weights(11, "int8", 1)
    B, Hp, Wp, Lk = 2, 4, 4, 8
    L = Hp * Wp
    x = orc.randn(5, B * L * D).reshape(B * L, D)
    ctx = dit_ref.prepare_context([orc.randn(6 + b, Lk * 1024).reshape(Lk, 1024) for b in range(B)])
    cs = orc.dit_rope_table(Hp, Wp)
    return W, B, L, x, ctx, cs


def _mods(rng, shift=None, scale=None, gate=None):
    out = []
    for _ in range(3):
        m = rng.standard_normal(3 * D).astype(np.float32) * 0.5
        if shift is not None:
            m[:D] = shift
        if scale is not None:
            m[D:2 * D] = scale
        if gate is not None:
            m[2 * D:] = gate
        out.append(m)
    return out


def test_block_gates_zero_is_identity(one_block):
    W, B, L, x, ctx, cs = one_block
    rng = np.random.default_rng(1)
    y = dit_ref.dit_block("w8a8", W, 0, x, _mods(rng, gate=0.0), cs, ctx, B, L)
    assert np.array_equal(y, x)
    # the same modulation with nonzero gates changes every sublayer's output
    y2 = dit_ref.dit_block("w8a8", W, 0, x, _mods(np.random.default_rng(1)), cs, ctx, B, L)
    assert not np.array_equal(y2, x)


def test_block_zero_modulated_rows(one_block):
    W, B, L, x, ctx, cs = one_block
    rng = np.random.default_rng(2)
    ms, mc, mm = _mods(rng, shift=0.0, scale=-1.0, gate=1.0)
    mc[2 * D:] = 0.0
    # self-attention and MLP on zero rows add exactly nothing
    y = dit_ref.dit_block("w8a8", W, 0, x, (ms, mc, mm), cs, ctx, B, L)
    assert np.array_equal(y, x)
    # cross-attention on a zero query row attends uniformly: the same added row for every token
    ms[2 * D:] = 0.0
    mm[2 * D:] = 0.0
    mc[2 * D:] = 1.0
    y = dit_ref.dit_block("w8a8", W, 0, x, (ms, mc, mm), cs, ctx, B, L)
    d = (y.astype(np.float64) - x).reshape(B, L, D)
    assert np.abs(d).max() > 0
    for b in range(B):
        assert np.abs(d[b] - d[b, :1]).max() <= 1e-6 * np.abs(d[b]).max() + 1e-6
    # with shift and scale swapped (scale 0, shift -1) the rows are not zero and the added rows vary
    mc[:D], mc[D:2 * D] = -1.0, 0.0
    y = dit_ref.dit_block("w8a8", W, 0, x, (ms, mc, mm), cs, ctx, B, L)
    d = (y.astype(np.float64) - x).reshape(B, L, D)
    assert np.abs(d[0] - d[0, :1]).max() > 1e-3 * np.abs(d[0]).max()


def test_time_cond_lora_chunks():
    W = synthetic.dit_weights(12, "int8", 2)
    for i in range(2):
        for nm in ("adaln_modulation_self_attn", "adaln_modulation_cross_attn", "adaln_modulation_mlp"):
            W[f"blocks.{i}.{nm}.2.weight"] = np.zeros_like(W[f"blocks.{i}.{nm}.2.weight"])
    W["final_layer.adaln_modulation.2.weight"] = np.zeros_like(W["final_layer.adaln_modulation.2.weight"])
    mods, mf = dit_ref.time_cond(W, 2, 0.4)
    temb = dit_ref.timestep_embedding(0.4)[None].astype(np.float64)
    w1 = dit_ref.bf16_to_f32(W["t_embedder.1.linear_1.weight"]).astype(np.float64)
    w2 = dit_ref.bf16_to_f32(W["t_embedder.1.linear_2.weight"]).astype(np.float64)
    h = temb @ w1.T
    lora = ((h / (1 + np.exp(-h))) @ w2.T)[0]
    for blk in mods:
        for m in blk:
            assert np.max(np.abs(m - lora[:3 * D])) <= 1e-5 * np.abs(lora).max()
    assert mf.shape == (2 * D,) and np.max(np.abs(mf - lora[:2 * D])) <= 1e-5 * np.abs(lora).max()


def test_splitmix64_known_answers():
    # Vigna's splitmix64.c from state 0: the state advances by 0x9e3779b97f4a7c15 per output
    golden = 0x9E3779B97F4A7C15
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    got = [orc.splitmix64_next((k * golden) & (2 ** 64 - 1)) for k in range(3)]
    assert got == want


def test_fill_kinds_ranges_and_moments():
    n = 1 << 18
    u8 = orc.fill_random(n, "u8", 7, 0x60, 0x6F)
    assert u8.min() == 0x60 and u8.max() == 0x6F
    i8 = orc.fill_random(n, "i8n", 7, 40, 0).astype(np.float64)
    # (sum of 4 bytes - 510) is symmetric about 0; the arithmetic shift floors, so the mean is -1/2
    assert abs(i8.std() - 40) < 0.5 and abs(i8.mean() + 0.5) < 0.3 and np.abs(i8).max() <= 127
    f = orc.fill_random(n, "f32", 7, -0.25, 0.75).astype(np.float64)
    assert f.min() >= -0.25 and f.max() < 0.75 and abs(f.mean() - 0.25) < 3e-3
    b = dit_ref.bf16_to_f32(orc.fill_random(n, "bf16", 7, -0.25, 0.75)).astype(np.float64)
    assert np.max(np.abs(b - f)) <= 2.0 ** -9  # the same draws, rounded to bf16
    g = orc.fill_random(n, "f32n", 7, 2.0, 1.0).astype(np.float64)
    assert abs(g.mean() - 1.0) < 0.02 and abs(g.std() - 2.0) < 0.02
    # seeds are independent streams: a different seed gives different draws
    assert not np.array_equal(orc.fill_random(64, "u8", 8, 0, 255), orc.fill_random(64, "u8", 9, 0, 255))


def test_synthetic_names_follow_js_source():
    # the FNV-1a name hash of js/weights.mjs (32-bit offset basis 0x811c9dc5, prime 0x01000193)
    assert synthetic.fnv1a32("") == 0x811C9DC5
    assert synthetic.fnv1a32("a") == 0xE40C292C
    assert synthetic.fnv1a32("foobar") == 0xBF9CF968
    W = synthetic.dit_weights(3, "w4a8", 3)
    assert "blocks.1.self_attn.q_proj.weight_codebook" in W and "blocks.0.self_attn.k_proj.weight_scale" in W
    assert W["blocks.1.self_attn.v_proj.weight"].shape == (D, D // 2)
    assert W["blocks.2.mlp.layer2.weight"].shape == (D, 8192)
