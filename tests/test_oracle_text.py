"""CPU pinning of the text-side oracle restatements (oracle/qwen3_ref.py, oracle/adapter_ref.py):
the causal GQA softmax against the C oracle's attention with kv_len (query i = attention over
keys 0..i), the RoPE table against the reference's formula and rotation invariants, RMSNorm
against its closed form."""

import math

import numpy as np

import oracle as orc
from oracle import qwen3_ref as q3


def test_causal_gqa_matches_c_oracle_truncation():
    rng = np.random.default_rng(0)
    L, H, KH, Dh = 9, 4, 2, 128
    q = rng.standard_normal((L, H, Dh))
    k = rng.standard_normal((L, KH, Dh))
    v = rng.standard_normal((L, KH, Dh))
    got = q3.causal_gqa(q, k, v, H // KH)
    for i in range(L):
        ref = orc.attention("f64", q[i].reshape(1, H * Dh).astype(np.float32), k.reshape(L, KH * Dh).astype(np.float32),
                            v.reshape(L, KH * Dh).astype(np.float32), B=1, Lq=1, Lk=L, H=H, D=Dh, ldq=H * Dh,
                            ldk=KH * Dh, ldv=KH * Dh, group=H // KH, kv_len=np.array([i + 1], np.int32))[0, 0]
        assert np.allclose(got[i].reshape(-1), ref, rtol=1e-5, atol=1e-5), i
    # the first query sees only key 0: its output is v[0] of its kv head
    assert np.allclose(got[0, 0], v[0, 0]) and np.allclose(got[0, H - 1], v[0, KH - 1])


def test_rope_table_and_rotation():
    L, Dh, theta = 40, 128, 1e6
    c, s = q3.rope_table(L, Dh, theta)
    # position 0 is the identity; angle(l, i) = l * fround(theta^(-2i/Dh)) (app/models/common.js:15-22)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    for l, i in ((1, 0), (7, 3), (39, 63)):
        ang = np.float32(l * float(np.float32(1.0 / theta ** ((2 * i) / Dh))))
        assert c[l, i] == np.float32(math.cos(ang)) and s[l, i] == np.float32(math.sin(ang))
    # rotation preserves each (i, i + Dh/2) pair's norm and gives relative-position dot products
    rng = np.random.default_rng(1)
    x = rng.standard_normal((L, 1, Dh))
    y = q3.rope(x, c, s)
    h = Dh // 2
    assert np.allclose(x[..., :h] ** 2 + x[..., h:] ** 2, y[..., :h] ** 2 + y[..., h:] ** 2)
    a, b = rng.standard_normal(Dh), rng.standard_normal(Dh)
    ca, sa = q3.rope_table(12, Dh, theta)
    rot = lambda vec, p: q3.rope(np.tile(vec, (12, 1, 1)), ca, sa)[p, 0]
    assert abs(rot(a, 5) @ rot(b, 3) - rot(a, 9) @ rot(b, 7)) < 1e-4  # depends on 5-3 = 9-7 only


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 64))
    w = rng.uniform(0.5, 1.5, 64)
    y = q3.rmsnorm(x, w)
    assert np.allclose(y, x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6) * w)
    assert np.allclose(q3.rmsnorm(1000.0 * x, w), y, rtol=1e-6)  # scale-invariant up to eps


def test_adapter_attention_matches_c_oracle():
    from oracle import adapter_ref as ad

    rng = np.random.default_rng(3)
    Lq, Lk = 5, 11
    q = rng.standard_normal((Lq, ad.H, ad.HD))
    k = rng.standard_normal((Lk, ad.H, ad.HD))
    v = rng.standard_normal((Lk, ad.H, ad.HD))
    got = ad._attn(q, k, v).reshape(Lq, ad.H * ad.HD)
    ref = orc.attention("f64", q.reshape(Lq, -1).astype(np.float32), k.reshape(Lk, -1).astype(np.float32),
                        v.reshape(Lk, -1).astype(np.float32), B=1, Lq=Lq, Lk=Lk, H=ad.H, D=ad.HD, ldq=ad.H * ad.HD,
                        ldk=ad.H * ad.HD, ldv=ad.H * ad.HD)[0]
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)
