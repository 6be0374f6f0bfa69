"""The torch fp32 restatement used as the CPU baseline (oracle/torch_ref.py) computes the same
attention as the C oracle the GPU parity tests use: its q/k RMSNorm + rotate-half RoPE + SDPA
(tools/reference.py:93-111, 174-187, 214-230) against orc.qk_norm_rope + the float64 attention, and
its 3D RoPE table against the C restatement of app/models/common.js:31-52."""

import numpy as np
import pytest

import oracle as orc

torch = pytest.importorskip("torch")
from oracle import torch_ref  # noqa: E402


def test_torch_rope_table_matches_c_oracle():
    Hp, Wp = 6, 10
    cos, sin = torch_ref.dit_rope(Hp, Wp)  # [L, 128], split-half duplicated
    L = Hp * Wp
    cs = orc.dit_rope_table(Hp, Wp)
    c_cos, c_sin = cs[: L * 64].reshape(L, 64), cs[L * 64:].reshape(L, 64)
    assert np.allclose(cos[:, :64].numpy(), c_cos, atol=2e-6) and np.allclose(cos[:, 64:].numpy(), c_cos, atol=2e-6)
    assert np.allclose(sin[:, :64].numpy(), c_sin, atol=2e-6) and np.allclose(sin[:, 64:].numpy(), c_sin, atol=2e-6)


def test_torch_self_attention_matches_c_oracle():
    B, Hp, Wp, H, D = 2, 6, 8, 3, 128
    L = Hp * Wp
    rng = np.random.default_rng(12)
    qkv = rng.standard_normal((B, L, 3 * H * D)).astype(np.float32)
    qn = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    cos, sin = torch_ref.dit_rope(Hp, Wp)
    with torch.no_grad():
        got = torch_ref.self_attention(torch.tensor(qkv), torch.tensor(qn), torch.tensor(kn), cos, sin, H, D).numpy()
    cs = orc.dit_rope_table(Hp, Wp)
    ld = 3 * H * D
    ref = np.empty((B, L, H * D), np.float32)
    for b in range(B):
        x = orc.qk_norm_rope(qkv[b], L, H, D, ld, qn, kn, cs, L * 64)
        ref[b] = orc.attention("f64", x, x, x, B=1, Lq=L, Lk=L, H=H, D=D, ldq=ld, ldk=ld, ldv=ld, q_off=0,
                               k_off=H * D, v_off=2 * H * D)[0]
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err < 1e-5, err
    # the comparison notices a RoPE that rotates interleaved pairs (2i, 2i+1) instead of (i, i+64)
    def rotate_interleaved(t):
        out = torch.empty_like(t)
        out[..., 0::2], out[..., 1::2] = -t[..., 1::2], t[..., 0::2]
        return out

    saved = torch_ref.rotate_half
    try:
        torch_ref.rotate_half = rotate_interleaved
        with torch.no_grad():
            bad = torch_ref.self_attention(torch.tensor(qkv), torch.tensor(qn), torch.tensor(kn), cos, sin, H, D).numpy()
    finally:
        torch_ref.rotate_half = saved
    assert np.linalg.norm(bad - ref) / np.linalg.norm(ref) > 1e-2
