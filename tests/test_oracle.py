"""Pins the CPU oracle (oracle/oracle.c) against independent statements of the same math:
library routines (torch.randn, torch float8, torch SDPA, torch layer_norm, numpy int64 matmul,
numpy Kronecker products), the C++ standard's mt19937 known answer, closed forms and
invariants.  No test here retypes the oracle's own formula.
"""

import math

import numpy as np
import pytest

import oracle as orc

# torch is imported lazily: the GPU test process collects this module too, and torch's bundled
# HIP runtime must not be the one libanima.so binds to.
torch = None
F = None


@pytest.fixture(autouse=True)
def _torch():
    global torch, F
    import torch as _t
    import torch.nn.functional as _F

    torch, F = _t, _F


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ------------------------------------------------------------------ RNG (app/rng.js)

def test_mt19937_known_answer():
    # C++11 [rand.predef]: the 10000th consecutive invocation of a default-constructed
    # std::mt19937 (seed 5489) produces 4123659995.
    assert int(orc.mt19937(5489, 10000)[-1]) == 4123659995


@pytest.mark.parametrize("seed,n", [(0, 16), (1, 17), (42, 100), (7, 1000), (123, 65543)])
def test_randn_matches_torch(seed, n):
    torch.manual_seed(seed)
    ref = torch.randn(n).numpy()
    got = orc.randn(seed, n)
    # app/rng.js:1-3: identical stream, values agree to ~2e-6 (vectorized log/cos in torch)
    assert np.max(np.abs(got - ref)) < 2e-5


# ------------------------------------------------------------------ fp8 / W4 (tools/quant.py)

def test_fp8e4m3_all_codes_match_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    for b in range(256):
        if b in (0x7F, 0xFF):
            # e4m3fn NaN encodings: the reference's closed form (gemm.js:144-151) decodes them
            # as +-480; the quantizer never emits them (s_rel <= 448).
            assert orc.fp8e4m3(b) == (480.0 if b == 0x7F else -480.0)
            continue
        assert orc.fp8e4m3(b) == ref[b], b


FIXED_LUT = (-0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
             0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671)


def test_w4_decode_matches_torch_grid_levels():
    rng = np.random.default_rng(3)
    N, K = 24, 128
    codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    # every finite positive e4m3 code, plus the sizes the quantizer emits
    srel = rng.integers(1, 0x7F, size=(N, K // 16), dtype=np.uint8)
    srel[0, : min(K // 16, 8)] = np.array([0x01, 0x08, 0x38, 0x40, 0x70, 0x7E, 0x30, 0x5A], np.uint8)[: min(K // 16, 8)]
    cb = np.array(FIXED_LUT, np.float32)
    got = orc.w4_decode(codes, srel, cb, N, K)
    # torch statement of tools/quant.py:172-182 (dequantize_w4a8 before the channel scale)
    packed = torch.from_numpy(codes).to(torch.int32)
    c = torch.empty(N, K, dtype=torch.int32)
    c[:, 0::2] = packed & 0xF
    c[:, 1::2] = (packed >> 4) & 0xF
    vals = torch.from_numpy(cb)[c].view(N, K // 16, 16)
    s = torch.from_numpy(srel).view(torch.float8_e4m3fn).float().unsqueeze(-1)
    ref = (vals * s).round().clamp(-127, 127).view(N, K).to(torch.int8).numpy()
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ Hadamard (quant.py:30-45)

def kron_h256():
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.float64)
    h = h4
    for _ in range(3):
        h = np.kron(h, h4)
    return h / 16.0


def test_hadamard_matches_kron_and_is_involution():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((12, 512)).astype(np.float32)
    H = kron_h256()
    assert np.allclose(H, H.T) and np.allclose(H @ H, np.eye(256))
    y = orc.hadamard256(x)
    ref = (x.astype(np.float64).reshape(-1, 256) @ H.T).reshape(x.shape)
    assert np.max(np.abs(y - ref)) < 1e-5
    # H.H = I (quant.py:83) and Parseval
    assert np.max(np.abs(orc.hadamard256(y) - x)) < 1e-5
    assert abs(np.linalg.norm(y) - np.linalg.norm(x)) / np.linalg.norm(x) < 1e-6
    # e_0 maps to row 0 of H (all +1/16)
    e0 = np.zeros(256, np.float32)
    e0[0] = 1
    assert np.array_equal(orc.hadamard256(e0), np.full(256, 0.0625, np.float32) * np.sign(H[0]))


# ------------------------------------------------------------------ RoPE (common.js / reference.py)

def test_dit_rope_angles_formula():
    Hp, Wp = 5, 7
    a = orc.dit_rope_angles(Hp, Wp)
    # tools/reference.py:174-187 in float64 numpy (independent of the JS fround chain)
    dim_h = 42
    sp = np.arange(0, dim_h, 2)[: dim_h // 2] / dim_h
    h_theta = 10000.0 * 4.0 ** (dim_h / (dim_h - 2))
    hf = 1.0 / h_theta ** sp
    hh, ww = np.meshgrid(np.arange(Hp), np.arange(Wp), indexing="ij")
    ref = np.concatenate([np.zeros((Hp * Wp, 22)), hh.reshape(-1, 1) * hf, ww.reshape(-1, 1) * hf], 1)
    assert np.max(np.abs(a - ref)) < 1e-5
    assert np.all(a[:, :22] == 0)
    # hf[0] = 1 exactly: slot 22 is the row index, slot 43 the column index
    assert np.array_equal(a[:, 22], hh.reshape(-1).astype(np.float32))
    assert np.array_equal(a[:, 43], ww.reshape(-1).astype(np.float32))


def np_rms_rope(x, w, cos, sin, eps=1e-6):
    """tools/reference.py:93-99, 215-216, 227-229 in float64: rms_norm then q*cos + rotate_half(q)*sin."""
    x = x.astype(np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w
    c = np.concatenate([cos, cos], -1)
    s = np.concatenate([sin, sin], -1)
    h = y.shape[-1] // 2
    rot = np.concatenate([-y[..., h:], y[..., :h]], -1)
    return y * c + rot * s


def test_qk_norm_rope_matches_reference_formulation():
    L, H, D = 12, 3, 128
    rng = np.random.default_rng(1)
    qkv = rng.standard_normal((L, 3 * H * D)).astype(np.float32)
    qn = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    ang = orc.dit_rope_angles(3, 4)
    cs = orc.rope_table(ang)
    out = orc.qk_norm_rope(qkv, L, H, D, 3 * H * D, qn, kn, cs, L * 64)
    cos, sin = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
    for part, w in ((0, qn), (1, kn)):
        x = qkv[:, part * H * D:(part + 1) * H * D].reshape(L, H, D)
        ref = np_rms_rope(x, w, cos[:, None, :], sin[:, None, :])
        got = out[:, part * H * D:(part + 1) * H * D].reshape(L, H, D)
        assert np.max(np.abs(got - ref)) < 2e-5
    # v untouched
    assert np.array_equal(out[:, 2 * H * D:], qkv[:, 2 * H * D:])


def test_rope_relative_position_property():
    # <R_m q, R_n k> depends only on m - n per axis (here along the width axis)
    Hp, Wp, D = 1, 16, 128
    cs = orc.dit_rope_table(Hp, Wp)
    rng = np.random.default_rng(2)
    q = rng.standard_normal(D).astype(np.float32)
    k = rng.standard_normal(D).astype(np.float32)
    Q = orc.rope(np.tile(q, (Wp, 1)), cs, Wp, 1, D, Wp * 64)
    K = orc.rope(np.tile(k, (Wp, 1)), cs, Wp, 1, D, Wp * 64)
    d1 = float(Q[5] @ K[2])
    d2 = float(Q[12] @ K[9])
    assert abs(d1 - d2) < 1e-4 * (np.linalg.norm(q) * np.linalg.norm(k))
    # norm preserving
    assert abs(np.linalg.norm(Q[7]) - np.linalg.norm(q)) < 1e-5 * np.linalg.norm(q)


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((9, 128)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    y = orc.rmsnorm(x, w, 128)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(y - ref)) < 1e-5


def test_layernorm_mod_matches_torch_layer_norm():
    rng = np.random.default_rng(5)
    cols = 512
    x = (rng.standard_normal((6, cols)) * 3 + 1).astype(np.float32)
    mod = (0.1 * rng.standard_normal(3 * cols)).astype(np.float32)
    ln = F.layer_norm(torch.from_numpy(x).double(), (cols,), eps=1e-6).numpy()
    ref = ln * (1 + mod[cols:2 * cols]) + mod[:cols]
    y = orc.layernorm_mod(x, mod, 0, cols, cols, rotate=False)
    assert np.max(np.abs(y - ref)) < 2e-5
    yr = orc.layernorm_mod(x, mod, 0, cols, cols, rotate=True)
    refr = (ref.reshape(-1, 256) @ kron_h256().T).reshape(ref.shape)
    assert np.max(np.abs(yr - refr)) < 2e-5


# ------------------------------------------------------------------ attention

def sdpa_f64(q, k, v, scale=None):
    """torch SDPA (tools/reference.py:109-111) in float64; q [H,Lq,D], k/v [H,Lk,D]."""
    return F.scaled_dot_product_attention(torch.from_numpy(q).double()[None], torch.from_numpy(k).double()[None],
                                          torch.from_numpy(v).double()[None], scale=scale)[0].numpy()


def make_qkv(rng, B, L, H, D):
    return rng.standard_normal((B, L, 3 * H * D)).astype(np.float32)


@pytest.mark.parametrize("kind", ["f64", "wgsl", "bf16"])
def test_attention_matches_torch_sdpa(kind):
    rng = np.random.default_rng(6)
    B, L, H, D = 2, 40, 2, 128
    qkv = make_qkv(rng, B, L, H, D)
    kv_len = np.array([40, 17], np.int32)
    o = orc.attention(kind, qkv, qkv, qkv, B=B, Lq=L, Lk=L, H=H, D=D, ldq=3 * H * D, ldk=3 * H * D, ldv=3 * H * D,
                      q_off=0, k_off=H * D, v_off=2 * H * D, kv_len=kv_len)
    for b in range(B):
        x = qkv[b].reshape(L, 3, H, D)
        n = kv_len[b]
        q = x[:, 0].transpose(1, 0, 2)
        k = x[:n, 1].transpose(1, 0, 2)
        v = x[:n, 2].transpose(1, 0, 2)
        if kind == "bf16":
            q, k, v = orc.bf16_round(q), orc.bf16_round(k), orc.bf16_round(v)
        ref = sdpa_f64(np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v))
        got = o[b].reshape(L, H, D).transpose(1, 0, 2)
        tol = {"f64": 1e-7, "wgsl": 2e-6, "bf16": 6e-3}[kind]  # f64 output is stored as fp32
        assert rel_l2(got, ref) < tol, (kind, b, rel_l2(got, ref))


def test_attention_invariants():
    rng = np.random.default_rng(7)
    H, D, Lq, Lk = 1, 128, 8, 33
    q = rng.standard_normal((Lq, D)).astype(np.float32)
    k = rng.standard_normal((Lk, D)).astype(np.float32)
    v = rng.standard_normal((Lk, D)).astype(np.float32)
    args = dict(B=1, Lq=Lq, Lk=Lk, H=H, D=D, ldq=D, ldk=D, ldv=D)
    for kind in ("f64", "wgsl", "bf16"):
        # every model normalizes by the sum of the weights it applies: convex combinations
        rtol = 1e-6
        # V = const -> O = const
        vc = np.full_like(v, 0.75)
        assert np.allclose(orc.attention(kind, q, k, vc, **args), 0.75, rtol=rtol, atol=0)
        # one key -> O = V
        o1 = orc.attention(kind, q, k, v, **{**args, "Lk": 1})
        ref = orc.bf16_round(v[0]) if kind == "bf16" else v[0]
        assert np.allclose(o1[0], np.tile(ref, (Lq, 1)), rtol=rtol, atol=1e-7)
        # key permutation equivariance
        perm = rng.permutation(Lk)
        a = orc.attention(kind, q, k, v, **args)
        b = orc.attention(kind, q, k[perm], v[perm], **args)
        assert rel_l2(a, b) < (2e-6 if kind != "f64" else 1e-12)


def test_bf16_round_known_values():
    x = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -3.14159265, 65504.0, 1e-40], np.float32)
    got = orc.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, ref)
    assert orc.lib().orc_bf16_round(1.00390625) == 1.0  # tie -> even
    assert orc.lib().orc_bf16_round(1.005859375) == float(torch.tensor(1.005859375).bfloat16().float())


# ------------------------------------------------------------------ per-token quant + int8 GEMM

def test_token_quant_properties():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((33, 256)).astype(np.float32) * rng.uniform(0.1, 10, size=(33, 1)).astype(np.float32)
    x[5] = 0
    q, s = orc.token_quant(x)
    assert q.dtype == np.int8 and np.all(np.abs(q.astype(int)) <= 127)
    assert s[5] == 0 and np.all(q[5] == 0)
    nz = np.arange(33) != 5
    # |x - s q| <= s/2, the amax element maps to +-127
    err = np.abs(x[nz] - s[nz, None] * q[nz].astype(np.float32))
    assert np.all(err <= s[nz, None] * 0.5 * (1 + 1e-5))
    am = np.argmax(np.abs(x[nz]), 1)
    assert np.all(np.abs(q[nz][np.arange(nz.sum()), am]) == 127)
    # idempotent on its own grid
    q2, s2 = orc.token_quant(s[:, None] * q.astype(np.float32))
    assert np.array_equal(q2, q)
    # the definition in numpy float32: s = amax/127, q = clip(rint(x * (127/amax)))
    amax = np.abs(x).max(1).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.float32(127.0) / amax
    qn = np.where(amax[:, None] == 0, 0, np.clip(np.rint(x * inv[:, None]), -127, 127)).astype(np.int8)
    assert np.array_equal(s, amax / np.float32(127.0)) and np.array_equal(q, qn)


def test_gemm_i8_matches_int64_matmul():
    rng = np.random.default_rng(9)
    qx = rng.integers(-127, 128, size=(17, 320)).astype(np.int8)
    qw = rng.integers(-128, 128, size=(23, 320)).astype(np.int8)
    ref = qx.astype(np.int64) @ qw.astype(np.int64).T
    assert np.array_equal(orc.gemm_i8(qx, qw).astype(np.int64), ref)


def test_gelu_silu_against_math():
    for x in np.linspace(-6, 6, 97):
        ref = 0.5 * x * (1 + math.erf(x / math.sqrt(2)))
        assert abs(orc.gelu(float(x)) - ref) < 2e-7 * max(1.0, abs(x)) + 1e-7
        assert abs(orc.silu(float(x)) - x / (1 + math.exp(-x))) < 1e-6 * max(1.0, abs(x))


def test_linear_epilogue_modes():
    rng = np.random.default_rng(10)
    acc = rng.integers(-(1 << 20), 1 << 20, size=(5, 7)).astype(np.int32)
    sx = rng.uniform(0.01, 1, 5).astype(np.float32)
    sw = rng.uniform(0.01, 1, 7).astype(np.float32)
    base = (acc.astype(np.float32) * sx[:, None]) * sw[None, :]
    assert np.array_equal(orc.linear_epilogue(acc, sx, sw), base)
    c0 = rng.standard_normal((5, 7)).astype(np.float32)
    assert np.array_equal(orc.linear_epilogue(acc, sx, sw, epi=1, c=c0), c0 + base)
    gate = rng.standard_normal(20).astype(np.float32)
    got = orc.linear_epilogue(acc, sx, sw, epi=2, gate=gate, g_off=3, c=c0)
    ref = (c0.astype(np.float64) + gate[3:10].astype(np.float64) * base.astype(np.float64))
    assert np.max(np.abs(got - ref)) < 1e-5 * np.max(np.abs(ref))
