"""GPU parity of the attention path through the C ABI (libanima.so) against the CPU oracle.

Inputs are seeded with the torch.randn restatement (oracle.randn) at the shapes of the
workloads: N=1024 single attention (B=1), N=4096 self-attention (B=2) and 4096x512
cross-attention with per-batch valid key lengths (B=2).  Tolerances (stated per test):
  fp32-MFMA kernel vs fp64 brute force:          rel L2 <= 1e-5, max|d| <= 1e-4
  fp32-MFMA kernel vs the WGSL-order fp32 oracle: rel L2 <= 1e-5
  bf16-MFMA kernel vs the bf16 numerics model:    rel L2 <= 3e-4
  bf16-MFMA kernel vs fp64 brute force:           rel L2 <= 1e-2 (bf16 operand rounding)
Row kernels (qk_norm_rope, rmsnorm, rope) are bit-exact against the oracle.
"""

import numpy as np
import pytest

import oracle as orc
from helpers import amd, rel_l2, max_abs, report

pytestmark = pytest.mark.gpu

HD = 128


@pytest.fixture(scope="module")
def ctx():
    m = amd()
    c = m.Context(0)
    yield c
    c.close()


def case(msg):
    print(f"[case] {msg}", flush=True)


def norm_weights(seed):
    qn = (1 + 0.02 * orc.randn(seed, HD)).astype(np.float32)
    kn = (1 + 0.02 * orc.randn(seed + 1, HD)).astype(np.float32)
    return qn, kn


def fused_inputs(seed, B, Hp, Wp, H=16):
    L = Hp * Wp
    qkv = orc.randn(seed, B * L * 3 * H * HD).reshape(B, L, 3 * H * HD)
    qn, kn = norm_weights(seed + 100)
    cs = orc.dit_rope_table(Hp, Wp)
    return qkv, qn, kn, cs, L


def cpu_norm_rope(qkv, qn, kn, cs, L, H):
    return np.stack([orc.qk_norm_rope(qkv[b], L, H, HD, 3 * H * HD, qn, kn, cs, L * 64) for b in range(qkv.shape[0])])


def run_fused(ctx, qkv, qn, kn, cs, L, H, precision):
    m = amd()
    B = qkv.shape[0]
    d_qkv = ctx.upload(qkv)
    d_qn, d_kn, d_cs = ctx.upload(qn), ctx.upload(kn), ctx.upload(cs)
    d_o = ctx.empty((B, L, H * HD))
    ld = 3 * H * HD
    ctx.attention(q=d_qkv, k=d_qkv, v=d_qkv, o=d_o, B=B, Lq=L, Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld,
                  q_off=0, k_off=H * HD, v_off=2 * H * HD, precision=precision,
                  q_norm=d_qn, k_norm=d_kn, rope_cs=d_cs, rope_sin_off=L * 64)
    out = d_o.numpy()
    for b in (d_qkv, d_qn, d_kn, d_cs, d_o):
        b.release()
    return out


def oracle_rows(kind, nqkv, b, rows, L, H):
    """Oracle attention for the query rows `rows` of batch b (all heads) of a normalized qkv."""
    ld = 3 * H * HD
    q = np.ascontiguousarray(nqkv[b, rows])
    kv = np.ascontiguousarray(nqkv[b])
    o = orc.attention(kind, q, kv, kv, B=1, Lq=len(rows), Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld,
                      q_off=0, k_off=H * HD, v_off=2 * H * HD)
    return o[0]


# ------------------------------------------------------------------ row kernels (bit-exact)

def test_row_kernels_bit_exact(ctx):
    case("qk_norm_rope / rmsnorm / rope, L=256 H=16")
    qkv, qn, kn, cs, L = fused_inputs(11, 1, 16, 16)
    x = qkv[0]
    d = ctx.upload(x)
    d_qn, d_kn, d_cs = ctx.upload(qn), ctx.upload(kn), ctx.upload(cs)
    ctx.qk_norm_rope(d, L, 16, HD, 3 * 16 * HD, d_qn, d_kn, d_cs, L * 64)
    got = d.numpy()
    ref = orc.qk_norm_rope(x, L, 16, HD, 3 * 16 * HD, qn, kn, cs, L * 64)
    assert np.array_equal(got, ref), report("qk_norm_rope", got, ref)

    rows = np.ascontiguousarray(x[:, :2048]).reshape(-1, 128)
    dx, dy = ctx.upload(rows), ctx.empty(rows.shape)
    ctx.rmsnorm(dx, d_qn, dy, rows.shape[0], 128)
    assert np.array_equal(dy.numpy(), orc.rmsnorm(rows, qn, 128))
    wide = np.ascontiguousarray(x[:, :2048])
    w2 = (1 + 0.1 * orc.randn(5, 2048)).astype(np.float32)
    dx2, dy2, dw2 = ctx.upload(wide), ctx.empty(wide.shape), ctx.upload(w2)
    ctx.rmsnorm(dx2, dw2, dy2, L, 2048)
    assert np.array_equal(dy2.numpy(), orc.rmsnorm(wide, w2, 2048))

    xr = ctx.upload(x)
    ctx.rope(xr, d_cs, L, 16, HD, L * 64, row_stride=3 * 16 * HD, col_off=16 * HD)
    assert np.array_equal(xr.numpy(), orc.rope(x, cs, L, 16, HD, L * 64, 3 * 16 * HD, 16 * HD))


# ------------------------------------------------------------------ single attention, N=1024

@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_attention_n1024_fused(ctx, precision):
    case(f"attention B=1 N=1024 H=16 fused norm+rope {precision}")
    m = amd()
    H = 16
    qkv, qn, kn, cs, L = fused_inputs(1, 1, 32, 32, H)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    got = run_fused(ctx, qkv, qn, kn, cs, L, H, prec)[0]
    nqkv = cpu_norm_rope(qkv, qn, kn, cs, L, H)
    rows = np.arange(0, L, 3)  # every third query row, all heads
    ref64 = oracle_rows("f64", nqkv, 0, rows, L, H)
    r, mx = report(f"{precision} vs fp64", got[rows], ref64)
    if precision == "fp32":
        assert r <= 1e-5 and mx <= 1e-4
        wg = oracle_rows("wgsl", nqkv, 0, rows, L, H)
        assert report("fp32 vs wgsl-order", got[rows], wg)[0] <= 1e-5
    else:
        assert r <= 1e-2
        model = oracle_rows("bf16", nqkv, 0, rows, L, H)
        assert report("bf16 vs bf16 model", got[rows], model)[0] <= 3e-4


# ------------------------------------------------------------------ self-attention, N=4096, B=2

@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_attention_n4096_b2_fused(ctx, precision):
    case(f"attention B=2 N=4096 H=16 fused norm+rope {precision}")
    m = amd()
    H = 16
    qkv, qn, kn, cs, L = fused_inputs(2, 2, 64, 64, H)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    got = run_fused(ctx, qkv, qn, kn, cs, L, H, prec)
    nqkv = cpu_norm_rope(qkv, qn, kn, cs, L, H)
    rng = np.random.default_rng(0)
    rows = np.unique(np.concatenate([np.arange(0, 32), rng.choice(L, 48, replace=False), np.arange(L - 32, L)]))
    for b in range(2):
        ref64 = oracle_rows("f64", nqkv, b, rows, L, H)
        r, mx = report(f"b={b} {precision} vs fp64", got[b, rows], ref64)
        if precision == "fp32":
            assert r <= 1e-5 and mx <= 1e-4
        else:
            assert r <= 1e-2
            model = oracle_rows("bf16", nqkv, b, rows, L, H)
            assert report(f"b={b} bf16 vs model", got[b, rows], model)[0] <= 3e-4
    assert np.all(np.isfinite(got))


def test_attention_constant_v_full_size(ctx):
    """Size-independent property at N=4096, B=2: V == c for every key -> O == c."""
    case("attention B=2 N=4096 constant V")
    m = amd()
    H = 16
    qkv, qn, kn, cs, L = fused_inputs(3, 2, 64, 64, H)
    qkv[:, :, 2 * H * HD:] = 0.625
    for prec, tol in ((m.PREC_BF16, 1e-5), (m.PREC_FP32, 1e-5)):
        got = run_fused(ctx, qkv, qn, kn, cs, L, H, prec)
        assert np.max(np.abs(got - 0.625)) <= tol * 0.625, (prec, np.max(np.abs(got - 0.625)))


# ------------------------------------------------------------------ cross-attention 4096 x 512

def test_prepared_kv_size_is_checked(ctx):
    """A prepared K/V buffer is only accepted with the byte count of its layout: K/V prepared in
    bf16 and passed to an fp32 call, or to a call with a shorter Lk, and a prepare_into whose
    kv_prep_bytes does not match, are refused on the host with ANIMA_E_ARG before any launch."""
    case("prepared K/V size checks (host-side refusals)")
    m = amd()
    B, Lq, Lk, H = 1, 256, 256, 2
    q = ctx.upload(orc.randn(41, B * Lq * H * HD))
    k = ctx.upload(orc.randn(42, B * Lk * H * HD))
    o = ctx.empty((B, Lq, H * HD))
    nb16 = m.Context.attention_kv_bytes(B, H, Lk, m.PREC_BF16)
    assert m.Context.attention_kv_bytes(B, H, Lk, m.PREC_FP32) != nb16
    prep = ctx.empty(m.Context.attention_kv_bytes(B, H, Lk, m.PREC_FP32), np.uint8)
    common = dict(B=B, Lq=Lq, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD)
    ctx.attention(q=q, k=k, v=k, o=o, Lk=Lk, prepare_into=prep, precision=m.PREC_BF16, **common)
    for kw in (dict(Lk=Lk, precision=m.PREC_FP32), dict(Lk=Lk - 64, precision=m.PREC_BF16)):
        with pytest.raises(m.AnimaError) as e:
            ctx.attention(q=q, k=None, v=None, o=o, kv_prep=prep, kv_prep_bytes=nb16, **common, **kw)
        assert e.value.code == -1, kw
    with pytest.raises(m.AnimaError) as e:
        ctx.attention(q=q, k=k, v=k, o=o, Lk=Lk, prepare_into=prep, kv_prep_bytes=nb16 - 256,
                      precision=m.PREC_BF16, **common)
    assert e.value.code == -1
    # the right size is accepted
    ctx.attention(q=q, k=None, v=None, o=o, Lk=Lk, kv_prep=prep, kv_prep_bytes=nb16, precision=m.PREC_BF16, **common)
    ctx.sync()
    for x in (q, k, o, prep):
        x.release()


@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_cross_attention_masked(ctx, precision):
    """Masked cross-attention against fp64 / the bf16 model; the same call on K/V prepared once
    by anima_attention_prepare_kv is bit-identical."""
    case(f"cross-attention B=2 Lq=4096 Lk=512 kv_len mask {precision}")
    m = amd()
    B, Lq, Lk, H = 2, 4096, 512, 16
    q = orc.randn(21, B * Lq * H * HD).reshape(B, Lq, H * HD)
    k = orc.randn(22, B * Lk * H * HD).reshape(B, Lk, H * HD)
    v = orc.randn(23, B * Lk * H * HD).reshape(B, Lk, H * HD)
    qn, kn = norm_weights(24)
    rng = np.random.default_rng(25)
    kv_len = rng.integers(64, Lk + 1, size=B).astype(np.int32)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dqn, dkn = ctx.upload(qn), ctx.upload(kn)
    do = ctx.empty((B, Lq, H * HD))
    ctx.attention(q=dq, k=dk, v=dv, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD,
                  kv_len=kv_len, precision=prec, q_norm=dqn, k_norm=dkn)
    got = do.numpy()
    # K/V converted once (anima_attention_prepare_kv) and reused: the same output, bit for bit
    prep = ctx.empty(m.Context.attention_kv_bytes(B, H, Lk, prec), np.uint8)
    common = dict(B=B, Lq=Lq, Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD, kv_len=kv_len, precision=prec,
                  q_norm=dqn, k_norm=dkn)
    ctx.attention(q=dq, k=dk, v=dv, o=do, prepare_into=prep, **common)
    do2 = ctx.empty((B, Lq, H * HD))
    for _ in range(2):
        ctx.attention(q=dq, k=None, v=None, o=do2, kv_prep=prep, **common)
        assert np.array_equal(do2.numpy(), got)
    for x in (dq, dk, dv, dqn, dkn, do, do2, prep):
        x.release()
    rows = np.unique(np.concatenate([np.arange(0, 16), rng.choice(Lq, 48, replace=False), np.arange(Lq - 16, Lq)]))
    for b in range(B):
        qb = orc.rmsnorm(q[b, rows].reshape(-1, HD), qn, HD).reshape(len(rows), H * HD)
        kb = orc.rmsnorm(k[b].reshape(-1, HD), kn, HD).reshape(Lk, H * HD)
        args = dict(B=1, Lq=len(rows), Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD, kv_len=kv_len[b:b + 1])
        ref64 = orc.attention("f64", qb, kb, v[b], **args)[0]
        r, mx = report(f"b={b} Lv={kv_len[b]} {precision} vs fp64", got[b, rows], ref64)
        if precision == "fp32":
            assert r <= 1e-5 and mx <= 1e-4
        else:
            assert r <= 1e-2
            model = orc.attention("bf16", qb, kb, v[b], **args)[0]
            assert report(f"b={b} bf16 vs model", got[b, rows], model)[0] <= 3e-4


@pytest.mark.parametrize("L,B,precision", [(300, 1, "bf16"), (300, 1, "fp32"), (1024, 2, "bf16")])
def test_causal_gqa_attention(ctx, L, B, precision):
    """Causal GQA attention, the text encoder's form (app/models/qwen3.js:60: Lq = Lk, H = 16 query
    heads over 8 kv heads; causal softmax limit = min(Lk, row + 1), app/gpu/kernels.js:49).  Query
    i attends to keys 0..i, which is the oracle's attention over the first i + 1 keys: each sampled
    query row is a batch element of the oracle (shared K/V, stride 0) with kv_len = i + 1.  L = 300
    spans three 128-query tiles and ends in a partial key block; L = 1024 at B = 2 is a grid the
    8-wave kernel would otherwise take."""
    case(f"causal GQA attention L={L} B={B} H=16/8 {precision}")
    m = amd()
    H, Hkv = 16, 8
    q = orc.randn(31, B * L * H * HD).reshape(B, L, H * HD)
    k = orc.randn(32, B * L * Hkv * HD).reshape(B, L, Hkv * HD)
    v = orc.randn(33, B * L * Hkv * HD).reshape(B, L, Hkv * HD)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    dq, dk, dv, do = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((B, L, H * HD))
    ctx.attention(q=dq, k=dk, v=dv, o=do, B=B, Lq=L, Lk=L, H=H, D=HD, ldq=H * HD, ldk=Hkv * HD, ldv=Hkv * HD,
                  group=H // Hkv, precision=prec, causal=1)
    got = do.numpy()
    for x in (dq, dk, dv, do):
        x.release()
    assert np.isfinite(got).all()
    rng = np.random.default_rng(34)
    rows = np.unique(np.concatenate([np.arange(0, 4), [63, 64, 127, 128, 129, 255, 256], rng.choice(L, 24, replace=False),
                                     [L - 2, L - 1]]))
    rows = rows[rows < L]
    for b in range(B):
        args = dict(B=len(rows), Lq=1, Lk=L, H=H, D=HD, ldq=H * HD, ldk=Hkv * HD, ldv=Hkv * HD, q_bs=H * HD,
                    k_bs=0, v_bs=0, group=H // Hkv, kv_len=(rows + 1).astype(np.int32))
        qr = np.ascontiguousarray(q[b, rows])
        ref64 = orc.attention("f64", qr, k[b], v[b], **args)[:, 0]
        r, mx = report(f"b={b} causal {precision} vs fp64", got[b, rows], ref64)
        if precision == "fp32":
            assert r <= 1e-5 and mx <= 1e-4
        else:
            assert r <= 1e-2
            model = orc.attention("bf16", qr, k[b], v[b], **args)[:, 0]
            assert report(f"b={b} causal bf16 vs model", got[b, rows], model)[0] <= 3e-4
    # query 0 sees key 0 only: its output is v row 0 of its kv head
    for hh in range(H):
        kvh = hh // (H // Hkv)
        assert np.allclose(got[:, 0, hh * HD:(hh + 1) * HD], v[:, 0, kvh * HD:(kvh + 1) * HD], rtol=1e-2 if precision == "bf16" else 1e-6, atol=1e-2 if precision == "bf16" else 1e-6)


@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_head_dim_64_attention(ctx, precision):
    """D = 64, the LLM adapter's attention (app/models/dit.js:147-160: 16 heads x 64 in 1024
    columns; its cross-attention to the text encoder's tokens) on the flash kernels with the
    operands zero-padded to 128 dims (ops.js:170 sends D = 64 to flashAttentionShader), scale 1/8,
    against the oracle (self Lq = Lk = 77 and cross Lq = 32, Lk = 100)."""
    case(f"attention D=64 {precision}")
    m = amd()
    H, D = 16, 64
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    for Lq, Lk, seed in ((77, 77, 41), (32, 100, 42)):
        q = orc.randn(seed, Lq * H * D).reshape(Lq, H * D)
        k = orc.randn(seed + 1, Lk * H * D).reshape(Lk, H * D)
        v = orc.randn(seed + 2, Lk * H * D).reshape(Lk, H * D)
        dq, dk, dv, do = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.empty((Lq, H * D))
        ctx.attention(q=dq, k=dk, v=dv, o=do, B=1, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D, ldk=H * D, ldv=H * D, precision=prec)
        got = do.numpy()
        for x in (dq, dk, dv, do):
            x.release()
        args = dict(B=1, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D, ldk=H * D, ldv=H * D)
        ref = orc.attention("f64", q, k, v, **args)[0]
        r, mx = report(f"D=64 Lq={Lq} Lk={Lk} {precision} vs fp64", got, ref)
        assert r <= (1e-5 if precision == "fp32" else 1e-2)


@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_head_dim_64_flash_path(ctx, precision):
    """D = 64 runs the flash kernels (the profiler names the flash launch, no chunked-path kernel)
    with the operands zero-padded to 128 dims: B = 2 with ragged valid key lengths, GQA (8 query
    heads over 4 kv heads), causal and not, strided rows (the heads of a fused [q | k | v] row),
    every query row against float64 restated on the host, and the padding columns of the output
    rows (other heads' slices) left untouched."""
    m = amd()
    B, Lq, Lk, H, group, D = 2, 200, 333, 8, 2, 64
    Hk = H // group
    kv_len = [333, 90]
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    rng = np.random.default_rng(640)
    ld = (H + 2 * Hk) * D + 64  # q | k | v heads, then 64 spare columns
    for causal in (0, 1):
        case(f"attention D=64 flash path {precision} causal={causal}")
        x = rng.standard_normal((B, max(Lq, Lk), ld)).astype(np.float32)
        dx = ctx.upload(x)
        o0 = np.full((B, Lq, H * D + 64), 7.0, np.float32)
        do = ctx.upload(o0)
        ctx.profile(True)
        ctx.profile_reset()
        ctx.attention(q=dx, k=dx, v=dx, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=D, group=group, ldq=ld, ldk=ld, ldv=ld,
                      ldo=H * D + 64, k_off=H * D, v_off=(H + Hk) * D, q_bstride=max(Lq, Lk) * ld,
                      k_bstride=max(Lq, Lk) * ld, v_bstride=max(Lq, Lk) * ld, o_bstride=Lq * (H * D + 64),
                      kv_len=kv_len, precision=prec, causal=causal)
        names = [r["name"] for r in ctx.profile_report()]
        ctx.profile(False)
        assert any(n.startswith("attn.flash") for n in names) and not any("chunk" in n for n in names), names
        got = do.numpy()
        for x_ in (dx, do):
            x_.release()
        assert np.all(got[:, :, H * D:] == 7.0)  # spare columns untouched
        for b in range(B):
            for h in range(H):
                hk = h // group
                q = x[b, :Lq, h * D:(h + 1) * D].astype(np.float64)
                k = x[b, :kv_len[b], H * D + hk * D:H * D + (hk + 1) * D].astype(np.float64)
                v = x[b, :kv_len[b], (H + Hk) * D + hk * D:(H + Hk) * D + (hk + 1) * D].astype(np.float64)
                s = q @ k.T / 8.0
                if causal:
                    s = np.where(np.arange(kv_len[b])[None, :] <= np.arange(Lq)[:, None], s, -np.inf)
                p = np.exp(s - s.max(-1, keepdims=True))
                ref = (p @ v) / p.sum(-1, keepdims=True)
                r, _ = report(f"D=64 flash b={b} h={h} causal={causal} {precision}", got[b, :, h * D:(h + 1) * D], ref)
                assert r <= (1e-5 if precision == "fp32" else 1e-2)


# ------------------------------------------------------------------ ragged shapes, GQA, strides

@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_attention_ragged_gqa(ctx, precision):
    case(f"attention ragged B=3 Lq=200 Lk=77 group=2 {precision}")
    m = amd()
    B, Lq, Lk, H, group = 3, 200, 77, 4, 2
    Hkv = H // group
    ldq, ldk = H * HD + 8, Hkv * HD + 4  # padded rows
    q = orc.randn(31, B * Lq * ldq).reshape(B, Lq, ldq)
    kv = orc.randn(32, B * Lk * 2 * ldk).reshape(B, Lk, 2 * ldk)
    kv_len = np.array([77, 1, 40], np.int32)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    dq, dkv = ctx.upload(q), ctx.upload(kv)
    do = ctx.empty((B, Lq, H * HD))
    ctx.attention(q=dq, k=dkv, v=dkv, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=HD, group=group, ldq=ldq, ldk=2 * ldk,
                  ldv=2 * ldk, q_off=4, k_off=0, v_off=ldk, kv_len=kv_len, precision=prec, scale=0.05)
    got = do.numpy()
    args = dict(B=B, Lq=Lq, Lk=Lk, H=H, D=HD, group=group, ldq=ldq, ldk=2 * ldk, ldv=2 * ldk, q_off=4, k_off=0,
                v_off=ldk, kv_len=kv_len, scale=0.05)
    ref64 = orc.attention("f64", q, kv, kv, **args)
    r, mx = report(f"{precision} vs fp64", got, ref64)
    if precision == "fp32":
        assert r <= 1e-5 and mx <= 1e-4
    else:
        assert r <= 1e-2
        assert report("bf16 vs model", got, orc.attention("bf16", q, kv, kv, **args))[0] <= 3e-4
    # kv_len == 1: every query returns that key's value row (bf16-rounded V for the bf16 kernel)
    v0 = kv[1, 0, ldk:ldk + Hkv * HD].reshape(Hkv, HD)
    if precision == "bf16":
        v0 = orc.bf16_round(v0)
    exp = np.repeat(v0, group, axis=0).reshape(-1)
    tol = 1e-6
    assert np.allclose(got[1], np.tile(exp, (Lq, 1)), rtol=tol, atol=1e-6)


@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_attention_late_large_scores(ctx, precision):
    """Scores that grow block by block: keys 64-127 align with the queries at 2x, keys 192-255 at
    6x (log2-domain scores ~98, past the 2^64 probability limit of the lazily raised offset) and
    the partial last block at 9x (~147: exp2 overflows to inf before the offset is raised)."""
    case(f"attention late large scores Lq=64 Lk=300 {precision}")
    m = amd()
    H, Lq, Lk = 2, 64, 300
    u = orc.randn(41, H * HD).reshape(H, HD)
    q = (u[None] + 0.1 * orc.randn(42, Lq * H * HD).reshape(Lq, H, HD)).reshape(Lq, H * HD).astype(np.float32)
    gain = np.full(Lk, 0.0, np.float32)
    gain[64:128], gain[192:256], gain[256:] = 2.0, 6.0, 9.0
    k = (0.05 * orc.randn(43, Lk * H * HD).reshape(Lk, H, HD) + gain[:, None, None] * u[None]).reshape(Lk, H * HD)
    k = k.astype(np.float32)
    v = orc.randn(44, Lk * H * HD).reshape(Lk, H * HD)
    prec = m.PREC_FP32 if precision == "fp32" else m.PREC_BF16
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    do = ctx.empty((Lq, H * HD))
    ctx.attention(q=dq, k=dk, v=dv, o=do, B=1, Lq=Lq, Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD,
                  precision=prec)
    got = do.numpy()
    assert np.all(np.isfinite(got))
    args = dict(B=1, Lq=Lq, Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD)
    r, mx = report(f"{precision} vs fp64", got, orc.attention("f64", q, k, v, **args))
    if precision == "fp32":
        # raw scores reach ~1150, whose fp32 spacing (1.2e-4) alone moves a weight by ~1e-5
        assert r <= 1e-4 and mx <= 1e-4
        assert report("fp32 vs WGSL-order oracle", got, orc.attention("wgsl", q, k, v, **args))[0] <= 1e-4
    else:
        # scores this large make the softmax sensitive to the bf16 rounding of Q and K (a 2^-9
        # relative change of a score of ~147 moves its weight by ~20%), so the fp64 distance is
        # only reported; the bar is the bf16 numerics model
        assert report("bf16 vs model", got, orc.attention("bf16", q, k, v, **args))[0] <= 3e-4


def test_attention_8wave_kernel_key_lengths(ctx):
    """16 batches x 16 heads x 256 queries: 256 workgroups of 256 queries, the grid that selects the
    8-wave direct-to-LDS kernel (checked through the profiler name).  Per-batch key lengths cover 1,
    2 and 3+ blocks of 64 with and without a partial tail; batches 8-15 get keys that align with the
    queries at 2x / 6x / 9x in later blocks (the overflow-triggered offset raise)."""
    case("attention 8-wave kernel B=16 H=16 Lq=256 Lk=320 ragged key lengths")
    m = amd()
    B, H, Lq, Lk = 16, 16, 256, 320
    kv_len = np.array([1, 63, 64, 65, 128, 129, 192, 200, 256, 257, 300, 320, 320, 320, 31, 2], np.int32)
    q = orc.randn(51, B * Lq * H * HD).reshape(B, Lq, H, HD)
    k = orc.randn(52, B * Lk * H * HD).reshape(B, Lk, H, HD)
    v = orc.randn(53, B * Lk * H * HD).reshape(B, Lk, H, HD).reshape(B, Lk, H * HD)
    u = orc.randn(54, H * HD).reshape(H, HD)
    gain = np.zeros(Lk, np.float32)
    gain[64:128], gain[192:256], gain[256:] = 2.0, 6.0, 9.0
    q[8:] = u[None, None] + 0.1 * q[8:]
    k[8:] = 0.05 * k[8:] + gain[None, :, None, None] * u[None, None]
    q = q.reshape(B, Lq, H * HD).astype(np.float32)
    k = k.reshape(B, Lk, H * HD).astype(np.float32)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    do = ctx.empty((B, Lq, H * HD))
    ctx.profile(True)
    ctx.profile_reset()
    ctx.attention(q=dq, k=dk, v=dv, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD,
                  kv_len=kv_len, precision=m.PREC_BF16)
    names = {r["name"] for r in ctx.profile_report()}
    ctx.profile(False)
    assert "attn.flash_bf16" in names, names
    got = do.numpy()
    assert np.all(np.isfinite(got))
    args = dict(B=B, Lq=Lq, Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD, kv_len=kv_len)
    model = orc.attention("bf16", q, k, v, **args)
    for b in range(B):
        assert report(f"b={b} kv_len={kv_len[b]} bf16 vs model", got[b], model[b])[0] <= 3e-4
    # batches 0-7 (no contrived scores): the fp64 distance stays at the bf16-operand level
    ref64 = orc.attention("f64", q[:8], k[:8], v[:8], **{**args, "B": 8, "kv_len": kv_len[:8]})
    assert report("b<8 bf16 vs fp64", got[:8], ref64)[0] <= 1e-2


@pytest.mark.parametrize("gqa", [False, True])
def test_attention_8wave_kernel_partial_query_tile(ctx, gqa):
    """B=4 H=16 Lq=1000: 4 x 16 x 4 = 256 workgroups of 256 queries (the 8-wave kernel), the last
    query tile a quarter full (rows past Lq are neither computed into nor stored).  Without GQA:
    fused q/k RMSNorm + RoPE on a 25 x 40 token grid; with GQA (2 query heads per K/V head):
    padded rows, ragged key lengths.  Sampled rows (every 7th and the last 40) against the bf16
    numerics model and float64."""
    case(f"attention 8-wave kernel B=4 H=16 Lq=1000 partial query tile gqa={gqa}")
    m = amd()
    B, H = 4, 16
    rows = np.unique(np.concatenate([np.arange(0, 1000, 7), np.arange(960, 1000)]))
    if not gqa:
        qkv, qn, kn, cs, L = fused_inputs(61, B, 25, 40, H)
        ctx.profile(True)
        ctx.profile_reset()
        got = run_fused(ctx, qkv, qn, kn, cs, L, H, m.PREC_BF16)
        names = {r["name"] for r in ctx.profile_report()}
        ctx.profile(False)
        nqkv = cpu_norm_rope(qkv, qn, kn, cs, L, H)
        for b in range(B):
            model = oracle_rows("bf16", nqkv, b, rows, L, H)
            assert report(f"b={b} bf16 vs model", got[b, rows], model)[0] <= 3e-4
        assert report("b=0 bf16 vs fp64", got[0, rows], oracle_rows("f64", nqkv, 0, rows, L, H))[0] <= 1e-2
    else:
        Lq, Lk, group = 1000, 777, 2
        Hkv = H // group
        ldq, ldk = H * HD + 4, 2 * Hkv * HD + 8
        q = orc.randn(62, B * Lq * ldq).reshape(B, Lq, ldq)
        kv = orc.randn(63, B * Lk * ldk).reshape(B, Lk, ldk)
        kv_len = np.array([777, 500, 64, 1], np.int32)
        dq, dkv = ctx.upload(q), ctx.upload(kv)
        do = ctx.empty((B, Lq, H * HD))
        ctx.profile(True)
        ctx.profile_reset()
        ctx.attention(q=dq, k=dkv, v=dkv, o=do, B=B, Lq=Lq, Lk=Lk, H=H, D=HD, group=group, ldq=ldq, ldk=ldk,
                      ldv=ldk, q_off=0, k_off=0, v_off=Hkv * HD, kv_len=kv_len, precision=m.PREC_BF16)
        names = {r["name"] for r in ctx.profile_report()}
        ctx.profile(False)
        got = do.numpy()
        qs = np.ascontiguousarray(q[:, rows])
        args = dict(B=B, Lq=len(rows), Lk=Lk, H=H, D=HD, group=group, ldq=ldq, ldk=ldk, ldv=ldk, q_off=0, k_off=0,
                    v_off=Hkv * HD, kv_len=kv_len)
        model = orc.attention("bf16", qs, kv, kv, **args)
        for b in range(B):
            assert report(f"b={b} kv_len={kv_len[b]} bf16 vs model", got[b, rows], model[b])[0] <= 3e-4
        ref64 = orc.attention("f64", qs, kv, kv, **args)
        assert report("bf16 vs fp64", got[:, rows], ref64)[0] <= 1e-2
    assert "attn.flash_bf16" in names, names
    assert np.all(np.isfinite(got))


def test_attention_rejects_bad_arguments(ctx):
    case("attention argument validation")
    m = amd()
    d = ctx.empty((64, 3 * 128))
    base = dict(q=d, k=d, v=d, o=d, B=1, Lq=64, Lk=64, H=1, D=128, ldq=384, ldk=384, ldv=384, ldo=384)
    # head dims outside {64, 128} run on the chunked path, which takes D % 4 == 0 and no fused
    # norm / RoPE
    with pytest.raises(m.AnimaError) as e:
        ctx.attention(**{**base, "D": 90, "ldo": 384})
    assert e.value.code == -5
    with pytest.raises(m.AnimaError) as e:
        ctx.attention(**{**base, "D": 96, "q_norm": d})
    assert e.value.code == -5
    with pytest.raises(m.AnimaError) as e:
        ctx.attention(**{**base, "ldq": 386})
    assert e.value.code == -1
    with pytest.raises(m.AnimaError) as e:
        ctx.attention(**{**base, "kv_len": [0]})
    assert e.value.code == -1
    with pytest.raises(m.AnimaError) as e:
        ctx.attention(**{**base, "q_off": 300})
    assert e.value.code == -1
    d.release()


@pytest.mark.parametrize("B,H,Lq,Lk,kernel", [(16, 16, 256, 320, "attn.flash_bf16"), (1, 2, 300, 200, "attn.flash_bf16_4w")])
def test_attention_bf16_output(ctx, B, H, Lq, Lk, kernel):
    """anima_attn_desc.o_bf16: the 8-wave kernel (a grid of one workgroup per CU) and the 4-wave
    kernel write O as bf16, each value the round-to-nearest-even of the fp32 output of the same call
    without it (bit for bit), into a wider row (ldo, o_off in bf16 elements) whose other columns
    stay untouched; refused with fp32 precision and on the chunked path (D = 96)."""
    case(f"attention bf16 O B={B} H={H} Lq={Lq} Lk={Lk} ({kernel})")
    m = amd()
    q = orc.randn(61, B * Lq * H * HD).reshape(B, Lq, H * HD)
    k = orc.randn(62, B * Lk * H * HD).reshape(B, Lk, H * HD)
    v = orc.randn(63, B * Lk * H * HD).reshape(B, Lk, H * HD)
    kv_len = [max(1, Lk - 37 * b) for b in range(B)]
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    args = dict(B=B, Lq=Lq, Lk=Lk, H=H, D=HD, ldq=H * HD, ldk=H * HD, ldv=H * HD, kv_len=kv_len, precision=m.PREC_BF16)
    do = ctx.empty((B, Lq, H * HD))
    ctx.attention(q=dq, k=dk, v=dv, o=do, **args)
    ref = do.numpy()
    ldo = H * HD + 8
    fill = np.full((B, Lq, ldo), 0x7FC1, np.uint16)
    d16 = ctx.upload(fill)
    ctx.profile(True)
    ctx.profile_reset()
    ctx.attention(q=dq, k=dk, v=dv, o=d16, ldo=ldo, o_off=4, o_bf16=True, **args)
    names = {r["name"] for r in ctx.profile_report()}
    ctx.profile(False)
    assert kernel in names, names
    got = d16.numpy().reshape(B, Lq, ldo)
    want = (orc.bf16_round(ref).view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(got[:, :, 4:4 + H * HD], want)
    assert np.all(got[:, :, :4] == 0x7FC1) and np.all(got[:, :, 4 + H * HD:] == 0x7FC1)
    with pytest.raises(m.AnimaError):
        ctx.attention(q=dq, k=dk, v=dv, o=d16, ldo=ldo, o_bf16=True, **{**args, "precision": m.PREC_FP32})
    q96 = ctx.upload(orc.randn(64, Lq * 96).reshape(Lq, 96))
    with pytest.raises(m.AnimaError):
        ctx.attention(q=q96, k=q96, v=q96, o=d16, B=1, Lq=Lq, Lk=Lq, H=1, D=96, ldq=96, ldk=96, ldv=96, o_bf16=True,
                      precision=m.PREC_BF16)
