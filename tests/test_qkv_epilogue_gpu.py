"""The stacked QKV projection with the attention's operand preparation in its epilogue
(anima_linear_qkv): Q columns as fp32, K rows RMS-normed + roped in bf16 and V^T in bf16, in the
layout of anima_attention_prepare_kv.

Bars: the K / V operand bytes equal those of anima_linear followed by
anima_attention_prepare_kv on its fp32 output, byte for byte (both form the row norm in the same
reduction tree), and the Q columns equal anima_linear's, bit for bit; the K rows are checked
against a float64 RMSNorm + RoPE of the linear's fp32 K columns (within bf16 rounding); the
attention on the fused operands equals the plain attention call bit for bit."""

import numpy as np
import pytest

import oracle as orc
from helpers import amd, report
from test_linear_gpu import FIXED_LUT, int8_weight, w4_weight

pytestmark = pytest.mark.gpu

HD = 128


@pytest.fixture(scope="module")
def ctx():
    c = amd().Context(0)
    yield c
    c.close()


def case(msg):
    print(f"[case] {msg}", flush=True)


def bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def make_weight(ctx, m, kind, seed, N, K, bias):
    bufs = []
    b = ctx.upload((0.05 * orc.randn(seed + 7, N)).astype(np.float32)) if bias else None
    if b is not None:
        bufs.append(b)
    if kind == "i8":
        qw, sw = int8_weight(seed, N, K)
        bufs += [ctx.upload(qw), ctx.upload(sw)]
        return m.weight(m.W_I8, N, K, bufs[-2], scale=bufs[-1], bias=b), bufs
    codes, srel, sw = w4_weight(seed, N, K)
    bufs += [ctx.upload(codes), ctx.upload(srel), ctx.upload(sw), ctx.upload(FIXED_LUT)]
    return m.weight(m.W_W4, N, K, bufs[-4], scale=bufs[-2], srel=bufs[-3], codebook=bufs[-1], bias=b), bufs


@pytest.mark.parametrize("kind,B,Hp,Wp,H,K,bias", [("i8", 2, 16, 16, 2, 512, False), ("w4", 3, 8, 24, 4, 1024, True),
                                                   ("w4_in_gemm", 3, 8, 24, 4, 1024, True),
                                                   ("i8", 2, 64, 64, 16, 2048, True), ("w4", 2, 64, 64, 16, 2048, False),
                                                   ("w4_in_gemm", 2, 64, 64, 16, 2048, False)])
def test_linear_qkv_operands_bit_exact(ctx, kind, B, Hp, Wp, H, K, bias):
    """W4 runs both ways: unpacked per call into the int8 scratch grid ("w4", the default) and
    inside the GEMM main loop ("w4_in_gemm")."""
    L = Hp * Wp
    M, N = B * L, 3 * H * HD
    case(f"linear_qkv {kind} B={B} L={L} H={H} K={K} bias={bias}")
    m = amd()
    ctx.set_w4_path(m.W4_IN_GEMM if kind == "w4_in_gemm" else m.W4_GRID_SCRATCH)
    try:
        run_linear_qkv_case(ctx, m, kind.split("_")[0], B, Hp, Wp, H, K, bias)
    finally:
        ctx.set_w4_path(m.W4_GRID_SCRATCH)


def run_linear_qkv_case(ctx, m, kind, B, Hp, Wp, H, K, bias):
    L = Hp * Wp
    M, N = B * L, 3 * H * HD
    W, wbufs = make_weight(ctx, m, kind, 300 + K + H, N, K, bias)
    rng = np.random.default_rng(400 + L)
    xq = ctx.upload(rng.integers(-127, 128, size=(M, K), dtype=np.int8))
    xs = ctx.upload(rng.uniform(0.002, 0.02, M).astype(np.float32))
    kn = (1 + 0.02 * orc.randn(401, HD)).astype(np.float32)
    qn = (1 + 0.02 * orc.randn(402, HD)).astype(np.float32)
    cs_np = orc.dit_rope_table(Hp, Wp)
    dkn, dqn, dcs = ctx.upload(kn), ctx.upload(qn), ctx.upload(cs_np)
    sin_off = L * 64
    nbytes = m.Context.attention_kv_bytes(B, H, L, m.PREC_BF16)
    # reference: the plain linear, then the K / V conversion of its fp32 output
    ref = ctx.empty((M, N))
    ctx.linear(W, M, ref, xq=xq, xs=xs)
    prep_ref = ctx.empty(nbytes, np.uint8)
    common = dict(B=B, Lq=L, Lk=L, H=H, D=HD, ldq=N, ldk=N, ldv=N, k_off=H * HD, v_off=2 * H * HD, precision=m.PREC_BF16)
    ctx.attention(q=ref, k=ref, v=ref, o=ref, prepare_into=prep_ref, k_norm=dkn, rope_cs=dcs, rope_sin_off=sin_off,
                  **common)
    # fused: Q into a [M, H*128] buffer, K / V straight into the operand layout
    q = ctx.empty((M, H * HD))
    prep = ctx.empty(nbytes, np.uint8)
    ctx.linear_qkv(W, M, q, B=B, L=L, H=H, k_norm=dkn, rope_cs=dcs, rope_sin_off=sin_off, kv_prep=prep, xq=xq, xs=xs,
                   ldc=H * HD)
    r = ref.numpy()
    got_prep, want_prep = prep.numpy(), prep_ref.numpy()
    kbytes = nbytes // 2
    print(f"K bytes differing: {int((got_prep[:kbytes] != want_prep[:kbytes]).sum())}, "
          f"V^T bytes differing: {int((got_prep[kbytes:] != want_prep[kbytes:]).sum())}", flush=True)
    assert np.array_equal(q.numpy(), r[:, :H * HD])
    assert np.array_equal(got_prep, want_prep)
    # K rows against float64 RMSNorm + RoPE of the fp32 K columns (the bf16 rounding bound)
    kplane = bf16_to_f32(got_prep[:kbytes].view(np.uint16)).reshape(B, H, L, HD)
    rows = np.unique(np.concatenate([np.arange(0, 8), rng.choice(L, 24, replace=False), np.arange(L - 8, L)]))
    cos = cs_np[:L * 64].reshape(L, 64).astype(np.float64)
    sin = cs_np[sin_off:sin_off + L * 64].reshape(L, 64).astype(np.float64)
    for b in (0, B - 1):
        k = r[b * L + rows, H * HD:2 * H * HD].astype(np.float64).reshape(len(rows), H, HD)
        kn64 = k / np.sqrt((k * k).mean(-1, keepdims=True) + 1e-6) * kn.astype(np.float64)
        lo, hi = kn64[..., :64], kn64[..., 64:]
        c, s = cos[rows][:, None, :], sin[rows][:, None, :]
        want = np.concatenate([lo * c - hi * s, hi * c + lo * s], -1)
        got = kplane[b][:, rows].transpose(1, 0, 2)
        err = np.abs(got - want) / np.maximum(np.abs(want), 1e-3)
        assert err.max() <= 2.0 ** -8 + 1e-5, err.max()
    # attention on the fused operands = the plain call
    if L <= 1024:
        o1, o2 = ctx.empty((M, H * HD)), ctx.empty((M, H * HD))
        ctx.attention(q=ref, k=ref, v=ref, o=o1, q_norm=dqn, k_norm=dkn, rope_cs=dcs, rope_sin_off=sin_off, **common)
        ctx.attention(q=q, k=None, v=None, o=o2, kv_prep=prep, q_norm=dqn, rope_cs=dcs, rope_sin_off=sin_off,
                      **dict(common, ldq=H * HD))
        assert np.array_equal(o1.numpy(), o2.numpy())
        o1.release()
        o2.release()
    for x in wbufs + [xq, xs, dkn, dqn, dcs, ref, prep_ref, q, prep]:
        x.release()


@pytest.mark.parametrize("kind,cols", [("i8", 2048), ("w4", 2048), ("i8", 0)])
def test_linear_qkv_lora(ctx, kind, cols):
    """The fused QKV epilogue with the LoRA term (anima_linear_desc lora_*): Q and the K / V operands
    bit-identical to the LoRA linear's fp32 output converted by anima_attention_prepare_kv.
    B = 2, 48 x 48 tokens (M = 4608: the plain linear also runs the product inside its epilogue,
    as it does from one 256 x 256 tile per CU up), H = 16, K = 2048; rank 32 per q / k / v block
    (lora_cols = 2048), or one rank-48 block over all columns (lora_cols = 0)."""
    case(f"linear_qkv LoRA {kind} cols={cols}")
    m = amd()
    B, Hp, Wp, H, K = 2, 48, 48, 16, 2048
    L = Hp * Wp
    M, N = B * L, 3 * H * HD
    R = 32 if cols else 48
    nb = N // cols if cols else 1
    W, wbufs = make_weight(ctx, m, kind, 777, N, K, True)
    rng = np.random.default_rng(778)
    xq = ctx.upload(rng.integers(-127, 128, size=(M, K), dtype=np.int8))
    xs = ctx.upload(rng.uniform(0.002, 0.02, M).astype(np.float32))
    xa = ctx.upload((0.5 * rng.standard_normal((M, nb * R))).astype(np.float32))
    Bm = ctx.upload((0.05 * rng.standard_normal((N, R))).astype(np.float32))
    planes = ctx.empty(3 * N * R, np.uint16)
    ctx.split3_bf16(Bm, planes, N * R)
    lk = dict(lora_xa=xa, ld_lora_xa=nb * R, lora_b=planes, lora_r=R, lora_cols=cols)
    kn = ctx.upload((1 + 0.02 * orc.randn(779, HD)).astype(np.float32))
    cs = ctx.upload(orc.dit_rope_table(Hp, Wp))
    sin_off = L * 64
    nbytes = m.Context.attention_kv_bytes(B, H, L, m.PREC_BF16)
    ref = ctx.empty((M, N))
    ctx.linear(W, M, ref, xq=xq, xs=xs, **lk)
    prep_ref = ctx.empty(nbytes, np.uint8)
    ctx.attention(q=ref, k=ref, v=ref, o=ref, prepare_into=prep_ref, k_norm=kn, rope_cs=cs, rope_sin_off=sin_off,
                  B=B, Lq=L, Lk=L, H=H, D=HD, ldq=N, ldk=N, ldv=N, k_off=H * HD, v_off=2 * H * HD,
                  precision=m.PREC_BF16)
    q = ctx.empty((M, H * HD))
    prep = ctx.empty(nbytes, np.uint8)
    ctx.linear_qkv(W, M, q, B=B, L=L, H=H, k_norm=kn, rope_cs=cs, rope_sin_off=sin_off, kv_prep=prep, xq=xq, xs=xs,
                   ldc=H * HD, **lk)
    got_prep, want_prep = prep.numpy(), prep_ref.numpy()
    print(f"differing prep bytes: {int((got_prep != want_prep).sum())}", flush=True)
    assert np.array_equal(q.numpy(), ref.numpy()[:, :H * HD])
    assert np.array_equal(got_prep, want_prep)
    for x in wbufs + [xq, xs, xa, Bm, planes, kn, cs, ref, prep_ref, q, prep]:
        x.release()


@pytest.mark.parametrize("kind,Hp,Wp", [("i8", 32, 32), ("w4", 33, 64), ("i8", 33, 64)])
def test_linear_qkv_prepared_q(ctx, kind, Hp, Wp):
    """Q prepared by the QKV epilogue (anima_qkv_desc q_prep: RMSNorm, RoPE, the attention's
    scale * log2(e), bf16): the attention on it equals the attention on the plain fp32 Q with
    q_norm + RoPE bit for bit (32 x 32 tokens: the 4-wave kernel; 33 x 64: the 8-wave kernel with
    a partial last query tile), and each prepared value is within bf16 rounding of float64."""
    case(f"linear_qkv prepared Q {kind} {Hp}x{Wp}")
    m = amd()
    B, H, K = 2, 16, 2048
    L = Hp * Wp
    M, N = B * L, 3 * H * HD
    W, wbufs = make_weight(ctx, m, kind, 880 + Hp, N, K, True)
    rng = np.random.default_rng(881)
    xq = ctx.upload(rng.integers(-127, 128, size=(M, K), dtype=np.int8))
    xs = ctx.upload(rng.uniform(0.002, 0.02, M).astype(np.float32))
    qn = (1 + 0.02 * orc.randn(882, HD)).astype(np.float32)
    kn = (1 + 0.02 * orc.randn(883, HD)).astype(np.float32)
    cs_np = orc.dit_rope_table(Hp, Wp)
    dqn, dkn, dcs = ctx.upload(qn), ctx.upload(kn), ctx.upload(cs_np)
    sin_off = L * 64
    nbytes = m.Context.attention_kv_bytes(B, H, L, m.PREC_BF16)
    ref = ctx.empty((M, N))
    ctx.linear(W, M, ref, xq=xq, xs=xs)
    prep_ref = ctx.empty(nbytes, np.uint8)
    common = dict(B=B, Lq=L, Lk=L, H=H, D=HD, ldq=N, ldk=N, ldv=N, precision=m.PREC_BF16, rope_cs=dcs,
                  rope_sin_off=sin_off)
    ctx.attention(q=ref, k=ref, v=ref, o=ref, prepare_into=prep_ref, k_norm=dkn, k_off=H * HD, v_off=2 * H * HD,
                  **common)
    qp = ctx.empty(M * H * HD, np.uint16)
    prep = ctx.empty(nbytes, np.uint8)
    ctx.linear_qkv(W, M, None, B=B, L=L, H=H, k_norm=dkn, rope_cs=dcs, rope_sin_off=sin_off, kv_prep=prep, xq=xq,
                   xs=xs, q_norm=dqn, q_prep=qp)
    assert np.array_equal(prep.numpy(), prep_ref.numpy())
    o1, o2 = ctx.empty((M, H * HD)), ctx.empty((M, H * HD))
    ctx.attention(q=ref, k=None, v=None, o=o1, kv_prep=prep_ref, q_norm=dqn, **common)
    ctx.attention(q=None, k=None, v=None, o=o2, kv_prep=prep, q_prep=qp, **common)
    a1, a2 = o1.numpy(), o2.numpy()
    print(f"attention outputs differing: {int((a1 != a2).sum())} of {a1.size}", flush=True)
    assert np.array_equal(a1, a2)
    # prepared values against float64 (RMSNorm, RoPE, scale * log2 e), sampled rows
    r = ref.numpy()
    rows = np.unique(np.concatenate([np.arange(0, 4), rng.choice(M, 16, replace=False), np.arange(M - 4, M)]))
    q64 = r[rows, :H * HD].astype(np.float64).reshape(len(rows), H, HD)
    q64 = q64 / np.sqrt((q64 * q64).mean(-1, keepdims=True) + 1e-6) * qn.astype(np.float64)
    li = rows % L
    c = cs_np[:L * 64].reshape(L, 64).astype(np.float64)[li][:, None, :]
    sn = cs_np[sin_off:sin_off + L * 64].reshape(L, 64).astype(np.float64)[li][:, None, :]
    lo, hi = q64[..., :64], q64[..., 64:]
    want = np.concatenate([lo * c - hi * sn, hi * c + lo * sn], -1) * (np.log2(np.e) / np.sqrt(HD))
    got = bf16_to_f32(qp.numpy().reshape(M, H, HD)[rows])
    err = np.abs(got - want) / np.maximum(np.abs(want), 1e-3)
    assert err.max() <= 2.0 ** -8 + 1e-5, err.max()
    for x in wbufs + [xq, xs, dqn, dkn, dcs, ref, prep_ref, qp, prep, o1, o2]:
        x.release()


@pytest.mark.parametrize("lora", [False, True])
def test_linear_q_only_prepared(ctx, lora):
    """A Q-only projection (W of H * 128 columns, anima_qkv_desc q_prep without K / V or RoPE: the
    cross-attention's q) feeding the attention against prepared K / V of 512 context keys (ragged
    kv_len): bit-identical to the plain linear + attention with q_norm; with a rank-32 LoRA term
    (lora_*, one block) on both sides as well."""
    case(f"linear_qkv Q-only prepared Q (cross-attention){' + LoRA' if lora else ''}")
    m = amd()
    B, L, H, K, Lk = 2, 4096, 16, 2048, 512
    M, N = B * L, H * HD
    W, wbufs = make_weight(ctx, m, "i8", 890, N, K, True)
    rng = np.random.default_rng(891)
    xq = ctx.upload(rng.integers(-127, 128, size=(M, K), dtype=np.int8))
    xs = ctx.upload(rng.uniform(0.002, 0.02, M).astype(np.float32))
    lk = {}
    if lora:
        R = 32
        xa = ctx.upload((0.5 * rng.standard_normal((M, R))).astype(np.float32))
        Bm = ctx.upload((0.05 * rng.standard_normal((N, R))).astype(np.float32))
        planes = ctx.empty(3 * N * R, np.uint16)
        ctx.split3_bf16(Bm, planes, N * R)
        lk = dict(lora_xa=xa, ld_lora_xa=R, lora_b=planes, lora_r=R)
        wbufs += [xa, Bm, planes]
    dqn = ctx.upload((1 + 0.02 * orc.randn(892, HD)).astype(np.float32))
    kv = ctx.upload(orc.randn(893, B * Lk * N).reshape(B * Lk, N))
    kv_len = [458, 263]
    nbytes = m.Context.attention_kv_bytes(B, H, Lk, m.PREC_BF16)
    prep = ctx.empty(nbytes, np.uint8)
    common = dict(B=B, Lq=L, Lk=Lk, H=H, D=HD, ldq=N, ldk=N, ldv=N, precision=m.PREC_BF16, kv_len=kv_len)
    ctx.attention(q=kv, k=kv, v=kv, o=kv, prepare_into=prep, **dict(common, Lq=Lk))
    q = ctx.empty((M, N))
    ctx.linear(W, M, q, xq=xq, xs=xs, **lk)
    qp = ctx.empty(M * N, np.uint16)
    ctx.linear_qkv(W, M, None, B=B, L=L, H=H, xq=xq, xs=xs, q_norm=dqn, q_prep=qp, **lk)
    o1, o2 = ctx.empty((M, N)), ctx.empty((M, N))
    ctx.attention(q=q, k=None, v=None, o=o1, kv_prep=prep, q_norm=dqn, **common)
    ctx.attention(q=None, k=None, v=None, o=o2, kv_prep=prep, q_prep=qp, **common)
    a1, a2 = o1.numpy(), o2.numpy()
    print(f"attention outputs differing: {int((a1 != a2).sum())} of {a1.size}", flush=True)
    assert np.array_equal(a1, a2)
    for x in wbufs + [xq, xs, dqn, kv, prep, q, qp, o1, o2]:
        x.release()


def test_linear_qkv_refusals(ctx):
    """Shapes the fused epilogue does not cover are refused on the host before any launch:
    L % 64 != 0 (ANIMA_E_UNSUPPORTED), a wrong operand buffer size, N != 3 * 128 * H and LoRA
    rank blocks that split a 256-column tile (ANIMA_E_ARG)."""
    case("linear_qkv host refusals")
    m = amd()
    H, K = 2, 256
    N = 3 * H * HD
    qw, sw = int8_weight(501, N, K)
    dq, ds = ctx.upload(qw), ctx.upload(sw)
    W = m.weight(m.W_I8, N, K, dq, scale=ds)
    kn, cs = ctx.upload(np.ones(HD, np.float32)), ctx.upload(orc.dit_rope_table(8, 12))
    for L, Hh, exp in ((96, H, -5), (128, 3, -1)):
        M = 2 * L
        xq, xs, out = ctx.empty((M, K), np.int8), ctx.empty(M), ctx.empty((M, N))
        prep = ctx.empty(m.Context.attention_kv_bytes(2, Hh, L, m.PREC_BF16), np.uint8)
        with pytest.raises(m.AnimaError) as e:
            ctx.linear_qkv(W, M, out, B=2, L=L, H=Hh, k_norm=kn, rope_cs=cs, rope_sin_off=96 * 64, kv_prep=prep,
                           xq=xq, xs=xs)
        assert e.value.code == exp, (L, Hh, e.value)
        for x in (xq, xs, out, prep):
            x.release()
    # LoRA rank blocks that split a 256-column tile (lora_cols = 384): ANIMA_E_ARG
    L, M = 128, 256
    xq, xs, out = ctx.empty((M, K), np.int8), ctx.empty(M), ctx.empty((M, N))
    prep = ctx.empty(m.Context.attention_kv_bytes(2, H, L, m.PREC_BF16), np.uint8)
    xa, planes = ctx.empty((M, 64)), ctx.empty(3 * N * 32, np.uint16)
    with pytest.raises(m.AnimaError) as e:
        ctx.linear_qkv(W, M, out, B=2, L=L, H=H, k_norm=kn, rope_cs=cs, rope_sin_off=96 * 64, kv_prep=prep, xq=xq,
                       xs=xs, lora_xa=xa, ld_lora_xa=64, lora_b=planes, lora_r=32, lora_cols=384)
    assert e.value.code == -1, e.value
    for x in (xq, xs, out, prep, xa, planes, dq, ds, kn, cs):
        x.release()
