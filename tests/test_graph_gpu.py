"""Recorded submission (anima_graph_*): a captured sequence of library calls replayed from a HIP
graph gives the same bits as the same calls made eagerly, replay after replay, with the inputs
rewritten and eager work on the stream between replays; and the capture rules (no host copies,
no synchronization; buffers freed during the capture, and the scratch its calls were handed, stay
the graph's -- and only those: the context keeps its own workspace)."""

import numpy as np
import pytest

import oracle as orc
from helpers import amd
from test_linear_gpu import FIXED_LUT, int8_weight, w4_weight

pytestmark = pytest.mark.gpu

HD = 128


def case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    m = amd()
    c = m.Context(0)
    yield c
    c.close()


def test_graph_replays_match_eager(ctx):
    """Graph: d2d copy (residual reset) -> gated int8 GEMM into it (persistent 256 kernel) -> W4
    GEMM from fp32 x (rotation + int8 rows + W4 decode into a pool buffer inside the call) ->
    fused self-attention with q/k RMSNorm + RoPE (K/V prep in the workspace).  Three replays,
    each with new inputs and the same calls run eagerly into other buffers first."""
    case("graph replay vs eager: gated i8 GEMM 4096x4096x1024, W4 GEMM, fused attention L=2048 H=8")
    m = amd()
    M, N, K = 4096, 4096, 1024
    qw, sw = int8_weight(61, N, K)
    Wi = m.weight(m.W_I8, N, K, ctx.upload(qw), scale=ctx.upload(sw))
    codes, srel, sw4 = w4_weight(62, N, K)
    W4 = m.weight(m.W_W4, N, K, ctx.upload(codes), scale=ctx.upload(sw4), srel=ctx.upload(srel),
                  codebook=ctx.upload(FIXED_LUT))
    H, L, Hp, Wp = 8, 2048, 32, 64
    ld = 3 * H * HD
    qn = ctx.upload((1 + 0.02 * orc.randn(63, HD)).astype(np.float32))
    kn = ctx.upload((1 + 0.02 * orc.randn(64, HD)).astype(np.float32))
    cs = ctx.upload(orc.dit_rope_table(Hp, Wp))
    gate = ctx.upload(orc.randn(65, 3 * N))
    # inputs (rewritten before every replay)
    xq, xs, x = ctx.empty((M, K), np.int8), ctx.empty(M), ctx.empty((M, K))
    res0, qkv = ctx.empty((M, N)), ctx.empty((L, ld))

    def run(out_res, out_w4, out_o):
        ctx._check(amd().lib().anima_d2d(ctx.h, out_res.ptr, res0.ptr, M * N * 4))
        ctx.linear(Wi, M, out_res, xq=xq, xs=xs, epilogue=m.EPI_GATED, gate=gate, gate_off=N)
        ctx.linear(W4, M, out_w4, x=x, x_rotated=False)
        ctx.attention(q=qkv, k=qkv, v=qkv, o=out_o, B=1, Lq=L, Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld,
                      q_off=0, k_off=H * HD, v_off=2 * H * HD, q_norm=qn, k_norm=kn, rope_cs=cs, rope_sin_off=L * 64)

    def fill(seed):
        xin = orc.randn(seed, M * K).reshape(M, K)
        x.write(xin)
        ctx.quant_rows(x, M, K, 1, xq, xs)
        res0.write(orc.randn(seed + 1, M * N))
        qkv.write(orc.randn(seed + 2, L * ld))

    gres, gw4, go = ctx.empty((M, N)), ctx.empty((M, N)), ctx.empty((L, H * HD))
    eres, ew4, eo = ctx.empty((M, N)), ctx.empty((M, N)), ctx.empty((L, H * HD))
    fill(70)
    run(eres, ew4, eo)  # eager once: the pool and the workspace hold what the capture needs
    ctx.sync()
    ctx.graph_begin()
    run(gres, gw4, go)
    g = ctx.graph_end()
    for r in range(3):
        fill(80 + 10 * r)
        run(eres, ew4, eo)
        ctx.graph_launch(g)
        ctx.sync()
        for name, a, b in (("gated i8", gres, eres), ("w4", gw4, ew4), ("attention", go, eo)):
            ga, eb = a.numpy(), b.numpy()
            assert np.isfinite(eb).all() and np.abs(eb).max() > 0, (r, name)
            assert np.array_equal(ga, eb), (r, name)
    ctx.graph_destroy(g)
    for b in (xq, xs, x, res0, qkv, gres, gw4, go, eres, ew4, eo, qn, kn, cs, gate):
        b.release()


def test_graph_capture_rules():
    """While capturing: host copies and synchronization fail with ANIMA_E_STATE (and leave the
    capture usable); a buffer freed during the capture is not handed out again until the graph is
    destroyed; the attention's K / V scratch inside the capture is a pool buffer of the size it
    needs, so the graph does not take the context's larger workspace; foreign or destroyed handles
    are rejected.  A fresh context, so that its workspace starts empty."""
    case("graph capture rules")
    m = amd()
    with m.Context(0) as ctx:
        _capture_rules(m, ctx)


def _capture_rules(m, ctx):
    H, ld = 8, 3 * 8 * HD
    qkv = ctx.upload(orc.randn(90, 2048 * ld))
    o = ctx.empty((2048, H * HD))

    def attn(L):
        ctx.attention(q=qkv, k=qkv, v=qkv, o=o, B=1, Lq=L, Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld,
                      q_off=0, k_off=H * HD, v_off=2 * H * HD)

    attn(2048)  # the context's workspace grows to Lk = 2048 (8 MiB of bf16 K / V^T)
    attn(1024)
    ctx.sync()
    ref = o.numpy()[:1024]
    y = ctx.empty(4096)
    a0 = ctx.mem_stats()["allocated"]
    ctx.graph_begin()
    attn(1024)  # its K / V conversion gets a 4 MiB pool buffer of its own, not the 8 MiB workspace
    with pytest.raises(m.AnimaError) as e:
        y.write(np.ones(4096, np.float32))
    assert e.value.code == -4
    with pytest.raises(m.AnimaError) as e:
        ctx.sync()
    assert e.value.code == -4
    with pytest.raises(m.AnimaError):
        ctx.graph_begin()  # already capturing
    tmp = ctx.empty(3 << 18)  # 3 MiB: a pool bucket of its own
    ctx.zero(tmp, 1 << 18)
    reserved = tmp.ptr
    tmp.release()
    g = ctx.graph_end()
    a1 = ctx.mem_stats()["allocated"]
    assert a1 - a0 <= (4 << 20) + (3 << 20), (a0, a1)  # the graph holds what its capture asked for
    attn(2048)  # the context kept its own workspace: no reallocation
    assert ctx.mem_stats()["allocated"] == a1
    other = ctx.empty(3 << 18)
    assert other.ptr != reserved  # still the graph's
    o.write(np.zeros((2048, H * HD), np.float32))
    ctx.graph_launch(g)
    assert np.array_equal(o.numpy()[:1024], ref)
    ctx.graph_destroy(g)
    again = ctx.empty(3 << 18)
    assert again.ptr == reserved  # back in the pool
    with pytest.raises(m.AnimaError):
        ctx.graph_launch(g)
    with pytest.raises(m.AnimaError):
        ctx.graph_destroy(g)
    with pytest.raises(m.AnimaError):
        ctx.graph_end()  # no capture in progress
    for b in (qkv, o, y, other, again):
        b.release()
