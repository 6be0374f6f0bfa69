"""GPU parity of the quantized-linear side of the attention sublayer through the C ABI:
ConvRot Hadamard, per-token int8 quantization, LayerNorm+adaLN(+Hadamard)(+int8), elementwise
ops, and the int8 / W4A8 MFMA GEMMs with the reference's epilogues.

Bars: Hadamard, quantization and LayerNorm are bit-exact against the oracle; GEMM int32
accumulators are bit-exact (sampled rows against the oracle, every row and column through exact
int64 checksums); the fp32 epilogue (acc * s_x * s_w, bias, gate) is bit-exact; GELU/SiLU
outputs within 1e-6 relative (device expf).  W8A8 against the reference's W8A32 semantics
(fp32 activations) is reported and bounded by 3e-2 rel L2 (activation quantization noise).
"""

import numpy as np
import pytest

import oracle as orc
from helpers import amd, rel_l2, report

pytestmark = pytest.mark.gpu

FIXED_LUT = np.array([-0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
                      0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671], np.float32)


@pytest.fixture(scope="module")
def ctx():
    c = amd().Context(0)
    yield c
    c.close()


def case(msg):
    print(f"[case] {msg}", flush=True)


def int8_weight(seed, N, K):
    """clip(round(40 N(0,1)), +-127) int8 weights, s_w = U(0.5, 1.5) / (127 sqrt(K))."""
    w = np.clip(np.rint(40 * orc.randn(seed, N * K)), -127, 127).astype(np.int8).reshape(N, K)
    rng = np.random.default_rng(seed)
    s = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
    return w, s


def w4_weight(seed, N, K):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    srel = rng.integers(0x60, 0x70, size=(N, K // 16), dtype=np.uint8)  # e4m3 values 32..120
    s = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
    return codes, srel, s


# ------------------------------------------------------------------ row kernels

def test_hadamard_and_quant_bit_exact(ctx):
    case("hadamard / quant_rows M=512 K=2048 and K=8192")
    x = orc.randn(41, 512 * 2048).reshape(512, 2048) * 3
    dx, dy = ctx.upload(x), ctx.empty(x.shape)
    ctx.hadamard(dx, dy, x.size)
    xr = orc.hadamard256(x)
    assert np.array_equal(dy.numpy(), xr)
    for rotate, src in ((1, x), (0, xr)):
        dq, ds = ctx.empty((512, 2048), np.int8), ctx.empty(512)
        ctx.quant_rows(ctx.upload(src), 512, 2048, rotate, dq, ds)
        q, s = orc.token_quant(xr)
        assert np.array_equal(ds.numpy(), s) and np.array_equal(dq.numpy(), q)
    x8 = orc.randn(42, 64 * 8192).reshape(64, 8192)
    x8[3] = 0.0  # all-zero row: s = 0, q = 0
    dq, ds = ctx.empty((64, 8192), np.int8), ctx.empty(64)
    ctx.quant_rows(ctx.upload(x8), 64, 8192, 1, dq, ds)
    q, s = orc.token_quant(orc.hadamard256(x8))
    assert np.array_equal(ds.numpy(), s) and np.array_equal(dq.numpy(), q)
    assert s[3] == 0 and not q[3].any()


@pytest.mark.parametrize("cols,rotate,shift", [(2048, True, 0), (2048, False, 0), (1024, True, 0), (8192, True, 0),
                                               (2048, True, 2)])
def test_layernorm_mod_bit_exact(ctx, cols, rotate, shift):
    """shift = 0: the wave-per-row kernel; shift = 2 (modulation vectors not 16-byte aligned): the
    workgroup-per-row kernel."""
    case(f"layernorm_mod rows=300 cols={cols} rotate={rotate} shift_off={shift}")
    rows = 300
    x = (orc.randn(43, rows * cols).reshape(rows, cols) * 2 + 0.5).astype(np.float32)
    mod = (0.1 * orc.randn(44, 3 * cols)).astype(np.float32)
    dx, dm, dy = ctx.upload(x), ctx.upload(mod), ctx.empty(x.shape)
    dq = ctx.empty((rows, cols), np.int8) if rotate else None
    ds = ctx.empty(rows) if rotate else None
    ctx.layernorm_mod(dx, dm, shift, cols, rows, cols, rotate=rotate, y=dy, q=dq, s=ds)
    ref = orc.layernorm_mod(x, mod, shift, cols, cols, rotate=rotate)
    got = dy.numpy()
    assert np.array_equal(got, ref), report("layernorm_mod", got, ref)
    if rotate:
        q, s = orc.token_quant(ref)
        assert np.array_equal(ds.numpy(), s) and np.array_equal(dq.numpy(), q)


@pytest.mark.parametrize("K,act,rotate", [(8192, "gelu", True), (2048, "silu", True), (768, "gelu", True),
                                          (3072, "gelu", False)])
def test_quant_rows_act(ctx, K, act, rotate):
    """anima_quant_rows_act: the activation of a linear applied in the Hadamard + int8 pass.  Its
    int8 rows and scales are bit-identical to anima_quant_rows on the output of an int8 linear
    with the same activation in its epilogue (same pre-activation values, same activation code);
    register-resident (K % 1024 == 0) and LDS kernels, with and without the rotation."""
    case(f"quant_rows_act K={K} act={act} rotate={rotate}")
    m = amd()
    M, Kin = 300, 1024
    x = orc.randn(61, M * Kin).reshape(M, Kin)
    qx, sx = orc.token_quant(orc.hadamard256(x))
    qw, sw = int8_weight(62, K, Kin)
    W = m.weight(m.W_I8, K, Kin, ctx.upload(qw), scale=ctx.upload(sw))
    dqx, dsx = ctx.upload(qx), ctx.upload(sx)
    pre, post = ctx.empty((M, K)), ctx.empty((M, K))
    ctx.linear(W, M, pre, xq=dqx, xs=dsx, alpha=3.0)
    ctx.linear(W, M, post, xq=dqx, xs=dsx, alpha=3.0, act=act)
    q1, s1 = ctx.empty((M, K), np.int8), ctx.empty(M)
    q2, s2 = ctx.empty((M, K), np.int8), ctx.empty(M)
    ctx.quant_rows(pre, M, K, rotate, q1, s1, act=act)
    ctx.quant_rows(post, M, K, rotate, q2, s2)
    assert np.array_equal(s1.numpy(), s2.numpy()) and np.array_equal(q1.numpy(), q2.numpy())
    # against the oracle's activation (correctly rounded formula): the int8 codes may differ by one
    # where the 1-ulp device activation crosses a rounding boundary
    p64 = pre.numpy().astype(np.float64)
    a = np.vectorize(orc.gelu if act == "gelu" else orc.silu)(p64).astype(np.float32)
    q, s = orc.token_quant(orc.hadamard256(a) if rotate else a)
    assert np.allclose(s1.numpy(), s, rtol=1e-6, atol=0)
    d = np.abs(q1.numpy().astype(np.int32) - q.astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_elementwise_and_zero(ctx):
    case("elementwise silu_mul/add/silu/copy, zero")
    n = 10007
    a = orc.randn(45, n) * 4
    b = orc.randn(46, n)
    da, db, dy = ctx.upload(a), ctx.upload(b), ctx.empty(n)
    silu = a.astype(np.float64) / (1 + np.exp(-a.astype(np.float64)))
    for op, ref in (("silu_mul", silu * b), ("add", a.astype(np.float64) + b), ("silu", silu), ("copy", a)):
        ctx.elementwise(op, da, db, dy, n)
        got = dy.numpy()
        assert np.allclose(got, ref, rtol=1e-6, atol=1e-6), op
    ctx.zero(dy, n)
    assert not dy.numpy().any()


@pytest.mark.parametrize("B,h,w", [(2, 128, 128), (1, 6, 10)])
def test_patchify_unpatchify(ctx, B, h, w):
    """Device patch layout against numpy reshapes of the reference's rearrange patterns
    "c (h m) (w n) -> (h w) (c m n)" (+ zero mask channel) and "(h w) (p1 p2 c) -> c (h p1) (w p2)"
    (dit.js:55-78); pure data movement, so bit-exact."""
    case(f"patchify / unpatchify B={B} h={h} w={w}")
    Hp, Wp = h // 2, w // 2
    lat = orc.randn(47, B * 16 * h * w).reshape(B, 16, h, w)
    want = lat.reshape(B, 16, Hp, 2, Wp, 2).transpose(0, 2, 4, 1, 3, 5).reshape(B * Hp * Wp, 64)
    want = np.concatenate([want, np.zeros((B * Hp * Wp, 4), np.float32)], axis=1)
    dl, dp = ctx.upload(lat), ctx.empty((B * Hp * Wp, 68))
    ctx.patchify(dl, B, h, w, dp)
    assert np.array_equal(dp.numpy(), want)
    o = orc.randn(48, B * Hp * Wp * 64).reshape(B * Hp * Wp, 64)
    want_v = o.reshape(B, Hp, Wp, 2, 2, 16).transpose(0, 5, 1, 3, 2, 4).reshape(B, 16, h, w)
    do, dv = ctx.upload(o), ctx.empty((B, 16, h, w))
    ctx.unpatchify(do, B, h, w, dv)
    assert np.array_equal(dv.numpy(), want_v)
    # round trip: the input columns are (c m n), the output columns (p1 p2 c)
    cmn = dp.numpy()[:, :64].reshape(-1, 16, 2, 2)
    dq = ctx.upload(np.ascontiguousarray(cmn.transpose(0, 2, 3, 1).reshape(-1, 64)))
    ctx.unpatchify(dq, B, h, w, dv)
    assert np.array_equal(dv.numpy(), lat)
    with pytest.raises(amd().AnimaError):
        ctx.patchify(dl, B, h - 1, w, dp)


# ------------------------------------------------------------------ int8 / W4A8 GEMM

def checksums_ok(qx, qw_int8, acc):
    """Exact int64 row and column sums of acc = qx @ qw^T."""
    qx64, qw64 = qx.astype(np.int64), qw_int8.astype(np.int64)
    acc64 = acc.astype(np.int64)
    rows = qx64 @ qw64.sum(0)
    cols = qw64 @ qx64.sum(0)
    return np.array_equal(acc64.sum(1), rows) and np.array_equal(acc64.sum(0), cols)


@pytest.mark.parametrize("kind", ["i8", "w4"])
def test_qkv_projection_full_size(ctx, kind):
    """x [2,4096,2048] -> ConvRot + per-token int8 -> QKV 2048 -> 6144 (one stacked GEMM)."""
    case(f"QKV projection M=8192 N=6144 K=2048 {kind}")
    m = amd()
    M, K, N = 8192, 2048, 6144
    x = orc.randn(51, M * K).reshape(M, K)
    dx = ctx.upload(x)
    dq, ds = ctx.empty((M, K), np.int8), ctx.empty(M)
    ctx.quant_rows(dx, M, K, 1, dq, ds)
    xr = orc.hadamard256(x)
    qx, sx = orc.token_quant(xr)
    assert np.array_equal(dq.numpy(), qx) and np.array_equal(ds.numpy(), sx)
    if kind == "i8":
        qw, sw = int8_weight(52, N, K)
        dw, dsw = ctx.upload(qw), ctx.upload(sw)
        W = m.weight(m.W_I8, N, K, dw, scale=dsw)
        qw_grid = qw
    else:
        codes, srel, sw = w4_weight(53, N, K)
        dw, dsw, dsr, dcb = ctx.upload(codes), ctx.upload(sw), ctx.upload(srel), ctx.upload(FIXED_LUT)
        W = m.weight(m.W_W4, N, K, dw, scale=dsw, srel=dsr, codebook=dcb)
        qw_grid = orc.w4_decode(codes, srel, FIXED_LUT, N, K)
    dout, dacc = ctx.empty((M, N)), ctx.empty((M, N), np.int32)
    ctx.linear(W, M, dout, xq=dq, xs=ds, acc_out=dacc)
    acc = dacc.numpy()
    out = dout.numpy()
    assert checksums_ok(qx, qw_grid, acc), "int32 accumulator checksums"
    rows = np.unique(np.concatenate([np.arange(0, 8), np.random.default_rng(0).choice(M, 24, replace=False), [M - 1]]))
    ref_acc = orc.gemm_i8(qx[rows], qw_grid)
    assert np.array_equal(acc[rows], ref_acc)
    assert np.array_equal(out[rows], orc.linear_epilogue(ref_acc, sx[rows], sw))
    # the reference's semantics: fp32 rotated activations x int grid weights, scale in the epilogue
    w8a32 = (xr[rows].astype(np.float64) @ qw_grid.astype(np.float64).T) * sw
    r, _ = report(f"{kind} W8A8 vs W8A32 (reference semantics)", out[rows], w8a32)
    assert r < 3e-2
    # the same GEMM from the fp32 input (rotation + quantization inside anima_linear)
    dout2 = ctx.empty((M, N))
    ctx.linear(W, M, dout2, x=dx, x_rotated=False)
    assert np.array_equal(dout2.numpy(), out)
    for b in (dx, dq, ds, dout, dacc, dout2, dw, dsw):
        b.release()


@pytest.mark.parametrize("kind", ["i8", "w4"])
def test_out_projection_gated_epilogue(ctx, kind):
    """Out projection 2048 -> 2048 with the gated residual into x (dit.js:289, gemm.js:192)."""
    case(f"out projection gated residual M=1000 {kind}")
    m = amd()
    M, K, N = 1000, 2048, 2048
    a = orc.randn(61, M * K).reshape(M, K)
    resid = orc.randn(62, M * N).reshape(M, N)
    mod = orc.randn(63, 3 * N).astype(np.float32)
    qx, sx = orc.token_quant(orc.hadamard256(a))
    if kind == "i8":
        qw, sw = int8_weight(64, N, K)
        dw = ctx.upload(qw)
        W = m.weight(m.W_I8, N, K, dw, scale=ctx.upload(sw), bias=ctx.upload(0.1 * orc.randn(65, N)))
        grid = qw
    else:
        codes, srel, sw = w4_weight(66, N, K)
        W = m.weight(m.W_W4, N, K, ctx.upload(codes), scale=ctx.upload(sw), srel=ctx.upload(srel),
                     codebook=ctx.upload(FIXED_LUT), bias=ctx.upload(0.1 * orc.randn(65, N)))
        grid = orc.w4_decode(codes, srel, FIXED_LUT, N, K)
    bias = (0.1 * orc.randn(65, N)).astype(np.float32)
    dout = ctx.upload(resid)
    ctx.linear(W, M, dout, x=ctx.upload(a), x_rotated=False, epilogue=m.EPI_GATED, gate=ctx.upload(mod),
               gate_off=2 * N)
    ref = orc.linear_epilogue(orc.gemm_i8(qx, grid), sx, sw, bias=bias, epi=2, gate=mod, g_off=2 * N, c=resid)
    got = dout.numpy()
    assert np.array_equal(got, ref), report("gated", got, ref)
    # plain residual
    dout = ctx.upload(resid)
    ctx.linear(W, M, dout, xq=ctx.upload(qx), xs=ctx.upload(sx), epilogue=m.EPI_RESID)
    assert np.array_equal(dout.numpy(), orc.linear_epilogue(orc.gemm_i8(qx, grid), sx, sw, bias=bias, epi=1, c=resid))


@pytest.fixture
def w4_path(ctx):
    """Sets the context's W4 path for one test (default afterwards)."""
    def set_path(name):
        m = amd()
        ctx.set_w4_path(m.W4_IN_GEMM if name == "in_gemm" else m.W4_GRID_SCRATCH)
    yield set_path
    ctx.set_w4_path(amd().W4_GRID_SCRATCH)


@pytest.mark.parametrize("kind,path", [("i8", "-"), ("w4", "scratch"), ("w4", "in_gemm")])
def test_256_tile_kernel_ragged_edges(ctx, w4_path, kind, path):
    """M=4500, N=4100: 18 x 17 tiles of 256 (the 256x256 persistent kernel), partial last row
    and column tiles (rows / columns past the edge read as zero through the buffer bounds; W4
    rows past N decode to zero), and a last group of 2 row tiles in the kernel's tile order
    (groups of 4); gated residual + bias epilogue and the int32 accumulators bit-exact on
    sampled rows, including the last ones, and the accumulator checksums over the whole
    product.  W4 both ways: unpacked into the scratch grid and inside the GEMM."""
    case(f"256x256-tile kernel M=4500 N=4100 K=1024 gated + bias {kind} {path}")
    w4_path(path)
    m = amd()
    M, K, N = 4500, 1024, 4100
    x = orc.randn(91, M * K).reshape(M, K)
    qx, sx = orc.token_quant(orc.hadamard256(x))
    bias = (0.1 * orc.randn(93, N)).astype(np.float32)
    mod = orc.randn(94, 3 * N).astype(np.float32)
    resid = orc.randn(95, M * N).reshape(M, N)
    if kind == "i8":
        qw, sw = int8_weight(92, N, K)
        W = m.weight(m.W_I8, N, K, ctx.upload(qw), scale=ctx.upload(sw), bias=ctx.upload(bias))
    else:
        codes, srel, sw = w4_weight(96, N, K)
        W = m.weight(m.W_W4, N, K, ctx.upload(codes), scale=ctx.upload(sw), srel=ctx.upload(srel),
                     codebook=ctx.upload(FIXED_LUT), bias=ctx.upload(bias))
        qw = orc.w4_decode(codes, srel, FIXED_LUT, N, K)
    dout, dacc = ctx.upload(resid), ctx.empty((M, N), np.int32)
    ctx.linear(W, M, dout, xq=ctx.upload(qx), xs=ctx.upload(sx), epilogue=m.EPI_GATED, gate=ctx.upload(mod),
               gate_off=N, acc_out=dacc)
    acc, got = dacc.numpy(), dout.numpy()
    assert checksums_ok(qx, qw, acc), "int32 accumulator checksums"
    rows = np.unique(np.concatenate([np.arange(0, 4), np.random.default_rng(1).choice(M, 16, replace=False),
                                     np.arange(M - 20, M)]))
    ref_acc = orc.gemm_i8(qx[rows], qw)
    assert np.array_equal(acc[rows], ref_acc)
    ref = orc.linear_epilogue(ref_acc, sx[rows], sw, bias=bias, epi=2, gate=mod, g_off=N, c=resid[rows])
    assert np.array_equal(got[rows], ref), report("gated", got[rows], ref)


@pytest.mark.parametrize("K,path", [(64, "in_gemm"), (192, "in_gemm"), (1024, "in_gemm"), (64, "scratch"),
                                    (1024, "scratch")])
def test_256_tile_kernel_w4_every_srel(ctx, w4_path, K, path):
    """W4 on the 256x256 kernel over all 256 s_rel bytes (fp8 e4m3 0 .. 480, so the grid clamps at
    +-127) with a non-uniform codebook reaching +-2 (a fitted one, quant.py:116-124), at
    M = N = 4096 (one tile per CU), unpacked inside the GEMM (K = 64 ends a tile at every stage,
    K = 192 alternates the stage parity across tiles, K = 1024 runs long tiles) and into the
    scratch grid.  int32 accumulators: checksums over the whole product and exact sampled rows;
    the store epilogue bit-exact."""
    case(f"256x256-tile kernel W4 every s_rel M=N=4096 K={K} {path}")
    w4_path(path)
    m = amd()
    M = N = 4096
    rng = np.random.default_rng(K)
    codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    srel = rng.integers(0, 256, size=(N, K // 16), dtype=np.uint8)
    srel[:, 0] = np.arange(N) % 256  # every byte value in use
    cb = np.sort(rng.uniform(-2.0, 2.0, 16)).astype(np.float32)
    sw = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
    qx = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    sx = rng.uniform(0.001, 0.01, M).astype(np.float32)
    W = m.weight(m.W_W4, N, K, ctx.upload(codes), scale=ctx.upload(sw), srel=ctx.upload(srel), codebook=ctx.upload(cb))
    grid = orc.w4_decode(codes, srel, cb, N, K)
    assert grid.min() == -127 or grid.max() == 127  # the clamp is exercised
    dout, dacc = ctx.empty((M, N)), ctx.empty((M, N), np.int32)
    ctx.linear(W, M, dout, xq=ctx.upload(qx), xs=ctx.upload(sx), acc_out=dacc)
    acc, got = dacc.numpy(), dout.numpy()
    assert checksums_ok(qx, grid, acc), "int32 accumulator checksums"
    rows = np.unique(np.concatenate([np.arange(0, 4), rng.choice(M, 16, replace=False), np.arange(M - 4, M)]))
    ref_acc = orc.gemm_i8(qx[rows], grid)
    assert np.array_equal(acc[rows], ref_acc)
    assert np.array_equal(got[rows], orc.linear_epilogue(ref_acc, sx[rows], sw))


@pytest.mark.parametrize("act,epi", [("gelu", 0), ("silu", 1)])
def test_256_tile_kernel_activation_epilogues(ctx, act, epi):
    """The 256x256 kernel with GELU (store) and SiLU (residual add) epilogues at M=4000, N=4100:
    accumulators exact (checksums + sampled rows), activations within 1e-6 relative of the
    oracle's correctly rounded formula (the device uses its 1-ulp reciprocal and exp2)."""
    case(f"256x256-tile kernel M=4000 N=4100 K=1024 {act} epi={epi}")
    m = amd()
    M, K, N = 4000, 1024, 4100
    x = orc.randn(97, M * K).reshape(M, K)
    qx, sx = orc.token_quant(orc.hadamard256(x))
    qw, sw = int8_weight(98, N, K)
    W = m.weight(m.W_I8, N, K, ctx.upload(qw), scale=ctx.upload(sw))
    resid = orc.randn(99, M * N).reshape(M, N)
    dout, dacc = ctx.upload(resid), ctx.empty((M, N), np.int32)
    ctx.linear(W, M, dout, xq=ctx.upload(qx), xs=ctx.upload(sx), act=act, epilogue=epi, acc_out=dacc)
    acc, got = dacc.numpy(), dout.numpy()
    assert checksums_ok(qx, qw, acc), "int32 accumulator checksums"
    rows = np.unique(np.concatenate([np.arange(0, 4), np.random.default_rng(2).choice(M, 16, replace=False),
                                     np.arange(M - 20, M)]))
    ref_acc = orc.gemm_i8(qx[rows], qw)
    assert np.array_equal(acc[rows], ref_acc)
    ref = orc.linear_epilogue(ref_acc, sx[rows], sw, act=1 if act == "gelu" else 2, epi=epi, c=resid[rows])
    g = got[rows]
    assert rel_l2(g, ref) < 1e-6 and np.max(np.abs(g - ref)) <= 1e-6 * np.max(np.abs(ref)), report(act, g, ref)


@pytest.mark.parametrize("act", ["gelu", "silu"])
def test_mlp1_activation_epilogue(ctx, act):
    case(f"mlp1 2048 -> 8192 {act} M=200 and mlp2 8192 -> 2048")
    m = amd()
    M, K, N = 200, 2048, 8192
    x = orc.randn(71, M * K).reshape(M, K)
    qw, sw = int8_weight(72, N, K)
    W = m.weight(m.W_I8, N, K, ctx.upload(qw), scale=ctx.upload(sw))
    dh = ctx.empty((M, N))
    ctx.linear(W, M, dh, x=ctx.upload(x), x_rotated=False, act=act)
    qx, sx = orc.token_quant(orc.hadamard256(x))
    ref = orc.linear_epilogue(orc.gemm_i8(qx, qw), sx, sw, act=1 if act == "gelu" else 2)
    got = dh.numpy()
    assert rel_l2(got, ref) < 1e-6 and np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref))
    # mlp2: K = 8192 input rotated + quantized inside the op
    qw2, sw2 = int8_weight(73, 2048, N)
    W2 = m.weight(m.W_I8, 2048, N, ctx.upload(qw2), scale=ctx.upload(sw2))
    dy = ctx.empty((M, 2048))
    ctx.linear(W2, M, dy, x=dh, x_rotated=False)
    qh, sh = orc.token_quant(orc.hadamard256(got))
    assert np.array_equal(dy.numpy(), orc.linear_epilogue(orc.gemm_i8(qh, qw2), sh, sw2))


def test_bf16_weight_linears(ctx):
    """bf16 weights widened exactly into the fp32 matrix-core kernels (x_embedder K=68 with a
    partial k-tile, final layer N=64 and a ragged N=200 on the tall-skinny kernel, a GELU epilogue
    on the swapped-operand kernel) and the M=1 GEMV, against float64."""
    case("bf16 weights: x_embedder K=68, final layer, GEMV M=1")
    m = amd()
    for (M, K, N, act) in ((300, 68, 2048, "none"), (1, 2048, 6144, "silu"), (97, 2048, 64, "none"),
                           (64, 1040, 200, "none"), (257, 1024, 516, "gelu")):
        x = orc.randn(81 + K, M * K).reshape(M, K)
        w32 = orc.bf16_round(0.05 * orc.randn(82 + N, N * K)).reshape(N, K)
        wb = (w32.view(np.uint32) >> 16).astype(np.uint16)
        bias = orc.randn(83, N).astype(np.float32)
        W = m.weight(m.W_BF16, N, K, ctx.upload(wb), bias=ctx.upload(bias))
        dy = ctx.empty((M, N))
        ctx.linear(W, M, dy, x=ctx.upload(x), act=act)
        ref = x.astype(np.float64) @ w32.astype(np.float64).T + bias
        if act == "silu":
            ref = ref / (1 + np.exp(-ref))
        elif act == "gelu":
            ref = np.vectorize(orc.gelu)(ref)
        r, _ = report(f"bf16 M={M} K={K} N={N}", dy.numpy(), ref)
        assert r < 1e-6


@pytest.mark.parametrize("M,K,N,epi", [(2048, 256, 2048, "store"), (512, 1024, 4096, "store"),
                                       (512, 2048, 1024, "resid"), (100, 3072, 1024, "gated"),
                                       (33, 1024, 388, "store"), (40, 224, 388, "gated"),
                                       (256, 384, 1152, "resid"), (32, 1056, 512, "store")])
def test_bf16_weight_split_kernel(ctx, M, K, N, epi):
    """bf16 weights with N > 256 and K % 32 == 0: x enters the bf16 matrix cores as three bf16
    terms, so every product is exact and the sums are fp32; within 1e-6 of float64 for each
    epilogue.  The shapes reach every kernel of the dispatch: the LDS-staged tiles (2048 x 256 x
    2048, 512 x 1024 x 4096: the text encoder's q/k/v and gate / up at 512 tokens), the k-sliced LDS
    kernel with its summing epilogue pass (512 x 2048 x 1024, 100 x 3072 x 1024, 33 x 1024 x 388:
    the o and down products, ragged M and N), and the register kernel with one, two and four
    k-groups per workgroup (40 x 224 x 388, 256 x 384 x 1152, 32 x 1056 x 512: too short a K
    for k-slices)."""
    case(f"bf16 split kernel M={M} K={K} N={N} epilogue {epi}")
    m = amd()
    x = orc.randn(151 + K, M * K).reshape(M, K)
    w32 = orc.bf16_round(0.05 * orc.randn(152 + N, N * K)).reshape(N, K)
    wb = (w32.view(np.uint32) >> 16).astype(np.uint16)
    bias = orc.randn(153, N).astype(np.float32)
    y0 = orc.randn(154, M * N).reshape(M, N)
    gate = orc.randn(155, N).astype(np.float32)
    W = m.weight(m.W_BF16, N, K, ctx.upload(wb), bias=ctx.upload(bias))
    dy = ctx.upload(y0)
    e = {"store": m.EPI_STORE, "resid": m.EPI_RESID, "gated": m.EPI_GATED}[epi]
    ctx.linear(W, M, dy, x=ctx.upload(x), epilogue=e, gate=ctx.upload(gate) if epi == "gated" else None)
    r64 = x.astype(np.float64) @ w32.astype(np.float64).T + bias
    ref = {"store": r64, "resid": y0 + r64, "gated": y0 + gate * r64}[epi]
    r, _ = report(f"bf16 split M={M} K={K} N={N} {epi}", dy.numpy(), ref)
    assert r < 1e-6


@pytest.mark.parametrize("M", [4000, 200])
def test_linear_add_term(ctx, M):
    """The optional fp32 add term (the LoRA delta input of gemm.js:189) after the bias: M=4000
    runs the 256-tile kernel (16-byte add rows, ld_add > N), M=200 the 128-tile kernel; gated
    epilogue, bit-exact against the oracle epilogue."""
    case(f"linear add term M={M} N=4100 K=1024 gated + bias")
    m = amd()
    K, N = 1024, 4100
    ld_add = N + 4
    x = orc.randn(131, M * K).reshape(M, K)
    qx, sx = orc.token_quant(orc.hadamard256(x))
    qw, sw = int8_weight(132, N, K)
    bias = (0.1 * orc.randn(133, N)).astype(np.float32)
    gate = orc.randn(134, 3 * N).astype(np.float32)
    resid = orc.randn(135, M * N).reshape(M, N)
    add = orc.randn(136, M * ld_add).reshape(M, ld_add)
    W = m.weight(m.W_I8, N, K, ctx.upload(qw), scale=ctx.upload(sw), bias=ctx.upload(bias))
    dout, dacc = ctx.upload(resid), ctx.empty((M, N), np.int32)
    ctx.linear(W, M, dout, xq=ctx.upload(qx), xs=ctx.upload(sx), epilogue=m.EPI_GATED, gate=ctx.upload(gate), gate_off=N,
               acc_out=dacc, add=ctx.upload(add), ld_add=ld_add)
    acc, got = dacc.numpy(), dout.numpy()
    assert checksums_ok(qx, qw, acc)
    rows = np.unique(np.concatenate([np.arange(0, 4), np.random.default_rng(3).choice(M, 12, replace=False),
                                     np.arange(M - 8, M)]))
    ref_acc = orc.gemm_i8(qx[rows], qw)
    assert np.array_equal(acc[rows], ref_acc)
    ref = orc.linear_epilogue(ref_acc, sx[rows], sw, bias=bias, epi=2, gate=gate, g_off=N, c=resid[rows],
                              add=np.ascontiguousarray(add[rows, :N]))
    assert np.array_equal(got[rows], ref), report("add term", got[rows], ref)


@pytest.mark.parametrize("M,epi,act", [(4000, "gated", "none"), (4000, "store", "gelu"), (4000, "resid", "none"),
                                       (200, "gated", "none")])
def test_linear_lora_epilogue(ctx, M, epi, act):
    """The LoRA delta computed from its two factors in the quantized GEMM (anima_linear_desc
    lora_xa / lora_b / lora_r): y += xa[m] . B[n] after the bias, before the activation / gate
    (ops.js:55-87 with the scale folded into B).  xa [M, R] fp32 with ld > R, B [N, R] as three
    bf16 planes (anima_split3_bf16), R = 48 (three 16-k slices); N = 4100 leaves a partial column
    tile.  M = 4000 runs the 256-tile kernel with the product inside its epilogue, M = 200 the
    128-tile kernel with the product as an add term.  Against the oracle epilogue fed the float64
    delta (rounded to fp32): rel-L2 <= 2e-6; the int32 accumulators bit-exact."""
    case(f"linear LoRA epilogue M={M} {epi} act={act}")
    m = amd()
    K, N, R, ld = 1024, 4100, 48, 52
    x = orc.randn(141, M * K).reshape(M, K)
    qx, sx = orc.token_quant(orc.hadamard256(x))
    qw, sw = int8_weight(142, N, K)
    bias = (0.1 * orc.randn(143, N)).astype(np.float32)
    gate = orc.randn(144, 3 * N).astype(np.float32)
    resid = orc.randn(145, M * N).reshape(M, N)
    xa = (0.5 * orc.randn(146, M * ld)).reshape(M, ld).astype(np.float32)
    Bm = (0.05 * orc.randn(147, N * R)).reshape(N, R).astype(np.float32)
    dB = ctx.upload(Bm)
    planes = ctx.empty(3 * N * R, np.uint16)
    ctx.split3_bf16(dB, planes, N * R)
    W = m.weight(m.W_I8, N, K, ctx.upload(qw), scale=ctx.upload(sw), bias=ctx.upload(bias))
    dout, dacc = ctx.upload(resid), ctx.empty((M, N), np.int32)
    e = {"store": m.EPI_STORE, "resid": m.EPI_RESID, "gated": m.EPI_GATED}[epi]
    ctx.linear(W, M, dout, xq=ctx.upload(qx), xs=ctx.upload(sx), epilogue=e, gate=ctx.upload(gate), gate_off=N,
               act=act, acc_out=dacc, lora_xa=ctx.upload(xa), ld_lora_xa=ld, lora_b=planes, lora_r=R)
    acc, got = dacc.numpy(), dout.numpy()
    assert checksums_ok(qx, qw, acc)
    rows = np.unique(np.concatenate([np.arange(0, 4), np.random.default_rng(5).choice(M, 12, replace=False),
                                     np.arange(M - 8, M)]))
    ref_acc = orc.gemm_i8(qx[rows], qw)
    assert np.array_equal(acc[rows], ref_acc)
    delta = (xa[rows, :R].astype(np.float64) @ Bm.astype(np.float64).T).astype(np.float32)
    ref = orc.linear_epilogue(ref_acc, sx[rows], sw, bias=bias, act={"none": 0, "gelu": 1}[act], epi=e, gate=gate,
                              g_off=N, c=resid[rows] if epi != "store" else None, add=delta)
    r, _ = report(f"LoRA epilogue {epi} {act} M={M}", got[rows], ref)
    assert r <= 2e-6


@pytest.mark.parametrize("M,N,cols", [(4000, 3072, 1024), (4000, 1152, 384), (200, 3072, 1024)])
def test_linear_lora_block_diagonal(ctx, M, N, cols):
    """Block-diagonal LoRA ranks (lora_cols: a stacked projection whose column blocks carry their
    own ranks, e.g. q / k / v): column n adds xa[m, (n // cols) * R + k] * B[n, k], B holding only
    each block's R = 32 ranks.  cols = 1024 runs the product inside the 256-tile kernel's
    epilogue (a tile lies in one block); cols = 384 splits tiles and M = 200 runs the 128-tile
    kernel, both taking the product as an add term, one split-bf16 product per block over its
    rows of the B planes.  Against the oracle epilogue fed the float64 delta: rel-L2 <= 2e-6."""
    case(f"linear LoRA block-diagonal M={M} N={N} cols={cols}")
    m = amd()
    K, R = 1024, 32
    nb = N // cols
    ld = nb * R + 4
    x = orc.randn(241, M * K).reshape(M, K)
    qx, sx = orc.token_quant(orc.hadamard256(x))
    qw, sw = int8_weight(242, N, K)
    gate = orc.randn(244, N).astype(np.float32)
    resid = orc.randn(245, M * N).reshape(M, N)
    xa = (0.5 * orc.randn(246, M * ld)).reshape(M, ld).astype(np.float32)
    Bm = (0.05 * orc.randn(247, N * R)).reshape(N, R).astype(np.float32)
    planes = ctx.empty(3 * N * R, np.uint16)
    ctx.split3_bf16(ctx.upload(Bm), planes, N * R)
    W = m.weight(m.W_I8, N, K, ctx.upload(qw), scale=ctx.upload(sw))
    dout = ctx.upload(resid)
    ctx.linear(W, M, dout, xq=ctx.upload(qx), xs=ctx.upload(sx), epilogue=m.EPI_GATED, gate=ctx.upload(gate),
               lora_xa=ctx.upload(xa), ld_lora_xa=ld, lora_b=planes, lora_r=R, lora_cols=cols)
    got = dout.numpy()
    rows = np.unique(np.concatenate([np.arange(0, 4), np.random.default_rng(6).choice(M, 12, replace=False),
                                     np.arange(M - 8, M)]))
    delta = np.zeros((len(rows), N))
    for b in range(nb):
        c = slice(b * cols, (b + 1) * cols)
        delta[:, c] = xa[rows, b * R:(b + 1) * R].astype(np.float64) @ Bm[c].astype(np.float64).T
    ref = orc.linear_epilogue(orc.gemm_i8(qx[rows], qw), sx[rows], sw, epi=m.EPI_GATED, gate=gate, g_off=0,
                              c=resid[rows], add=delta.astype(np.float32))
    r, _ = report(f"LoRA block-diagonal M={M} cols={cols}", got[rows], ref)
    assert r <= 2e-6


def test_linear_lora_epilogue_refusals(ctx):
    """The LoRA factors are refused on the host: a rank that is not a multiple of 16 or an ld below
    it, rank blocks that do not divide N or whose ranks do not fit the ld (ANIMA_E_ARG), together
    with an add term or on a bf16 weight (ANIMA_E_UNSUPPORTED)."""
    case("linear LoRA epilogue refusals")
    m = amd()
    buf = ctx.empty(1 << 20)
    W = m.weight(m.W_I8, 64, 128, buf, scale=buf)
    for kw, code in ((dict(lora_r=40, ld_lora_xa=40), -1), (dict(lora_r=32, ld_lora_xa=16), -1),
                     (dict(lora_r=32, ld_lora_xa=64, lora_cols=24), -1), (dict(lora_r=32, ld_lora_xa=32, lora_cols=32), -1),
                     (dict(lora_r=32, ld_lora_xa=32, add=buf, ld_add=64), -5)):
        with pytest.raises(m.AnimaError) as e:
            ctx.linear(W, 4, buf, xq=buf, xs=buf, lora_xa=buf, lora_b=buf, **kw)
        assert e.value.code == code, (kw, e.value)
    Wb = m.weight(m.W_BF16, 64, 128, buf)
    with pytest.raises(m.AnimaError) as e:
        ctx.linear(Wb, 4, buf, x=buf, lora_xa=buf, lora_b=buf, lora_r=32, ld_lora_xa=32)
    assert e.value.code == -5


def test_f32_weight_linears(ctx):
    """fp32 weights (the LoRA A / B matrices): tall-skinny and short-K shapes against float64,
    with alpha, column offset into a wider output (ldc) and residual accumulation."""
    case("fp32 weights: LoRA A (N=16, K=2048) and B (N=2048, K=16)")
    m = amd()
    M = 300
    x = orc.randn(141, M * 2048).reshape(M, 2048)
    A = (0.05 * orc.randn(142, 16 * 2048)).reshape(16, 2048).astype(np.float32)
    B = (0.05 * orc.randn(143, 2048 * 16)).reshape(2048, 16).astype(np.float32)
    WA = m.weight(m.W_F32, 16, 2048, ctx.upload(A))
    t = ctx.empty((M, 16))
    ctx.linear(WA, M, t, x=ctx.upload(x))
    t_ref = x.astype(np.float64) @ A.T
    assert report("x A^T", t.numpy(), t_ref)[0] < 1e-6
    WB = m.weight(m.W_F32, 2048, 16, ctx.upload(B))
    base = orc.randn(144, M * 2560).reshape(M, 2560)
    dd = ctx.upload(base)
    ctx.linear(WB, M, dd.ptr + 256 * 4, x=t, ldc=2560, alpha=0.5, epilogue=m.EPI_RESID)
    ref = base.astype(np.float64)
    ref[:, 256:2304] += 0.5 * (t.numpy().astype(np.float64) @ B.T)
    assert report("+= 0.5 t B^T into columns 256..2303", dd.numpy(), ref)[0] < 1e-6


@pytest.mark.parametrize("N,K,M", [(32, 2048, 257), (64, 1040, 64), (96, 2048, 300), (200, 8192, 45)])
def test_f32_tall_skinny(ctx, N, K, M):
    """The tall-skinny fp32 product (stacked LoRA A matrices, N <= 256, K >= 512): every column
    tile count, a partial last k-tile (K = 1040), partial row / column blocks, bias + store and
    a ldx wider than K, against float64."""
    case(f"fp32 tall-skinny N={N} K={K} M={M}")
    m = amd()
    ldx = K + 12
    x = orc.randn(151, M * ldx).reshape(M, ldx)
    A = (0.05 * orc.randn(152, N * K)).reshape(N, K).astype(np.float32)
    bias = orc.randn(153, N).astype(np.float32)
    W = m.weight(m.W_F32, N, K, ctx.upload(A), bias=ctx.upload(bias))
    t = ctx.empty((M, N))
    ctx.linear(W, M, t, x=ctx.upload(x), ldx=ldx, alpha=0.75)
    ref = 0.75 * (x[:, :K].astype(np.float64) @ A.T.astype(np.float64)) + bias
    assert report("0.75 x A^T + b", t.numpy(), ref)[0] < 1e-6


def split3_host(a):
    """The three bf16 planes of anima_split3_bf16, restated: each plane is the round-to-nearest-
    even bf16 of what the previous planes leave (the differences are exact in fp32)."""
    a = np.asarray(a, np.float32)
    h = orc.bf16_round(a)
    r = (a - h).astype(np.float32)
    m = orc.bf16_round(r)
    l_ = orc.bf16_round((r - m).astype(np.float32))
    return [h, m, l_]


def bits16(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_split3_planes(ctx):
    """anima_split3_bf16: every plane bit-exact against the restatement; the three planes sum to
    the fp32 input within 2^-24 relative (and exactly for values with <= 24 significant bits)."""
    case("split3 bf16 planes")
    n = 8 * 12345
    x = (orc.randn(161, n) * np.exp(orc.randn(162, n))).astype(np.float32)
    x[:8] = [0.0, -0.0, 1.0, -3.5, 1e-30, 3.0e38, 2 ** -20, 1.0 + 2 ** -23]
    dst = ctx.empty((3, n), np.uint16)
    ctx.split3_bf16(ctx.upload(x), dst, n)
    got = dst.numpy()
    ref = split3_host(x)
    for p in range(3):
        assert np.array_equal(got[p], bits16(ref[p])), p
    tot = sum(r.astype(np.float64) for r in ref)
    assert np.all(np.abs(tot - x) <= 2.0 ** -24 * np.abs(x.astype(np.float64)) + 1e-45)
    with pytest.raises(amd().AnimaError):
        ctx.split3_bf16(ctx.upload(x), dst, 12)


@pytest.mark.parametrize("N,K,M,epi", [(32, 2048, 257, "store"), (96, 2048, 300, "store"), (200, 1040, 45, "store"),
                                      (32, 1032, 70, "store"), (64, 520, 33, "resid"), (96, 1544, 64, "gated"),
                                      (30, 1040, 33, "resid"),
                                      (2048, 32, 300, "resid"), (2048, 8, 97, "gated"), (516, 24, 64, "store"),
                                      (2052, 40, 8200, "resid")])
def test_split3_linears(ctx, N, K, M, epi):
    """ANIMA_W_F32S3 (fp32 matrices as three bf16 planes, products split the same way on the
    bf16 matrix cores): the tall-skinny LoRA-A shapes (ragged N and M; K = 1032, 520, 1544 end
    inside a 32-k step; N = 30 at M = 33 makes M * N odd, summed element by element) and the
    swapped-operand LoRA-B shapes (K = rank 32 / 8 / 24, store / residual into a wider output /
    gated; at M = 8200, N = 2052, K = 40 the four-tiles-per-wave grid with ragged rows, columns and
    a partial k-chunk) within 1e-6 of float64, as the fp32 kernels."""
    case(f"split3 linear N={N} K={K} M={M} {epi}")
    m = amd()
    ldx = K + 8
    x = orc.randn(171, M * ldx).reshape(M, ldx)
    w = (0.05 * orc.randn(172, N * K)).reshape(N, K).astype(np.float32)
    dw = ctx.empty((3, N, K), np.uint16)
    ctx.split3_bf16(ctx.upload(w), dw, N * K)
    W = m.weight(m.W_F32S3, N, K, dw)
    ref = 0.5 * (x[:, :K].astype(np.float64) @ w.T.astype(np.float64))
    ldc = N + 12
    base = orc.randn(173, M * ldc).reshape(M, ldc)
    gate = orc.randn(174, N).astype(np.float32)
    dout = ctx.upload(base)
    kw = dict(x=ctx.upload(x), ldx=ldx, ldc=ldc, alpha=0.5)
    if epi == "resid":
        kw["epilogue"] = m.EPI_RESID
    elif epi == "gated":
        kw.update(epilogue=m.EPI_GATED, gate=ctx.upload(gate))
    ctx.linear(W, M, dout, **kw)
    want = base.astype(np.float64)
    if epi == "store":
        want[:, :N] = ref
    elif epi == "resid":
        want[:, :N] += ref
    else:
        want[:, :N] += gate.astype(np.float64) * ref
    got = dout.numpy()
    assert np.array_equal(got[:, N:], base[:, N:])
    assert report(f"split3 {epi}", got[:, :N], want[:, :N])[0] < 1e-6


@pytest.mark.parametrize("N,K,M,epi", [(32, 2048, 257, "store"), (96, 2048, 4000, "store"), (64, 8192, 600, "store"),
                                      (200, 1040, 45, "gated"), (48, 256, 70, "resid"), (300, 512, 33, "store")])
def test_split3_int8_rows(ctx, N, K, M, epi):
    """ANIMA_W_F32S3 over per-token int8 rows (xq, xs; the LoRA A product of a quantized linear
    from the rows its GEMM reads): y = alpha * xs[m] * sum_k q[m][k] W[n][k] within 1e-6 of
    float64.  The tall kernel with int8 x (rank 32 / 96 / 64 at K = 2048 / 8192; N = 200 in
    64-column workgroups with K = 1040 ending inside a 32-k step; ragged M) and the shapes it does
    not take (K < 512, N > 256: the rows widened to fp32 first)."""
    case(f"split3 int8 rows N={N} K={K} M={M} {epi}")
    m = amd()
    rng = np.random.default_rng(181)
    ldx = K + 16
    q = rng.integers(-127, 128, size=(M, ldx), dtype=np.int8)
    s = rng.uniform(0.001, 0.02, M).astype(np.float32)
    w = (0.05 * orc.randn(182, N * K)).reshape(N, K).astype(np.float32)
    dw = ctx.empty((3, N, K), np.uint16)
    ctx.split3_bf16(ctx.upload(w), dw, N * K)
    W = m.weight(m.W_F32S3, N, K, dw)
    ref = 0.5 * s.astype(np.float64)[:, None] * (q[:, :K].astype(np.float64) @ w.T.astype(np.float64))
    ldc = N + 12
    base = orc.randn(183, M * ldc).reshape(M, ldc)
    gate = orc.randn(184, N).astype(np.float32)
    dout = ctx.upload(base)
    dq, ds = ctx.upload(q), ctx.upload(s)
    kw = dict(xq=dq, xs=ds, ldx=ldx, ldc=ldc, alpha=0.5)
    if epi == "resid":
        kw["epilogue"] = m.EPI_RESID
    elif epi == "gated":
        kw.update(epilogue=m.EPI_GATED, gate=ctx.upload(gate))
    ctx.linear(W, M, dout, **kw)
    want = base.astype(np.float64)
    if epi == "store":
        want[:, :N] = ref
    elif epi == "resid":
        want[:, :N] += ref
    else:
        want[:, :N] += gate.astype(np.float64) * ref
    got = dout.numpy()
    assert np.array_equal(got[:, N:], base[:, N:])
    assert report(f"split3 int8 rows {epi}", got[:, :N], want[:, :N])[0] < 1e-6
    # refused: int8 rows with x as well, without their scales, or with K % 16 != 0
    with pytest.raises(m.AnimaError):
        ctx.linear(W, M, dout, x=ctx.upload(base), **kw)
    with pytest.raises(m.AnimaError):
        ctx.linear(W, M, dout, xq=dq, ldx=ldx, ldc=ldc)
    W8 = m.weight(m.W_F32S3, N, K - 8, dw)
    with pytest.raises(m.AnimaError):
        ctx.linear(W8, M, dout, xq=dq, xs=ds, ldx=ldx, ldc=ldc)


def test_grouped_bf16_gemv(ctx):
    """G products in one launch (the adaLN modulation stage of timeCond): every group bit-exact
    against its own anima_linear GEMV call with the same bias, and within 1e-6 of float64."""
    case("grouped bf16 GEMV G=9 M=1 N=768 K=256, shared bias")
    m = amd()
    G, M, N, K = 9, 1, 768, 256
    x = orc.randn(101, G * K).reshape(G, K)  # group g reads x[g]
    w32 = orc.bf16_round(0.05 * orc.randn(102, G * N * K)).reshape(G, N, K)
    wb = np.ascontiguousarray((w32.view(np.uint32) >> 16).astype(np.uint16))
    bias = orc.randn(103, N).astype(np.float32)
    dx, dw, db = ctx.upload(x), ctx.upload(wb), ctx.upload(bias)
    dy = ctx.empty((G, N))
    ctx.linear_grouped_bf16(G, M, N, K, dx, K, K, dw, N * K, db, 0, dy, N, N)
    got = dy.numpy()
    for g in range(G):
        W = m.weight(m.W_BF16, N, K, ctx.upload(wb[g]), bias=db)
        one = ctx.empty((1, N))
        ctx.linear(W, 1, one, x=ctx.upload(x[g:g + 1]))
        assert np.array_equal(got[g], one.numpy()[0]), g
        ref = x[g].astype(np.float64) @ w32[g].astype(np.float64).T + bias
        r, _ = report(f"group {g}", got[g], ref)
        assert r < 1e-6
    with pytest.raises(m.AnimaError):
        ctx.linear_grouped_bf16(G, 9, N, K, dx, K, K, dw, N * K, db, 0, dy, N, N)  # M > 8


def test_linear_rejects_bad_arguments(ctx):
    case("linear argument validation")
    m = amd()
    buf = ctx.empty(1 << 16)
    W = m.weight(m.W_I8, 64, 100, buf, scale=buf)
    with pytest.raises(m.AnimaError) as e:
        ctx.linear(W, 4, buf, xq=buf, xs=buf)
    assert e.value.code == -1  # K % 64
    W = m.weight(7, 64, 128, buf, scale=buf)
    with pytest.raises(m.AnimaError):
        ctx.linear(W, 4, buf, xq=buf, xs=buf)
    W = m.weight(m.W_I8, 64, 128, buf, scale=buf)
    with pytest.raises(m.AnimaError):
        ctx.linear(W, 4, buf, xq=buf, xs=buf, epilogue=m.EPI_GATED)  # no gate
    with pytest.raises(m.AnimaError) as e:
        ctx.set_w4_path(2)  # neither ANIMA_W4_GRID_SCRATCH nor ANIMA_W4_IN_GEMM
    assert e.value.code == -1


@pytest.mark.parametrize("K", [64, 2048])
def test_weight_unpack_w4_grid_and_linear(ctx, K):
    """anima_weight_unpack_w4: the int8 grid of a W4 weight equals the oracle's decode
    (quant.py:127-129 / gemm.js:141-158) for every s_rel byte and a clamping codebook, and the i8
    weight {grid, s_channel} gives the same linear output and accumulators as the W4 weight."""
    case(f"W4 -> int8 grid unpack N=512 K={K}")
    m = amd()
    N, M = 512, 300
    rng = np.random.default_rng(K + 5)
    codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    srel = rng.integers(0, 256, size=(N, K // 16), dtype=np.uint8)
    srel[:, 0] = np.arange(N) % 256
    cb = np.sort(rng.uniform(-2.0, 2.0, 16)).astype(np.float32)
    sw = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
    dsw = ctx.upload(sw)
    W4 = m.weight(m.W_W4, N, K, ctx.upload(codes), scale=dsw, srel=ctx.upload(srel), codebook=ctx.upload(cb))
    dgrid = ctx.empty((N, K), np.int8)
    ctx.weight_unpack_w4(W4, dgrid)
    grid = dgrid.numpy()
    assert np.array_equal(grid, orc.w4_decode(codes, srel, cb, N, K))
    W8 = m.weight(m.W_I8, N, K, dgrid, scale=dsw)
    qx = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    sx = rng.uniform(0.001, 0.01, M).astype(np.float32)
    dq, ds = ctx.upload(qx), ctx.upload(sx)
    outs = []
    for W in (W4, W8):
        do, da = ctx.empty((M, N)), ctx.empty((M, N), np.int32)
        ctx.linear(W, M, do, xq=dq, xs=ds, acc_out=da)
        outs.append((do.numpy(), da.numpy()))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    with pytest.raises(m.AnimaError):
        ctx.weight_unpack_w4(W8, dgrid)  # not a W4 weight


@pytest.mark.parametrize("G,N,K,acc", [(85, 256, 32, True), (84, 32, 256, False), (1, 2720, 2048, False),
                                       (3, 6144, 8, True)])
def test_gemv_grouped_f32(ctx, G, N, K, acc):
    """anima_gemv_grouped_f32 (the grouped LoRA products of the adaLN modulation): y_g = alpha W_g x_g
    (+ y_g) for G groups in one launch, within 1e-6 of float64 (first-stage B products: 85 x 256
    from rank 32; second-stage A products: 84 x rank 32 from 256; one stacked A product over K =
    2048; gaps between the groups' x and y slices)."""
    case(f"grouped fp32 GEMV G={G} N={N} K={K} acc={acc}")
    m = amd()
    xs, ys = K + 4, N + 8
    x = orc.randn(191, G * xs).astype(np.float32)
    w = (0.05 * orc.randn(192, G * N * K)).astype(np.float32)
    y0 = orc.randn(193, G * ys).astype(np.float32)
    dx, dw, dy = ctx.upload(x), ctx.upload(w), ctx.upload(y0)
    ctx.gemv_grouped_f32(G, N, K, dx, xs, dw, N * K, dy, ys, alpha=0.75, accumulate=acc)
    got = dy.numpy().reshape(G, ys)
    X = x.reshape(G, xs)[:, :K].astype(np.float64)
    Wm = w.reshape(G, N, K).astype(np.float64)
    ref = 0.75 * np.einsum("gnk,gk->gn", Wm, X)
    want = y0.reshape(G, ys).astype(np.float64).copy()
    want[:, :N] = want[:, :N] + ref if acc else ref
    assert np.array_equal(got[:, N:], y0.reshape(G, ys)[:, N:])
    assert report("grouped fp32 GEMV", got[:, :N], want[:, :N])[0] < 1e-6
    with pytest.raises(m.AnimaError):
        ctx.gemv_grouped_f32(G, N, K + 2, dx, xs, dw, N * K, dy, ys)
    with pytest.raises(m.AnimaError):
        ctx.gemv_grouped_f32(G, N, K, dx, xs + 2, dw, N * K, dy, ys)


@pytest.mark.parametrize("K,rotate", [(2048, True), (1024, False), (8192, True)])
def test_quant_rows_bf16(ctx, K, rotate):
    """anima_quant_rows_bf16 (the quantized output projection's input written as bf16 by the
    attention): int8 rows and scales bit-identical to anima_quant_rows on the rows widened to fp32,
    and to the oracle's token quantization of them; M = 300 (a partial last workgroup), a zero row."""
    case(f"quant_rows_bf16 K={K} rotate={rotate}")
    M = 300
    x = orc.bf16_round(3 * orc.randn(201, M * K)).reshape(M, K)
    x[7] = 0.0
    bits = (x.view(np.uint32) >> 16).astype(np.uint16)
    q1, s1 = ctx.empty((M, K), np.int8), ctx.empty(M)
    q2, s2 = ctx.empty((M, K), np.int8), ctx.empty(M)
    ctx.quant_rows_bf16(ctx.upload(bits), M, K, rotate, q1, s1)
    ctx.quant_rows(ctx.upload(x), M, K, rotate, q2, s2)
    assert np.array_equal(q1.numpy(), q2.numpy()) and np.array_equal(s1.numpy(), s2.numpy())
    q, s = orc.token_quant(orc.hadamard256(x) if rotate else x)
    assert np.array_equal(q1.numpy(), q) and np.array_equal(s1.numpy(), s)
    with pytest.raises(amd().AnimaError):
        ctx.quant_rows_bf16(ctx.upload(bits), M, 768, rotate, q1, s1)
