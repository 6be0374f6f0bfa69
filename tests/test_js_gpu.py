"""GPU parity of the JavaScript host path (ops.mjs -> N-API addon -> libanima.so) against the
oracle: the same bars as the direct C-ABI tests, through the reference's op signatures."""

import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from helpers import PKG_DIR, RUN_CASE, report

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]

JS = os.path.join(PKG_DIR, "js")
HD = 128


def run_case(tmp_path, spec, flags=()):
    path = tmp_path / "case.json"
    path.write_text(json.dumps(spec))
    print(f"[case] js {spec['case']}", flush=True)
    r = subprocess.run(["node", *flags, RUN_CASE, str(path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    return r


def write(tmp_path, name, arr):
    p = tmp_path / name
    np.ascontiguousarray(arr).tofile(p)
    return str(p)


def read(path, dtype=np.float32):
    return np.fromfile(path, dtype)


def test_js_attention_fused(tmp_path):
    B, Hp, Wp, H = 2, 32, 32, 16
    L = Hp * Wp
    qkv = orc.randn(91, B * L * 3 * H * HD).reshape(B, L, 3 * H * HD)
    qn = (1 + 0.02 * orc.randn(92, HD)).astype(np.float32)
    kn = (1 + 0.02 * orc.randn(93, HD)).astype(np.float32)
    out = str(tmp_path / "o.bin")
    run_case(tmp_path, {"case": "attention", "B": B, "Hp": Hp, "Wp": Wp, "H": H, "precision": "bf16",
                        "qkv": write(tmp_path, "qkv.bin", qkv), "qn": write(tmp_path, "qn.bin", qn),
                        "kn": write(tmp_path, "kn.bin", kn), "out": out})
    cs = orc.dit_rope_table(Hp, Wp)
    assert np.array_equal(read(out + ".cs"), cs)  # the JS-built RoPE table
    got = read(out).reshape(B, L, H * HD)
    ld = 3 * H * HD
    rows = np.arange(0, L, 7)
    for b in range(B):
        nq = orc.qk_norm_rope(qkv[b], L, H, HD, ld, qn, kn, cs, L * 64)
        model = orc.attention("bf16", np.ascontiguousarray(nq[rows]), nq, nq, B=1, Lq=len(rows), Lk=L, H=H, D=HD,
                              ldq=ld, ldk=ld, ldv=ld, k_off=H * HD, v_off=2 * H * HD)[0]
        assert report(f"js attention b={b} vs bf16 model", got[b, rows], model)[0] <= 3e-4


def test_js_attention_default_precision_is_fp32(tmp_path):
    """ops.attention without a precision runs the reference's fp32 arithmetic (the fp32-MFMA kernel):
    within the fp32 bar of the float64 oracle, which the bf16 kernel (~3e-3) would miss."""
    B, Hp, Wp, H = 1, 16, 16, 4
    L = Hp * Wp
    qkv = orc.randn(95, B * L * 3 * H * HD).reshape(B, L, 3 * H * HD)
    qn = (1 + 0.02 * orc.randn(96, HD)).astype(np.float32)
    kn = (1 + 0.02 * orc.randn(97, HD)).astype(np.float32)
    out = str(tmp_path / "o.bin")
    run_case(tmp_path, {"case": "attention", "B": B, "Hp": Hp, "Wp": Wp, "H": H, "qkv": write(tmp_path, "qkv.bin", qkv),
                        "qn": write(tmp_path, "qn.bin", qn), "kn": write(tmp_path, "kn.bin", kn), "out": out})
    cs = orc.dit_rope_table(Hp, Wp)
    ld = 3 * H * HD
    nq = orc.qk_norm_rope(qkv[0], L, H, HD, ld, qn, kn, cs, L * 64)
    ref = orc.attention("f64", nq, nq, nq, B=1, Lq=L, Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld, k_off=H * HD,
                        v_off=2 * H * HD)[0]
    assert report("js attention (default precision) vs fp64", read(out).reshape(L, H * HD), ref)[0] <= 1e-5


def test_js_tensor_finalizer_returns_dropped_buffers(tmp_path):
    """Device Tensors dropped without release() go back to the pool when the garbage collector
    reclaims their handles (the leak guard of gpu.mjs / addon.c); release() disarms the finalizer."""
    r = run_case(tmp_path, {"case": "leak", "n": 24, "mb": 64}, flags=("--expose-gc",))
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"leak"' in ln))["leak"]
    print(f"leak guard: {info}", flush=True)
    assert info["finalized"] >= info["n"] - 2  # the last allocations may still be referenced
    assert info["peak"] <= 6 * info["bytes"]  # freed buffers are reused, not accumulated
    assert info["released_twice_ok"]


def test_js_device_limits(tmp_path):
    """GPU.limits / GPU.maxBinding carry the device's limits under WebGPU's names
    (app/gpu/device.js:83-88): the buffer and binding bounds are the device memory."""
    r = run_case(tmp_path, {"case": "limits"})
    d = json.loads(next(ln for ln in r.stdout.splitlines() if '"limits"' in ln))
    L = d["limits"]
    print(f"js limits: {d}", flush=True)
    assert d["maxBinding"] == min(L["maxStorageBufferBindingSize"], L["maxBufferSize"]) >= 250 * 10**9
    assert L["maxComputeWorkgroupStorageSize"] >= 64 * 1024 and L["subgroupSize"] == 64
    assert d["info"]["architecture"] == "gfx950"


def test_js_exit_with_unreleased_tensors(tmp_path):
    """A script that ends normally -- no release(), no destroy(), no process.exit() -- with device
    Tensors outstanding (collected, unreachable and still referenced) exits with status 0: the
    addon's environment cleanup hook retires the buffer handles before Node's N-API teardown."""
    r = run_case(tmp_path, {"case": "teardown", "n": 24}, flags=("--expose-gc",))
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"teardown"' in ln))["teardown"]
    print(f"teardown: {info}, rc {r.returncode}", flush=True)
    assert r.returncode == 0 and info["kept"] == 8
    assert "Segmentation" not in r.stderr and "FATAL" not in r.stderr


def test_js_qk_norm_rope_bit_exact(tmp_path):
    Hp, Wp, H = 16, 16, 16
    L = Hp * Wp
    qkv = orc.randn(94, L * 3 * H * HD).reshape(L, 3 * H * HD)
    qn = (1 + 0.02 * orc.randn(95, HD)).astype(np.float32)
    kn = (1 + 0.02 * orc.randn(96, HD)).astype(np.float32)
    out = str(tmp_path / "x.bin")
    run_case(tmp_path, {"case": "qknr", "Hp": Hp, "Wp": Wp, "H": H, "qkv": write(tmp_path, "qkv.bin", qkv),
                        "qn": write(tmp_path, "qn.bin", qn), "kn": write(tmp_path, "kn.bin", kn), "out": out})
    ref = orc.qk_norm_rope(qkv, L, H, HD, 3 * H * HD, qn, kn, orc.dit_rope_table(Hp, Wp), L * 64)
    assert np.array_equal(read(out).reshape(ref.shape), ref)


@pytest.mark.parametrize("kind", ["i8", "w4"])
def test_js_linear_gated(tmp_path, kind):
    M, K, N = 300, 2048, 2048
    x = orc.randn(97, M * K).reshape(M, K)
    resid = orc.randn(98, M * N).reshape(M, N)
    gate = orc.randn(99, 3 * N).astype(np.float32)
    rng = np.random.default_rng(5)
    sw = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
    W = {"kind": kind, "N": N, "K": K, "scale": write(tmp_path, "sw.bin", sw)}
    if kind == "i8":
        qw = np.clip(np.rint(40 * orc.randn(100, N * K)), -127, 127).astype(np.int8).reshape(N, K)
        W["w"] = write(tmp_path, "w.bin", qw)
        grid = qw
    else:
        codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
        srel = rng.integers(0x60, 0x70, size=(N, K // 16), dtype=np.uint8)
        cb = np.array([-0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
                       0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671], np.float32)
        W.update(w=write(tmp_path, "w.bin", codes), srel=write(tmp_path, "sr.bin", srel), codebook=write(tmp_path, "cb.bin", cb))
        grid = orc.w4_decode(codes, srel, cb, N, K)
    out = str(tmp_path / "y.bin")
    run_case(tmp_path, {"case": "linear", "M": M, "W": W, "x": write(tmp_path, "x.bin", x), "resid": write(tmp_path, "r.bin", resid),
                        "gate": write(tmp_path, "g.bin", gate), "gOff": 2 * N, "out": out})
    qx, sx = orc.token_quant(orc.hadamard256(x))
    ref = orc.linear_epilogue(orc.gemm_i8(qx, grid), sx, sw, epi=2, gate=gate, g_off=2 * N, c=resid)
    assert np.array_equal(read(out).reshape(M, N), ref)


def test_js_layernorm_mod(tmp_path):
    rows, cols = 257, 2048
    x = orc.randn(101, rows * cols).reshape(rows, cols)
    mod = (0.1 * orc.randn(102, 3 * cols)).astype(np.float32)
    out = str(tmp_path / "y.bin")
    run_case(tmp_path, {"case": "lnmod", "rows": rows, "cols": cols, "rotate": True, "x": write(tmp_path, "x.bin", x),
                        "mod": write(tmp_path, "m.bin", mod), "out": out})
    ref = orc.layernorm_mod(x, mod, 0, cols, cols, rotate=True)
    assert np.array_equal(read(out).reshape(rows, cols), ref)
    q, s = orc.token_quant(ref)
    assert np.array_equal(read(out + ".q", np.int8).reshape(rows, cols), q)
    assert np.array_equal(read(out + ".s"), s)


def test_js_dit_step_synthetic_smoke():
    """The full step machinery through JS: 2 blocks at 512x512 (mixed int8 layout), finite output."""
    print("[case] js bench_dit 2 blocks 512", flush=True)
    r = subprocess.run(["node", os.path.join(JS, "bench_dit.mjs"), "--size", "512", "--blocks", "3", "--steps", "1",
                        "--warmup", "1"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    print(out, flush=True)
    assert out["finite"] and out["dit_step_ms"] > 0


# ------------------------------------------------------------------ LoRA side paths (ops.js:55-87)

def lora_delta(xin, entries, N):
    """sum_e scale_e * (xin A_e^T) B_e^T on columns [off, off + n), in float64."""
    d = np.zeros((xin.shape[0], N))
    for e in entries:
        d[:, e["off"]:e["off"] + e["n"]] += e["scale"] * ((xin.astype(np.float64) @ e["A"].T.astype(np.float64))
                                                           @ e["B"].T.astype(np.float64))
    return d


@pytest.mark.parametrize("kind,act,stack,rotated", [("i8", "none", False, False), ("bf16", "none", False, False),
                                                    ("i8", "gelu", True, False), ("bf16", "gelu", False, False),
                                                    ("i8", "none", True, True), ("i8", "gelu", False, True)])
def test_js_linear_lora(tmp_path, kind, act, stack, rotated):
    """ops.linear with two LoRA entries (a full-width one and a column slice): the delta enters
    after the bias and before the activation (gemm.js:189): through the epilogue's add term with
    an activation, accumulated into the stored output without one; stack: one product over the
    stacked A matrices; rotated: the caller passes only the rotated input, so the rotated A (made
    on the device) is used.  The reference formula for ConvRot layers is B (A H)(x H)^T; the
    unrotated x A^T equals it up to fp32 rounding.  i8: the int8 accumulators and the W8A8
    epilogue are the oracle's; the only difference is the fp32 delta, so the result is within 1e-6
    of the oracle epilogue fed the float64 delta; bf16: within 1e-6 of float64."""
    M, K, N = 300, 1024, 512
    x = orc.randn(111, M * K).reshape(M, K)
    rng = np.random.default_rng(12)
    ents = [dict(r=8, scale=0.5, off=0, n=N), dict(r=4, scale=2.0, off=128, n=256)]
    for i, e in enumerate(ents):
        e["A"] = (0.05 * orc.randn(112 + i, e["r"] * K)).reshape(e["r"], K).astype(np.float32)
        e["B"] = (0.05 * orc.randn(114 + i, e["n"] * e["r"])).reshape(e["n"], e["r"]).astype(np.float32)
    W = {"kind": kind, "N": N, "K": K}
    if kind == "i8":
        qw = np.clip(np.rint(40 * orc.randn(116, N * K)), -127, 127).astype(np.int8).reshape(N, K)
        sw = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
        W.update(w=write(tmp_path, "w.bin", qw), scale=write(tmp_path, "sw.bin", sw))
    else:
        w32 = orc.bf16_round(0.05 * orc.randn(117, N * K)).reshape(N, K)
        W["w"] = write(tmp_path, "w.bin", (w32.view(np.uint32) >> 16).astype(np.uint16))
    spec_l = [dict(A=write(tmp_path, f"a{i}.bin", e["A"]), B=write(tmp_path, f"b{i}.bin", e["B"]), r=e["r"],
                   scale=e["scale"], off=e["off"], n=e["n"]) for i, e in enumerate(ents)]
    out = str(tmp_path / "y.bin")
    run_case(tmp_path, {"case": "lora", "M": M, "W": W, "x": write(tmp_path, "x.bin", x), "lora": spec_l, "out": out,
                        "act": act, "stack": stack, "rotated": rotated})
    got, base = read(out).reshape(M, N), read(out + ".base").reshape(M, N)
    actid = {"none": 0, "gelu": 1}[act]
    if kind == "i8":
        xr = orc.hadamard256(x)
        delta = lora_delta(xr, [dict(e, A=orc.hadamard256(e["A"])) for e in ents], N)
        qx, sx = orc.token_quant(xr)
        acc = orc.gemm_i8(qx, qw)
        base_ref = orc.linear_epilogue(acc, sx, sw, act=actid)
        if act == "none":
            assert np.array_equal(base, base_ref)
        else:  # GELU on the hardware reciprocal / exponential: ~2e-8 relative
            assert report("i8 gelu base", base, base_ref)[0] < 1e-6
        ref = orc.linear_epilogue(acc, sx, sw, act=actid, add=delta.astype(np.float32))
    else:
        delta = lora_delta(x, ents, N)
        ref = x.astype(np.float64) @ w32.astype(np.float64).T + delta
        if act == "gelu":
            ref = np.vectorize(orc.gelu)(ref)
    r, _ = report(f"{kind} {act} linear + LoRA", got, ref)
    assert r < 1e-6
    if act == "none":
        assert report(f"{kind} LoRA delta alone", got.astype(np.float64) - base, delta)[0] < 1e-4


@pytest.mark.parametrize("act", ["none", "gelu"])
def test_js_linear_lora_int8_rows(tmp_path, act):
    """A quantized linear whose LoRA A product reads the int8 rows its GEMM reads (the default LoRA
    input): y = epilogue(acc, s_x, s_w) + B (A H)(s_x q)^T, within 1e-6 of the oracle epilogue fed
    that delta in float64 (q, s_x: the oracle's token_quant of the rotated x, which the GPU's rows
    equal bit for bit).  With setLoraInput("fp32") the same linear takes the fp32 rotated rows, the
    reference's LoRA input, within 1e-6 of that float64 delta; the two deltas differ by the int8
    rounding of the LoRA input only (rel-L2 <= 1e-2)."""
    M, K, N = 300, 1024, 512
    x = orc.randn(141, M * K).reshape(M, K)
    rng = np.random.default_rng(142)
    ents = [dict(r=8, scale=0.5, off=0, n=N), dict(r=4, scale=2.0, off=128, n=256)]
    for i, e in enumerate(ents):
        e["A"] = (0.05 * orc.randn(143 + i, e["r"] * K)).reshape(e["r"], K).astype(np.float32)
        e["B"] = (0.05 * orc.randn(145 + i, e["n"] * e["r"])).reshape(e["n"], e["r"]).astype(np.float32)
    qw = np.clip(np.rint(40 * orc.randn(147, N * K)), -127, 127).astype(np.int8).reshape(N, K)
    sw = (rng.uniform(0.5, 1.5, N) / (127 * np.sqrt(K))).astype(np.float32)
    W = {"kind": "i8", "N": N, "K": K, "w": write(tmp_path, "w.bin", qw), "scale": write(tmp_path, "sw.bin", sw)}
    spec_l = [dict(A=write(tmp_path, f"a{i}.bin", e["A"]), B=write(tmp_path, f"b{i}.bin", e["B"]), r=e["r"],
                   scale=e["scale"], off=e["off"], n=e["n"]) for i, e in enumerate(ents)]
    out = str(tmp_path / "y.bin")
    run_case(tmp_path, {"case": "loraq", "M": M, "W": W, "x": write(tmp_path, "x.bin", x), "lora": spec_l,
                        "out": out, "act": act})
    xr = orc.hadamard256(x)
    qx, sx = orc.token_quant(xr)
    assert np.array_equal(np.fromfile(out + ".q", np.int8).reshape(M, K), qx)
    assert np.array_equal(read(out + ".s"), sx)
    actid = {"none": 0, "gelu": 1}[act]
    acc = orc.gemm_i8(qx, qw)
    ents_r = [dict(e, A=orc.hadamard256(e["A"])) for e in ents]
    dq = lora_delta(sx.astype(np.float64)[:, None] * qx.astype(np.float64), ents_r, N)
    df = lora_delta(xr, ents_r, N)
    got, got_f = read(out).reshape(M, N), read(out + ".fp32").reshape(M, N)
    ref_q = orc.linear_epilogue(acc, sx, sw, act=actid, add=dq.astype(np.float32))
    ref_f = orc.linear_epilogue(acc, sx, sw, act=actid, add=df.astype(np.float32))
    assert report(f"i8 {act} LoRA on the int8 rows", got, ref_q)[0] < 1e-6
    assert report(f"i8 {act} LoRA on the fp32 rotated rows", got_f, ref_f)[0] < 1e-6
    d_rel = report("LoRA delta: int8 rows vs fp32 rows (float64)", dq, df)[0]
    assert 0 < d_rel < 1e-2
    if act == "none":
        base = read(out + ".base").reshape(M, N)
        assert report("LoRA delta alone, int8 rows", got.astype(np.float64) - base, dq)[0] < 1e-4


def test_js_lora_file(tmp_path):
    """loadLora on a 1-block synthetic DiT from a safetensors file in PEFT and kohya naming: the
    k_proj slice of the stacked qkv and mlp.layer2 (alpha / r scaling) match, a LoKr tensor is
    counted unsupported, a module of a missing block is skipped; A is rotated on the device for
    the int8 layers.  Columns outside the LoRA's slice are bit-identical to the plain linear."""
    from safetensors.numpy import save_file

    M = 64
    rk, rl = 8, 4
    Ak = (0.05 * orc.randn(121, rk * 2048)).reshape(rk, 2048).astype(np.float32)
    Bk = (0.05 * orc.randn(122, 2048 * rk)).reshape(2048, rk).astype(np.float32)
    Al = (0.05 * orc.randn(123, rl * 8192)).reshape(rl, 8192).astype(np.float32)
    Bl = (0.05 * orc.randn(124, 2048 * rl)).reshape(2048, rl).astype(np.float32)
    tensors = {
        "diffusion_model.blocks.0.self_attn.k_proj.lora_A.weight": Ak,
        "diffusion_model.blocks.0.self_attn.k_proj.lora_B.weight": Bk,
        "lora_unet_blocks_0_mlp_layer2.lora_down.weight": Al,
        "lora_unet_blocks_0_mlp_layer2.lora_up.weight": Bl,
        "lora_unet_blocks_0_mlp_layer2.alpha": np.array(2.0, np.float32),
        "diffusion_model.blocks.0.cross_attn.q_proj.lokr_w1": np.zeros((4, 4), np.float32),
        "diffusion_model.blocks.9.mlp.layer1.lora_A.weight": np.zeros((2, 2048), np.float32),
        "diffusion_model.blocks.9.mlp.layer1.lora_B.weight": np.zeros((8192, 2), np.float32),
    }
    path = str(tmp_path / "lora.safetensors")
    save_file(tensors, path)
    x = orc.randn(125, M * 2048).reshape(M, 2048)
    h = orc.randn(126, M * 8192).reshape(M, 8192)
    out = str(tmp_path / "y")
    r = run_case(tmp_path, {"case": "lorafile", "mode": "int8", "lora": path, "strength": 1.5, "M": M,
                            "x": write(tmp_path, "x.bin", x), "h": write(tmp_path, "h.bin", h), "out": out})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"matched"' in ln))
    assert (info["matched"], info["total"], info["unsupported"], info["skipped"]) == (2, 3, 1, 1), info
    assert info["entries"] == [[{"r": rk, "scale": 1.5, "off": 2048, "n": 2048}], [{"r": rl, "scale": 0.75, "off": 0, "n": 2048}]]
    q, qb = read(out + ".qkv").reshape(M, 6144), read(out + ".qkv.base").reshape(M, 6144)
    assert np.array_equal(q[:, :2048], qb[:, :2048]) and np.array_equal(q[:, 4096:], qb[:, 4096:])
    dk = lora_delta(orc.hadamard256(x), [dict(A=orc.hadamard256(Ak), B=Bk, scale=1.5, off=0, n=2048)], 2048)
    assert report("k_proj LoRA delta", q[:, 2048:4096].astype(np.float64) - qb[:, 2048:4096], dk)[0] < 1e-4
    l, lb = read(out + ".l2").reshape(M, 2048), read(out + ".l2.base").reshape(M, 2048)
    dl = lora_delta(orc.hadamard256(h), [dict(A=orc.hadamard256(Al), B=Bl, scale=0.75, off=0, n=2048)], 2048)
    assert report("mlp.layer2 LoRA delta", l.astype(np.float64) - lb, dl)[0] < 1e-4


def test_js_lora_text_encoder(tmp_path):
    """loadLora with text-encoder names (PEFT `text_encoder.` and kohya `lora_te_`, app/lora.js:21,
    89) onto the Qwen3 encoder's registry: layer 1's q_proj and mlp.down_proj (bf16 weights, no
    rotation) get scale * B (A x) within 1e-4 of float64, a DiT-named module finds no target (no
    DiT registry), and the encoding changes once the LoRA is attached."""
    from safetensors.numpy import save_file

    M = 48
    rq, rd = 8, 4
    Aq = (0.05 * orc.randn(141, rq * 1024)).reshape(rq, 1024).astype(np.float32)
    Bq = (0.05 * orc.randn(142, 2048 * rq)).reshape(2048, rq).astype(np.float32)
    Ad = (0.05 * orc.randn(143, rd * 3072)).reshape(rd, 3072).astype(np.float32)
    Bd = (0.05 * orc.randn(144, 1024 * rd)).reshape(1024, rd).astype(np.float32)
    tensors = {
        "text_encoder.model.layers.1.self_attn.q_proj.lora_A.weight": Aq,
        "text_encoder.model.layers.1.self_attn.q_proj.lora_B.weight": Bq,
        "lora_te_model_layers_1_mlp_down_proj.lora_down.weight": Ad,
        "lora_te_model_layers_1_mlp_down_proj.lora_up.weight": Bd,
        "lora_te_model_layers_1_mlp_down_proj.alpha": np.array(2.0, np.float32),
        "diffusion_model.blocks.0.mlp.layer1.lora_A.weight": np.zeros((2, 2048), np.float32),
        "diffusion_model.blocks.0.mlp.layer1.lora_B.weight": np.zeros((8192, 2), np.float32),
    }
    path = str(tmp_path / "lora_te.safetensors")
    save_file(tensors, path)
    x = orc.randn(145, M * 1024).reshape(M, 1024)
    h = orc.randn(146, M * 3072).reshape(M, 3072)
    out = str(tmp_path / "t")
    r = run_case(tmp_path, {"case": "lorate", "lora": path, "strength": 0.8, "M": M,
                            "x": write(tmp_path, "x.bin", x), "h": write(tmp_path, "h.bin", h), "out": out})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"matched"' in ln))
    assert (info["matched"], info["total"], info["unsupported"], info["skipped"]) == (2, 3, 0, 1), info
    assert info["entries"] == [[{"r": rq, "scale": 0.8, "off": 0, "n": 2048}], [{"r": rd, "scale": 0.4, "off": 0, "n": 1024}]]
    q, qb = read(out + ".q").reshape(M, 2048), read(out + ".q.base").reshape(M, 2048)
    dq = lora_delta(x, [dict(A=Aq, B=Bq, scale=0.8, off=0, n=2048)], 2048)
    assert report("text encoder q_proj LoRA delta", q.astype(np.float64) - qb, dq)[0] < 1e-4
    d, db = read(out + ".down").reshape(M, 1024), read(out + ".down.base").reshape(M, 1024)
    dd = lora_delta(h, [dict(A=Ad, B=Bd, scale=0.4, off=0, n=1024)], 1024)
    assert report("text encoder down_proj LoRA delta", d.astype(np.float64) - db, dd)[0] < 1e-4
    e, eb = read(out + ".enc"), read(out + ".enc.base")
    assert np.all(np.isfinite(e)) and np.abs(e - eb).max() > 1e-3 * np.abs(eb).max()


def test_js_lora_modulation(tmp_path):
    """LoRAs on adaLN modulation linears (a first stage, a second stage and the final layer's
    second stage): timeCond on the fused path (one stacked first-stage GEMV + one grouped
    second-stage GEMV, the LoRA products applied per part) equals the per-linear path within fp32
    summation-order noise, and the LoRAs change the outputs they target."""
    from safetensors.numpy import save_file

    r1, r2, rf = 4, 8, 4
    T = {}
    def mod(name, r, n, k, seed):
        T[f"diffusion_model.{name}.lora_A.weight"] = (0.1 * orc.randn(seed, r * k)).reshape(r, k).astype(np.float32)
        T[f"diffusion_model.{name}.lora_B.weight"] = (0.1 * orc.randn(seed + 1, n * r)).reshape(n, r).astype(np.float32)
    mod("blocks.0.adaln_modulation_cross_attn.1", r1, 256, 2048, 131)
    mod("blocks.0.adaln_modulation_mlp.2", r2, 6144, 256, 133)
    mod("final_layer.adaln_modulation.2", rf, 4096, 256, 135)
    path = str(tmp_path / "lora.safetensors")
    save_file(T, path)
    out = str(tmp_path / "m")
    r = run_case(tmp_path, {"case": "loramod", "mode": "int8", "lora": path, "strength": 1.0, "sigma": 0.7, "out": out})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"fused"' in ln))
    assert info["fused"] == info["plain"] == {"matched": 3, "skipped": 0}, info
    fused, plain = read(out + ".fused"), read(out + ".plain")
    fb, pb = read(out + ".fused.base"), read(out + ".plain.base")
    assert report("modulation without LoRA: fused vs per-linear", fb, pb.astype(np.float64))[0] < 1e-6
    assert report("modulation with LoRA: fused vs per-linear", fused, plain.astype(np.float64))[0] < 1e-6
    D = 2048
    segs = {"self": (0, 3 * D), "cross": (3 * D, 6 * D), "mlp": (6 * D, 9 * D), "final": (9 * D, 11 * D)}
    for name, (a, b) in segs.items():
        changed = np.abs(fused[a:b] - fb[a:b]).max()
        if name == "self":
            assert changed == 0, name
        else:
            assert changed > 1e-3 * np.abs(fb[a:b]).max(), (name, changed)


def test_js_forward_graph(tmp_path):
    """ForwardGraph (forwardDevice recorded once into a HIP graph) against eager forwardDevice on
    a 3-block synthetic DiT at 1024x1024, B=2, W4A8 mixed (block 1 W4): every replay, each with a
    new latent, another sigma (timeCond copied into the graph's slot) and an eager forward before
    it, gives the eager velocities bit for bit."""
    out = str(tmp_path / "g")
    r = run_case(tmp_path, {"case": "graph", "mode": "w4a8", "blocks": 3, "size": 1024, "Lk": 64,
                            "sigmas": [0.9, 0.5, 0.1], "out": out})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"graph"' in ln))["graph"]
    assert info["diffs"] == [0, 0, 0], info
    for i in range(3):
        e, g = read(f"{out}.eager{i}"), read(f"{out}.graph{i}")
        assert np.array_equal(e, g) and np.isfinite(e).all() and np.abs(e).max() > 0
    assert not np.array_equal(read(f"{out}.eager0"), read(f"{out}.eager1"))


def test_js_qwen3_text_encoder(tmp_path):
    """Qwen3.encode (js/qwen3.mjs, the reference's qwen3.js forward on this build's ops: causal GQA
    attention on the flash kernels, bf16 linears on the split-bf16 matrix-core kernel, RMSNorm, 1D
    RoPE, SiLU * up) on a seeded 2-layer synthetic encoder against the oracle's float64 restatement
    fed the same weights: fp32 attention within 1e-5 relative L2, bf16 attention within 1e-2.  The
    encodings come from the recorded HIP graph; its first call, a second replay and the eager pass
    are bit-identical."""
    from oracle import qwen3_ref

    out = str(tmp_path / "te")
    ids = [int(x) for x in np.random.default_rng(5).integers(0, 97, size=37)]
    run_case(tmp_path, {"case": "qwen3", "layers": 2, "vocab": 97, "ids": ids, "out": out})
    D, H, KH, Dh, F = 1024, 16, 8, 128, 3072
    shapes = {"q": (H * Dh, D), "k": (KH * Dh, D), "v": (KH * Dh, D), "o": (D, H * Dh), "gate": (F, D), "up": (F, D),
              "down": (D, F)}
    W = {"norm": read(f"{out}.w.norm").astype(np.float64), "embed": read(f"{out}.w.embed").reshape(97, D).astype(np.float64)}
    for i in range(2):
        for n in ("ln1", "ln2", "qn", "kn"):
            W[f"{i}.{n}"] = read(f"{out}.w.{i}.{n}").astype(np.float64)
        for n, shp in shapes.items():
            bits = read(f"{out}.w.{i}.{n}", np.uint16).astype(np.uint32) << 16
            W[f"{i}.{n}"] = bits.view(np.float32).reshape(shp).astype(np.float64)
    ref = qwen3_ref.encode(W, ids, 2)
    got32, got16 = read(f"{out}.fp32").reshape(len(ids), D), read(f"{out}.bf16").reshape(len(ids), D)
    assert np.isfinite(got32).all() and np.isfinite(got16).all()
    assert report("qwen3 fp32 attention vs float64", got32, ref)[0] <= 1e-5
    assert report("qwen3 bf16 attention vs float64", got16, ref)[0] <= 1e-2
    for prec in ("fp32", "bf16"):
        g = read(f"{out}.{prec}")
        assert np.array_equal(g, read(f"{out}.{prec}.replay")), f"{prec}: graph replay differs"
        assert np.array_equal(g, read(f"{out}.{prec}.eager")), f"{prec}: graph vs eager"


def test_js_llm_adapter(tmp_path):
    """The LLM adapter (js/dit.mjs adapt: self- and cross-attention with 16 x 64 heads on the
    padded D = 64 path, q/k RMSNorm, 1D RoPE, biased GELU MLP, out_proj, norm, prompt weights,
    zero rows to 512) on a seeded 2-block synthetic adapter against the oracle's float64
    restatement fed the same weights and text-encoder states."""
    from oracle import adapter_ref

    out = str(tmp_path / "ad")
    rng = np.random.default_rng(7)
    ids = [int(x) for x in rng.integers(0, 64, size=19)]
    weights = [float(x) for x in rng.uniform(0.5, 1.5, size=19)]
    run_case(tmp_path, {"case": "adapter", "blocks": 2, "vocab": 64, "Ls": 23, "ids": ids, "weights": weights, "out": out})
    D, F = 1024, 4096
    f64 = lambda name, shp=None: read(f"{out}.w.{name}").astype(np.float64).reshape(shp if shp else -1)

    def bf(name, shp):
        return (read(f"{out}.w.{name}", np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(shp).astype(np.float64)

    W = {"embed": f64("embed", (64, D)), "norm": f64("norm"), "out": bf("out", (D, D)), "out.bias": f64("out.bias")}
    for i in range(2):
        for n in ("nSelf", "nCross", "nMlp"):
            W[f"{i}.{n}"] = f64(f"{i}.{n}")
        for a in ("self", "cross"):
            for n in ("q", "k", "v", "o"):
                W[f"{i}.{a}.{n}"] = bf(f"{i}.{a}.{n}", (D, D))
            for n in ("qn", "kn"):
                W[f"{i}.{a}.{n}"] = f64(f"{i}.{a}.{n}")
        W[f"{i}.mlp0"], W[f"{i}.mlp2"] = bf(f"{i}.mlp0", (F, D)), bf(f"{i}.mlp2", (D, F))
        W[f"{i}.mlp0.bias"], W[f"{i}.mlp2.bias"] = f64(f"{i}.mlp0.bias"), f64(f"{i}.mlp2.bias")
    hidden = read(f"{out}.hidden").reshape(23, D).astype(np.float64)
    ref = adapter_ref.adapt(W, hidden, ids, weights, 2)
    for prec, tol in (("fp32", 1e-5), ("bf16", 1e-2)):
        got = read(f"{out}.{prec}").reshape(512, D)
        assert np.all(got[19:] == 0)
        assert report(f"adapter {prec} attention vs float64", got[:19], ref[:19])[0] <= tol


def test_js_prompt_to_velocity_chain(tmp_path):
    """The conditioning chain on the device path: prompt token ids -> Qwen3.encode -> the LLM
    adapter -> prepareContext -> one DiT forward (synthetic 2-layer encoder, 2-block adapter,
    1-block int8 DiT at 64x64, cond + uncond prompts of different lengths): finite velocities,
    different for the two prompts.  Each stage's parity is checked by its own test."""
    out = str(tmp_path / "ch")
    prompts = [{"qwen": [3, 17, 5, 88, 41, 9, 60], "t5": [1, 5, 9, 33, 2], "weights": [1, 1, 1.2, 1, 0.8]},
               {"qwen": [7, 7, 21], "t5": [4, 2], "weights": [1, 1]}]
    run_case(tmp_path, {"case": "chain", "prompts": prompts, "size": 64, "out": out})
    v0, v1 = read(f"{out}.0"), read(f"{out}.1")
    assert v0.size == 16 * 8 * 8 and np.isfinite(v0).all() and np.isfinite(v1).all()
    assert np.abs(v0).max() > 0 and not np.array_equal(v0, v1)


def test_js_pipeline_encode_cache(tmp_path):
    """LatentPipeline.encode (app/pipeline.js:192-211): token ids -> Qwen3 -> the LLM adapter ->
    prepareContext, cached per prompt.  A repeated prompt (equal ids, new arrays) returns the
    cached conditioning without encoding again; the cached conditionings of two prompts, stacked,
    give bit-identical velocities to prepareContext over both contexts at once; a new prompt with
    the default keep list evicts the others."""
    prompts = [{"qwen": [3, 17, 5, 88, 41, 9, 60], "t5": [1, 5, 9, 33, 2], "weights": [1, 1, 1.2, 1, 0.8]},
               {"qwen": [7, 7, 21], "t5": [4, 2], "weights": [1, 1]},
               {"qwen": [11, 2], "t5": [8], "weights": [1]}]
    r = run_case(tmp_path, {"case": "encode", "prompts": prompts, "size": 64})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"encode"' in ln))["encode"]
    print(f"encode cache: {info}", flush=True)
    assert info["reused"]
    assert info["stats1"]["encodeMisses"] == 2 and info["stats1"]["encodeHits"] == 1
    assert info["diffs"] == 0 and info["n"] == 16 * 8 * 8 and info["finite"]
    assert info["after"] == {"size": 1, "hasP0": False}
