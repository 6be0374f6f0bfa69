"""GPU parity of the JavaScript host path (ops.mjs -> N-API addon -> libanima.so) against the
oracle: the same bars as the direct C-ABI tests, through the reference's op signatures."""

import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from helpers import PKG_DIR, report

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]

JS = os.path.join(PKG_DIR, "js")
HD = 128


def run_case(tmp_path, spec):
    path = tmp_path / "case.json"
    path.write_text(json.dumps(spec))
    print(f"[case] js {spec['case']}", flush=True)
    r = subprocess.run(["node", os.path.join(JS, "run_case.mjs"), str(path)], capture_output=True, text=True, timeout=300)
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
