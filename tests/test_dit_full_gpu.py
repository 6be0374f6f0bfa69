"""The full-depth DiT step (28 blocks, W4A8 "mixed": int8 first / last block, W4 between;
tools/build_assets.py:119) through the JavaScript host (js/dit.mjs -> N-API -> libanima.so):

  * at 256x256 (256 tokens, B=2 CFG, 512 context tokens) against the oracle's restatement of the
    same seeded weights (oracle/synthetic.py + oracle/dit_ref.py), at the reference's bar rel L2 <=
    5e-3 (tools/check.js:103, 109), for the velocities and the residual stream after block 0;
  * at its real size, 1024x1024 (4096 tokens, B=2, 512 context tokens): finite velocities, the cond
    and uncond halves different, bit-identical halves when both prompts are the same (batch
    elements do not mix), and the HIP-graph replay bit-identical to the eager step;
  * the seeded weight fill itself, bit-exact against the oracle's restatement (every kind).
"""

import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from helpers import RUN_CASE, amd, rel_l2, report

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")]


def run_case(tmp_path, spec, timeout=600):
    path = tmp_path / "case.json"
    path.write_text(json.dumps(spec))
    print(f"[case] js {spec['case']} {json.dumps({k: v for k, v in spec.items() if k in ('blocks', 'size', 'h', 'Lk')})}",
          flush=True)
    r = subprocess.run(["node", RUN_CASE, str(path)], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-3000:]
    return r


def test_fill_random_matches_oracle():
    m = amd()
    with m.Context() as ctx:
        n = 100003
        for kind, lo, hi, dt in (("u8", 0x60, 0x6F, np.uint8), ("u8", 0, 255, np.uint8), ("i8n", 40, 0, np.int8),
                                 ("f32", -0.3, 0.7, np.float32), ("f32", -0.05, 0.05, np.float32),
                                 ("bf16", -0.05, 0.05, np.uint16),
                                 ("f32n", 1.5, 0.25, np.float32)):
            print(f"[case] fill {kind} [{lo}, {hi}]", flush=True)
            d = ctx.empty(n, dt)
            ctx.fill_random(d, n, kind, 123456789, lo, hi)
            got = d.numpy()
            d.release()
            ref = orc.fill_random(n, kind, 123456789, lo, hi)
            assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), kind


@pytest.mark.timeout(600)
def test_dit_28_blocks_matches_oracle(tmp_path):
    from oracle import dit_ref, synthetic

    nblocks, h, w, Lk, sigma, seed = 28, 32, 32, 512, 0.9, 5
    lat = [orc.randn(201 + b, 16 * h * w).reshape(16, h, w) for b in range(2)]
    ctx = [orc.randn(211 + b, Lk * 1024).reshape(Lk, 1024) for b in range(2)]
    files = {}
    for b in range(2):
        files[f"lat{b}"] = str(tmp_path / f"lat{b}.bin")
        lat[b].tofile(files[f"lat{b}"])
        files[f"ctx{b}"] = str(tmp_path / f"ctx{b}.bin")
        ctx[b].tofile(files[f"ctx{b}"])
    out = str(tmp_path / "v")
    run_case(tmp_path, {"case": "synthdit", "seed": seed, "mode": "w4a8", "blocks": nblocks, "sigma": sigma, "Lk": Lk,
                        "h": h, "w": w, "ctx": [files["ctx0"], files["ctx1"]],
                        "latents": [files["lat0"], files["lat1"]], "out": out})
    got = np.stack([np.fromfile(out + f".{b}", np.float32).reshape(16, h, w) for b in range(2)])
    got_b0 = np.fromfile(out + ".block0", np.float32)
    print("[case] oracle: 28-block W8A8 step on the restated weights", flush=True)
    W = synthetic.dit_weights(seed, "w4a8", nblocks)
    ref, ref_b0 = dit_ref.dit_step(W, nblocks, lat, h, w, ctx, sigma, mode="w8a8")
    assert np.all(np.isfinite(got))
    rb0, _ = report("28-block dit_block0 vs W8A8 oracle", got_b0, ref_b0.reshape(-1))
    rv, _ = report("28-block velocity vs W8A8 oracle", got, np.stack(ref))
    assert rb0 < 5e-3 and rv < 5e-3


@pytest.mark.timeout(600)
def test_dit_full_size_step(tmp_path):
    out = str(tmp_path / "v")
    r = run_case(tmp_path, {"case": "fullstep", "seed": 9, "mode": "w4a8", "blocks": 28, "size": 1024, "Lk": 512,
                            "sigma": 0.9, "out": out})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"fullstep"' in ln))["fullstep"]
    n = info["n"]
    print(f"full 28-block step 1024x1024 B=2 (eager, first call): {info['ms']:.2f} ms", flush=True)
    e = np.fromfile(out + ".eager", np.float32)
    same = np.fromfile(out + ".same", np.float32)
    g = np.fromfile(out + ".graph", np.float32)
    assert e.size == 2 * n and np.all(np.isfinite(e))
    d = rel_l2(e[:n], e[n:])
    print(f"cond vs uncond velocity: rel L2 {d:.3e}", flush=True)
    assert d > 1e-3
    # the cond half does not depend on the other batch element: equal to the run with both prompts
    # the same, and the two halves of that run equal each other
    assert np.array_equal(same[:n], same[n:])
    assert np.array_equal(same[:n], e[:n])
    assert np.array_equal(g, e)


@pytest.mark.timeout(600)
def test_dit_w4_unpacked_at_load_is_bit_identical(tmp_path):
    """AnimaDiT.unpackW4 (W4 block linears converted to their int8 grids at load) gives the same
    velocity, bit for bit, as the in-GEMM nibble unpack: a 4-block W4A8-mixed step at 256x256."""
    nblocks, h, w, Lk, sigma, seed = 4, 32, 32, 64, 0.7, 11
    files = {}
    for b in range(2):
        files[f"lat{b}"] = str(tmp_path / f"lat{b}.bin")
        orc.randn(301 + b, 16 * h * w).tofile(files[f"lat{b}"])
        files[f"ctx{b}"] = str(tmp_path / f"ctx{b}.bin")
        orc.randn(311 + b, Lk * 1024).tofile(files[f"ctx{b}"])
    outs = []
    for unpack in (False, True):
        out = str(tmp_path / f"v{int(unpack)}")
        r = run_case(tmp_path, {"case": "synthdit", "seed": seed, "mode": "w4a8", "blocks": nblocks, "sigma": sigma,
                                "Lk": Lk, "h": h, "w": w, "ctx": [files["ctx0"], files["ctx1"]],
                                "latents": [files["lat0"], files["lat1"]], "out": out, "unpackW4": unpack})
        if unpack:
            info = json.loads(next(ln for ln in r.stdout.splitlines() if '"unpacked"' in ln))
            # blocks 1 and 2 are W4 (0 and 3 int8): stacked qkv, self out, cross q / k / v / out, mlp 1 / 2
            assert info["unpacked"] == 2 * 8
        outs.append(np.concatenate([np.fromfile(out + f".{b}", np.float32) for b in range(2)]))
    assert np.all(np.isfinite(outs[0])) and np.array_equal(outs[0], outs[1])


@pytest.mark.timeout(600)
def test_dit_lora_int8_rows(tmp_path):
    """Seeded rank-16 LoRAs on every block linear of a 3-block W4A8 synthetic DiT (256x256, B=2):
    the forward with the LoRA A products on the int8 rows that the quantized linears read (the
    default) against the same forward with them on the fp32 rotated rows (the reference's LoRA
    input).  The LoRAs move the velocity (rel L2 > 1e-3 from the forward without them), and the two
    LoRA inputs differ by the int8 rounding of the LoRA input only: below 5% of that move."""
    h = w = 32
    Lk = 64
    files = {}
    for b in range(2):
        files[f"lat{b}"] = str(tmp_path / f"lat{b}.bin")
        orc.randn(221 + b, 16 * h * w).tofile(files[f"lat{b}"])
        files[f"ctx{b}"] = str(tmp_path / f"ctx{b}.bin")
        orc.randn(231 + b, Lk * 1024).tofile(files[f"ctx{b}"])
    out = str(tmp_path / "v")
    r = run_case(tmp_path, {"case": "loradit", "seed": 11, "mode": "w4a8", "blocks": 3, "sigma": 0.7, "Lk": Lk,
                            "h": h, "w": w, "rank": 16, "ctx": [files["ctx0"], files["ctx1"]],
                            "latents": [files["lat0"], files["lat1"]], "out": out})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"loradit"' in ln))["loradit"]
    assert info["int8"] > 0 and info["modules"] > 0, info
    v = {k: np.concatenate([np.fromfile(f"{out}.{k}.{b}", np.float32) for b in range(2)]) for k in ("base", "int8", "fp32")}
    assert all(np.all(np.isfinite(a)) for a in v.values())
    move = rel_l2(v["fp32"], v["base"])
    diff = rel_l2(v["int8"], v["fp32"])
    print(f"LoRA move rel L2 {move:.3e}; int8 vs fp32 LoRA input rel L2 {diff:.3e} ({diff / move:.3f} of the move)",
          flush=True)
    assert move > 1e-3 and 0 < diff < 0.05 * move
