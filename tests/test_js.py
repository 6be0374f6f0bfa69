"""CPU checks of the JavaScript host: Node parses every module, the N-API addon loads and
exports the op surface, and errors from the C ABI surface as JS exceptions."""

import json
import os
import shutil
import subprocess

import pytest

from helpers import PKG_DIR

JS = os.path.join(PKG_DIR, "js")
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def node(code):
    return subprocess.run([NODE, "--input-type=module", "-e", code], cwd=JS, capture_output=True, text=True, timeout=60)


def test_modules_import():
    r = node("import * as ops from './ops.mjs'; import { AnimaDiT } from './dit.mjs'; "
             "import { SafeTensors, concatLinears, SyntheticWeights } from './weights.mjs'; "
             "import * as c from './common.mjs'; console.log(JSON.stringify(Object.keys(ops)))")
    assert r.returncode == 0, r.stderr
    names = json.loads(r.stdout)
    # the op surface of the reference's app/gpu/ops.js
    for n in ("linear", "rotate", "needsRotation", "attention", "qkNormRope", "rmsnorm", "rope", "layernormMod",
              "elementwise", "zero"):
        assert n in names, n


def test_addon_exports_and_error_path():
    r = node("import { native } from './gpu.mjs'; const ks = Object.keys(native); "
             "let msg = ''; try { native.init(0) } catch (e) { msg = e.message } "
             "console.log(JSON.stringify({ ks, msg }))")
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    for k in ("init", "attention", "linear", "layernormMod", "qkNormRope", "h2d", "d2h", "alloc", "free", "mark", "waitMark"):
        assert k in out["ks"], k
    if out["msg"]:  # no GPU here: the C ABI status becomes a JS Error with the library's message
        assert "anima error" in out["msg"]


def test_rope_angles_match_oracle():
    import numpy as np

    import oracle as orc

    r = node("import { ditRopeAngles } from './common.mjs'; console.log(JSON.stringify(Array.from(ditRopeAngles(5, 7))))")
    assert r.returncode == 0, r.stderr
    got = np.array(json.loads(r.stdout), np.float32)
    assert np.array_equal(got, orc.dit_rope_angles(5, 7).reshape(-1))


def test_patchify_roundtrip():
    # patchify packs (c m n) + a zero mask channel (dit.js:55-65); unpatchify reads (p1 p2 c)
    # (dit.js:68-78): re-packing each token's 64 values from (c m n) to (m n c) makes them inverse.
    r = node("import { patchify, unpatchify } from './common.mjs'; const h = 8, w = 12, T = (h / 2) * (w / 2); "
             "const lat = new Float32Array(16 * h * w).map((_, i) => i * 0.5); "
             "const p = patchify(lat, h, w); const q = new Float32Array(T * 64); let mask = 0; "
             "for (let t = 0; t < T; t++) { for (let c = 0; c < 16; c++) for (let m = 0; m < 2; m++) for (let n = 0; n < 2; n++) "
             "q[t * 64 + m * 32 + n * 16 + c] = p[t * 68 + c * 4 + m * 2 + n]; for (let k = 64; k < 68; k++) mask += Math.abs(p[t * 68 + k]); } "
             "const back = unpatchify(q, h, w); "
             "console.log(back.every((v, i) => v === lat[i]) && mask === 0 ? 'ok' : 'bad')")
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr + r.stdout


def test_non_finite_numbers_raise_range_error():
    # a NaN or infinity reaching the C ABI would be cast to an integer (undefined behaviour in C): the
    # addon raises a RangeError instead and makes no call; a later valid call is unaffected
    r = node("import { native } from './gpu.mjs'; const out = {}; "
             "for (const [k, f] of [['nan', () => native.attentionKvBytes(NaN, 16, 512, 0)], "
             "['inf', () => native.attentionKvBytes(2, 16, Infinity, 0)], "
             "['ok', () => native.attentionKvBytes(2, 16, 512, 0)]]) { "
             "try { out[k] = f(); } catch (e) { out[k] = e.name + ': ' + e.message; } } "
             "console.log(JSON.stringify(out))")
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    assert out["nan"].startswith("RangeError") and out["inf"].startswith("RangeError")
    assert out["ok"] == 2 * 2 * 16 * 512 * 128 * 2


def test_attention_precision_default_is_fp32():
    # ops.attention keeps the reference's fp32 arithmetic unless the caller asks for bf16; an unknown
    # precision is rejected before any device work
    r = node("import * as ops from './ops.mjs'; let msg = ''; "
             "try { ops.attention({ ctx: null, empty: () => ({ buf: 0 }) }, { q: { buf: 0 }, Lq: 1, Lk: 1, H: 1, D: 128, "
             "ldq: 128, precision: 'fp16' }); } catch (e) { msg = e.message; } console.log(JSON.stringify({ msg }))")
    assert r.returncode == 0, r.stderr
    assert "unknown precision fp16" in json.loads(r.stdout)["msg"]
