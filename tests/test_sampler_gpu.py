"""GPU parity of the sampling loop: anima_sampler_step (CFG combine + denoised + sampler update,
app/pipeline.js:276-283 and app/samplers.js:104-218) against the oracle through the C ABI, bit
for bit; and the device loop of js/pipeline.mjs against the reference's host loop on a synthetic
DiT, bit for bit."""

import json
import shutil

import numpy as np
import pytest

import oracle as orc
from oracle import samplers as so
from helpers import amd
from test_js_gpu import read, run_case

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)

SAMPLERS = ["euler", "euler_a", "dpmpp_2m", "er_sde"]


@pytest.fixture(scope="module")
def ctx():
    m = amd()
    c = m.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("name", SAMPLERS)
@pytest.mark.parametrize("guided", [True, False])
def test_sampler_step_matches_oracle(ctx, name, guided):
    """Every step of a 9-step schedule (first, middle, final; DPM++ and ER-SDE history buffers,
    noise where the sampler draws it), n ragged: x, den, old and old_d bit-exact."""
    case(f"sampler step {name} guided={guided}")
    n = 16 * 9 * 7 + 3
    sig = so.simple_sigmas(9, 3.0)
    steps = so.plan(name, sig, 3.0)
    x = orc.randn(21, n)
    dx, dden = ctx.upload(x), ctx.empty((n,))
    dold, doldd = ctx.upload(np.zeros(n, np.float32)), ctx.upload(np.zeros(n, np.float32))
    state = {}
    gen = so.TorchRandnStream(5)
    cfg = 4.5 if guided else 1.0
    for i, st in enumerate(steps):
        vc = orc.randn(200 + i, n)
        vu = orc.randn(300 + i, n) if guided else None
        eps = gen.randn(n) if st["noise"] else None
        den = so.cfg_denoised(x, vc, vu, cfg, st["sigma"])
        x = so.apply(st, x, den, state, eps)
        uses_old = st["kind"] >= 2
        ctx.sampler_step(name, n, dx, ctx.upload(vc), v_uncond=ctx.upload(vu) if guided else None, cfg=cfg,
                         sigma=st["sigma"], final_step=st["final"], stage=st["stage"], den_out=dden,
                         old=dold if uses_old else None, old_d=doldd if name == "er_sde" else None,
                         eps=ctx.upload(eps) if eps is not None else None, c=st["c"])
        ctx.sync()
        assert np.array_equal(dden.numpy(), den), (name, i, "den")
        assert np.array_equal(dx.numpy(), x), (name, i, "x")
        if uses_old:
            assert np.array_equal(dold.numpy(), state["old"]), (name, i, "old")
        if name == "er_sde" and st["stage"] >= 2 and not st["final"]:
            assert np.array_equal(doldd.numpy(), state["old_d"]), (name, i, "old_d")
    assert np.isfinite(x).all()


def test_sampler_step_rejects_bad_arguments(ctx):
    m = amd()
    n = 64
    x, v = ctx.empty((n,)), ctx.empty((n,))
    with pytest.raises(m.AnimaError):
        ctx.sampler_step(7, n, x, v, sigma=0.5)
    with pytest.raises(m.AnimaError):
        ctx.sampler_step("euler_a", n, x, v, sigma=0.5, c=(0.5, 0.5, 1.0, 0.1))  # no eps
    with pytest.raises(m.AnimaError):
        ctx.sampler_step("dpmpp_2m", n, x, v, sigma=0.5, stage=1)  # no old
    with pytest.raises(m.AnimaError):
        ctx.sampler_step("er_sde", n, x, v, sigma=0.5, stage=4)
    with pytest.raises(m.AnimaError):
        ctx.sampler_step("euler", n, None, v, sigma=0.5)


@pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")
def test_js_generate_device_equals_host(tmp_path):
    """LatentPipeline.generate (velocities stay on the device; one fused kernel per step) against
    generateHost (velocities read back; CFG, denoised and the update over Float32Arrays, as
    app/pipeline.js and app/samplers.js do) on a 1-block synthetic DiT at 64x64: identical
    latents for every sampler, with and without CFG, both schedulers, also with the device loop's
    forwards replayed from a HIP graph.  The host run reuses the device run's timeCond results
    from the cache."""
    case("js generate: device loop vs host loop")
    runs = []
    for nm in SAMPLERS:
        runs.append(dict(key=f"{nm}_cfg", sampler=nm, scheduler="simple", steps=6, cfg=4.0, seed=11))
    runs.append(dict(key="euler_a_nocfg", sampler="euler_a", scheduler="beta", steps=8, cfg=1, seed=3))
    runs.append(dict(key="er_sde_beta", sampler="er_sde", scheduler="beta", steps=7, cfg=2.5, seed=4))
    # steps 1.. replayed from the forward recorded into a HIP graph
    runs.append(dict(key="dpmpp_2m_graph", sampler="dpmpp_2m", scheduler="simple", steps=6, cfg=4.0, seed=12, graph=True))
    runs.append(dict(key="euler_a_nocfg_graph", sampler="euler_a", scheduler="beta", steps=5, cfg=1, seed=13, graph=True))
    out = str(tmp_path / "g")
    r = run_case(tmp_path, {"case": "generate", "mode": "int8", "size": 64, "Lk": 8, "runs": runs, "out": out})
    info = json.loads(next(ln for ln in r.stdout.splitlines() if '"runs"' in ln))
    for run in runs:
        dev, host = read(f"{out}.{run['key']}.dev"), read(f"{out}.{run['key']}.host")
        assert dev.size == 16 * 8 * 8 and np.isfinite(dev).all()
        assert np.array_equal(dev, host), run["key"]
        assert np.abs(dev).max() > 0
    # each step's sigma is computed once per distinct (sigma, LoRA set) and reused by the host run
    assert info["stats"]["timeCondHits"] >= sum(v["steps"] for v in info["runs"].values())
