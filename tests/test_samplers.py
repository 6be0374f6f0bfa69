"""CPU checks of the sampling loop (app/samplers.js, app/pipeline.js:225-293, app/rng.js).

The oracle (oracle/samplers.py) is pinned here by what the mathematics fixes: the schedules by
their closed form and, for the beta schedule, by scipy's inverse regularized incomplete beta; the
noise stream by torch's own CPU generator; the step coefficients by the identities the samplers
are built on (Euler's affine weights, the ancestral and ER-SDE steps preserving the marginal
variance, DPM++ 2M's second-order combination preserving constants, the ER-SDE integrals against
adaptive quadrature); whole runs by closed-form trajectories of a constant denoiser.  The
JavaScript host (js/samplers.mjs, js/rng.mjs) is then compared with the oracle bit for bit.
"""

import json
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from oracle import samplers as so
from helpers import PKG_DIR

JS = os.path.join(PKG_DIR, "js")
NODE = shutil.which("node")
SAMPLERS = ["euler", "euler_a", "dpmpp_2m", "er_sde"]


def node(code):
    r = subprocess.run([NODE, "--input-type=module", "-e", code], cwd=JS, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


# ------------------------------------------------------------------ schedules

@pytest.mark.parametrize("shift", [1.0, 3.0, 6.5])
@pytest.mark.parametrize("steps", [1, 4, 8, 30, 1000])
def test_simple_schedule_closed_form(steps, shift):
    sig = so.simple_sigmas(steps, shift)
    assert len(sig) == steps + 1 and sig[-1] == 0.0 and sig[0] == 1.0  # t = 1 maps to 1 at any shift
    for k in range(steps):
        t = (1000 - math.floor(k * 1000 / steps)) / 1000
        assert sig[k] == float(np.float32(shift * t / (1 + (shift - 1) * t))), k
        if shift == 1.0:
            assert sig[k] == float(np.float32(t))
    assert all(a > b for a, b in zip(sig, sig[1:]))


@pytest.mark.parametrize("steps", [4, 8, 20, 30, 50])
def test_beta_schedule_against_scipy(steps):
    """The restated incomplete-beta inverse (Lanczos ln-gamma, Lentz continued fraction,
    bisection) gives the same table indices as scipy.stats.beta.ppf."""
    from scipy.stats import beta as sbeta

    ours = so.beta_sigmas(steps, 3.0)
    lib = so.beta_sigmas(steps, 3.0, ppf=lambda p, a, b: float(sbeta.ppf(p, a, b)))
    assert ours == lib
    for p in (0.01, 0.3, 0.5, 0.77, 0.999):
        assert abs(so.beta_ppf(p, 0.6, 0.6) - sbeta.ppf(p, 0.6, 0.6)) < 1e-12
        assert abs(so.beta_cdf(p, 0.6, 0.6) - sbeta.cdf(p, 0.6, 0.6)) < 1e-12
    assert ours[-1] == 0.0 and all(a > b for a, b in zip(ours, ours[1:]))


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_js_schedules_equal_oracle():
    got = node("import { simpleSigmas, betaSigmas } from './samplers.mjs'; "
               "const o = {}; for (const s of [1, 4, 8, 30]) { o['simple' + s] = simpleSigmas(s, 3); "
               "o['beta' + s] = betaSigmas(s, 3); } o.shift = simpleSigmas(12, 6.5); console.log(JSON.stringify(o))")
    for s in (1, 4, 8, 30):
        assert got[f"simple{s}"] == so.simple_sigmas(s, 3.0)
        assert got[f"beta{s}"] == so.beta_sigmas(s, 3.0)
    assert got["shift"] == so.simple_sigmas(12, 6.5)


# ------------------------------------------------------------------ noise stream

def test_noise_stream_against_torch():
    """torch.manual_seed(seed); torch.randn(n) twice on one generator: the stream continues
    across calls (the sampler's ancestral noise), ragged n redraws its tail."""
    import torch

    for seed, sizes in ((0, [64, 64]), (1234, [1000, 37, 256]), (2 ** 32 + 5, [48])):
        st = so.TorchRandnStream(seed)
        g = torch.Generator().manual_seed(seed % 2 ** 64)
        for n in sizes:
            ours = st.randn(n)
            ref = torch.randn(n, generator=g, dtype=torch.float32).numpy()
            assert np.abs(ours - ref).max() < 4e-6 * max(1.0, np.abs(ref).max()), (seed, n)
    assert np.array_equal(so.TorchRandnStream(7).randn(1000), orc.randn(7, 1000))


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_js_noise_equals_oracle():
    got = node("import { TorchGenerator } from './rng.mjs'; const g = new TorchGenerator(42); "
               "const a = Array.from(g.randn(1000)), b = Array.from(g.randn(37)); "
               "console.log(JSON.stringify({ a, b, c: Array.from(new TorchGenerator(2 ** 33 + 3).randn(64)) }))")
    st = so.TorchRandnStream(42)
    assert np.array_equal(np.array(got["a"], np.float32), st.randn(1000))
    assert np.array_equal(np.array(got["b"], np.float32), st.randn(37))
    assert np.array_equal(np.array(got["c"], np.float32), so.TorchRandnStream((2 ** 33 + 3) % 2 ** 32).randn(64))


# ------------------------------------------------------------------ step coefficients

@pytest.mark.parametrize("sched", ["simple", "beta"])
def test_coefficient_identities(sched):
    sig = so.SCHEDULERS[sched](20, 3.0)
    n = len(sig) - 1
    for st, s, s1 in zip(so.plan("euler", sig), sig, sig[1:]):
        if not st["final"]:
            assert abs(st["c"][0] + st["c"][1] - 1) < 1e-15 and abs(st["c"][0] - s1 / s) < 1e-15
    for st, s, s1 in zip(so.plan("euler_a", sig), sig, sig[1:]):
        if st["final"]:
            continue
        r, _, k, renoise = st["c"][:4]
        # x0 = 0, x ~ N(0, s^2): the ancestral step lands on N(0, s1^2)
        assert abs((k * r * s) ** 2 + renoise ** 2 - s1 * s1) < 1e-12
        assert st["noise"]
    for i, (st, s, s1) in enumerate(zip(so.plan("dpmpp_2m", sig), sig, sig[1:])):
        if st["final"]:
            continue
        assert abs(st["c"][1] - (1 - s1 / s)) < 1e-14  # 1 - e^-h with h = ln(s / s1)
        if i:
            assert abs(st["c"][2] + st["c"][3] - 1) < 1e-14  # the 2nd-order blend keeps constants
    sg = list(sig)
    sg[0] = float(np.float32(so.time_shift(3.0, 1 - 1e-4))) if sg[0] >= 1 else sg[0]
    for i, st in enumerate(so.plan("er_sde", sig)):
        assert st["sigma"] == sg[i] and st["stage"] == min(3, i + 1)
        if st["final"]:
            continue
        st_, s1_ = sg[i], sg[i + 1]
        a_s, a_t = 1 - st_, 1 - s1_
        c = st["c"]
        # x = a_s x0 + s eps with eps = 0: the deterministic part lands on a_t x0
        assert abs(c[0] * a_s + c[1] - a_t) < 1e-12
        # x0 = 0: Var(c0 x + c8 c9 eps) = s1^2
        assert abs((c[0] * st_) ** 2 + (c[8] * c[9]) ** 2 - s1_ * s1_) < 1e-12
    assert n == len(so.plan("er_sde", sig))


def test_er_sde_integrals_against_quadrature():
    """c4 / c7 hold alpha_t (dt + S0 scaler(l_t)) and alpha_t (dt^2/2 + S1 scaler(l_t)) with
    S0 = int_{l_t}^{l_s} dl / scaler(l), S1 = int_{l_t}^{l_s} (l - l_s) / scaler(l) dl as 200-point
    left Riemann sums; both are within the Riemann error of scipy's adaptive quadrature."""
    from scipy.integrate import quad

    sig = so.simple_sigmas(10, 3.0)
    sg = list(sig)
    sg[0] = float(np.float32(so.time_shift(3.0, 1 - 1e-4)))
    lam = [0.0 if v == 0 else v / (1 - v) for v in sg]
    sc = so._er_scaler
    for i, st in enumerate(so.plan("er_sde", sig)):
        if st["final"] or st["stage"] < 2:
            continue
        ls, lt = lam[i], lam[i + 1]
        a_t = sg[i + 1] / lt
        dt = lt - ls
        s0 = (st["c"][4] / a_t - dt) / sc(lt)
        q0 = quad(lambda l: 1 / sc(l), lt, ls)[0]
        assert abs(s0 - q0) < 0.02 * abs(q0) + 1e-12, (i, s0, q0)
        if st["stage"] >= 3:
            s1 = (st["c"][7] / a_t - dt * dt / 2) / sc(lt)
            q1 = quad(lambda l: (l - ls) / sc(l), lt, ls)[0]
            assert abs(s1 - q1) < 0.02 * abs(q1) + 1e-12, (i, s1, q1)


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_js_plans_equal_oracle():
    got = node("import { SamplerPlan, simpleSigmas, betaSigmas } from './samplers.mjs'; const o = {}; "
               "for (const nm of ['euler', 'euler_a', 'dpmpp_2m', 'er_sde']) for (const [k, sg] of "
               "[['s', simpleSigmas(9, 3)], ['b', betaSigmas(13, 2.5)]]) { const p = new SamplerPlan(nm, sg, k === 's' ? 3 : 2.5); "
               "o[nm + k] = Array.from({ length: p.steps }, (_, i) => p.step(i)); } console.log(JSON.stringify(o))")
    for nm in SAMPLERS:
        for k, sg, sh in (("s", so.simple_sigmas(9, 3.0), 3.0), ("b", so.beta_sigmas(13, 2.5), 2.5)):
            ref = so.plan(nm, sg, sh)
            js = got[nm + k]
            assert len(js) == len(ref)
            for a, b in zip(js, ref):
                assert a["kind"] == b["kind"] and a["sigma"] == b["sigma"] and a["final"] == b["final"]
                assert a["stage"] == b["stage"] and a["noise"] == b["noise"]
                # V8's Math.log / exp / expm1 / pow and the C library's may differ in the last ulp
                assert np.allclose(a["c"], b["c"], rtol=1e-14, atol=0), (nm, k)


# ------------------------------------------------------------------ whole runs

@pytest.mark.parametrize("name", ["euler", "dpmpp_2m"])
def test_constant_denoiser_closed_form(name):
    """With den(x) = x0 the flow ODE solution is x(s) = x0 + (s / s_0)(x_init - x0): Euler and
    DPM++ 2M both follow it at every step (their weights are affine in s_{i+1} / s_i)."""
    sig = so.simple_sigmas(12, 3.0)
    x0 = orc.randn(3, 512)
    xi = orc.randn(4, 512)
    traj = []
    so.sample(name, lambda x, s, i: (traj.append(x.copy()), x0)[1], xi, sig)
    for i, x in enumerate(traj):
        ref = x0.astype(np.float64) + sig[i] / sig[0] * (xi.astype(np.float64) - x0)
        assert np.abs(x - ref).max() < 1e-5 * (1 + i), (name, i)


def synthetic_denoiser_js():
    return ("const den = (x, s, i) => { const o = new Float32Array(x.length); const a = 0.3 * s, b = 1 - 0.3 * s; "
            "for (let j = 0; j < x.length; j++) o[j] = a * x[j] + b * T[j] + 0.001 * i; return o; };")


def synthetic_denoiser(T):
    def den(x, s, i):
        return (0.3 * s * x.astype(np.float64) + (1 - 0.3 * s) * T.astype(np.float64) + 0.001 * i).astype(np.float32)
    return den


@pytest.mark.skipif(NODE is None, reason="node is not installed")
@pytest.mark.parametrize("sched", ["simple", "beta"])
def test_js_sample_equals_oracle(sched):
    """The host loop of js/samplers.mjs (the reference's `sample` signature) against the oracle on
    a synthetic affine denoiser, all four samplers, noise from the seeded stream.  On the JS
    plan's coefficients the oracle loop is bit-exact; on its own (last-ulp libm differences in
    the coefficients) within 1e-6."""
    n = 16 * 8 * 9 + 5  # ragged: exercises the noise tail
    T = orc.randn(11, n)
    x = orc.randn(12, n)
    got = node("import { sample, SCHEDULERS, SamplerPlan } from './samplers.mjs'; "
               f"const T = new Float32Array({json.dumps(T.tolist())}); const X = new Float32Array({json.dumps(x.tolist())}); "
               + synthetic_denoiser_js() +
               f"const sg = SCHEDULERS['{sched}'](10, 3); const o = {{}}; (async () => {{ "
               "for (const nm of ['euler', 'euler_a', 'dpmpp_2m', 'er_sde']) { const p = new SamplerPlan(nm, sg, 3); "
               "o[nm] = { x: Array.from(await sample(nm, den, X, sg, { seed: 77, shift: 3 })), "
               "plan: Array.from({ length: p.steps }, (_, i) => p.step(i)) }; } console.log(JSON.stringify(o)); })()")
    sg = so.SCHEDULERS[sched](10, 3.0)
    for nm in SAMPLERS:
        js = np.array(got[nm]["x"], np.float32)
        ref = so.sample(nm, synthetic_denoiser(T), x, sg, seed=77, shift=3.0, steps=got[nm]["plan"])
        assert np.array_equal(js, ref), nm
        own = so.sample(nm, synthetic_denoiser(T), x, sg, seed=77, shift=3.0)
        assert np.abs(own - js).max() <= 1e-6 * np.abs(js).max(), nm
