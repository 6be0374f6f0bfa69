"""CPU oracle of the sampling loop -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of app/samplers.js (sigma schedules, the four sampler updates), of the CFG
combine and denoised estimate of app/pipeline.js:276-283, and of the continuing torch.randn
stream the samplers draw from (app/rng.js:36-67, app/samplers.js:105).  The reference computes
in JavaScript doubles and rounds to float wherever it stores into a Float32Array; every function
here does the same (float64 arithmetic, ``np.float32`` at the same points), so results are
comparable bit for bit.  Only tests and the bench's CPU leg use this module, as the checker.
"""

from __future__ import annotations

import math

import numpy as np

from . import lib, mt19937, _p, _u32p  # noqa: F401  (lib() builds nothing; mt19937 feeds the stream)

F32 = np.float32


# ------------------------------------------------------------------ schedules (samplers.js:6-100)

def time_shift(shift: float, t: float) -> float:
    """samplers.js:6"""
    return (shift * t) / (1 + (shift - 1) * t)


def sigma_table(shift: float) -> np.ndarray:
    """samplers.js:9-13: sigma(i / 1000), i = 1..1000, rounded to float."""
    return np.array([F32(time_shift(shift, i / 1000)) for i in range(1, 1001)], np.float64)


def simple_sigmas(steps: int, shift: float) -> list:
    """samplers.js:16-23"""
    table = sigma_table(shift)
    ss = 1000 / steps
    return [float(table[999 - math.floor(x * ss)]) for x in range(steps)] + [0.0]


_LANCZOS = [0.99999999999980993, 676.5203681218851, -1259.1392167224028, 771.32342877765313,
            -176.61502916214059, 12.507343278686905, -0.13857109526572012, 9.9843695780195716e-6,
            1.5056327351493116e-7]


def _ln_gamma(z: float) -> float:
    """samplers.js:26-36 (Lanczos, g = 7)."""
    if z < 0.5:
        return math.log(math.pi / math.sin(math.pi * z)) - _ln_gamma(1 - z)
    z -= 1
    x = _LANCZOS[0]
    for i in range(1, 9):
        x += _LANCZOS[i] / (z + i)
    t = z + 7.5
    return 0.5 * math.log(2 * math.pi) + (z + 0.5) * math.log(t) - t + math.log(x)


def _betacf(a: float, b: float, x: float) -> float:
    """samplers.js:38-60 (continued fraction, modified Lentz)."""
    fpmin = 1e-300
    c, d = 1.0, 1 - ((a + b) * x) / (a + 1)
    if abs(d) < fpmin:
        d = fpmin
    d = 1 / d
    h = d
    for m in range(1, 301):
        m2 = 2 * m
        aa = (m * (b - m) * x) / ((a - 1 + m2) * (a + m2))
        d = 1 + aa * d
        d = fpmin if abs(d) < fpmin else d
        c = 1 + aa / c
        c = fpmin if abs(c) < fpmin else c
        d = 1 / d
        h *= d * c
        aa = (-(a + m) * (a + b + m) * x) / ((a + m2) * (a + 1 + m2))
        d = 1 + aa * d
        d = fpmin if abs(d) < fpmin else d
        c = 1 + aa / c
        c = fpmin if abs(c) < fpmin else c
        d = 1 / d
        dl = d * c
        h *= dl
        if abs(dl - 1) < 1e-15:
            break
    return h


def beta_cdf(x: float, a: float, b: float) -> float:
    """samplers.js:62-68"""
    if x <= 0:
        return 0.0
    if x >= 1:
        return 1.0
    lbt = _ln_gamma(a + b) - _ln_gamma(a) - _ln_gamma(b) + a * math.log(x) + b * math.log(1 - x)
    if x < (a + 1) / (a + b + 2):
        return (math.exp(lbt) * _betacf(a, b, x)) / a
    return 1 - (math.exp(lbt) * _betacf(b, a, 1 - x)) / b


def beta_ppf(p: float, a: float, b: float) -> float:
    """samplers.js:70-79 (100 bisection steps)."""
    if p <= 0:
        return 0.0
    if p >= 1:
        return 1.0
    lo, hi = 0.0, 1.0
    for _ in range(100):
        mid = (lo + hi) / 2
        if beta_cdf(mid, a, b) < p:
            lo = mid
        else:
            hi = mid
    return (lo + hi) / 2


def beta_sigmas(steps: int, shift: float, alpha: float = 0.6, beta: float = 0.6, ppf=beta_ppf) -> list:
    """samplers.js:83-95; `ppf` can be swapped for a library inverse."""
    table = sigma_table(shift)
    out, last = [], -1
    for i in range(steps):
        t = _js_round(ppf(1 - i / steps, alpha, beta) * 999)
        if t != last:
            out.append(float(table[t]))
        last = t
    return out + [0.0]


def _js_round(v: float) -> int:
    """Math.round: halves go up."""
    return int(math.floor(v + 0.5))


SCHEDULERS = {"simple": simple_sigmas, "beta": beta_sigmas}


# ------------------------------------------------------------------ noise stream (rng.js:36-67)

class TorchRandnStream:
    """torch.manual_seed(seed) followed by successive torch.randn(n) calls on the CPU generator,
    restated from rng.js: uniforms from the low 24 bits of MT19937 outputs, Box-Muller over each
    block of 16 (pairs j, j+8) with float rounding after every step, a ragged tail redrawn."""

    def __init__(self, seed: int):
        self.seed = seed
        self.pos = 0
        self.buf = np.zeros(0, np.uint32)

    def _u32(self, k: int) -> np.ndarray:
        need = self.pos + k
        if need > self.buf.size:
            self.buf = mt19937(self.seed, max(need, 2 * self.buf.size))
        out = self.buf[self.pos:need]
        self.pos = need
        return out

    def _uniform(self, k: int) -> np.ndarray:
        return ((self._u32(k) & 0xFFFFFF).astype(np.float64) / 16777216.0).astype(F32)

    @staticmethod
    def _fill16(d: np.ndarray) -> None:
        """rng.js:44-53 on a [blocks, 16] float32 view, in place."""
        u1 = (F32(1) - d[:, :8]).astype(F32)
        u2 = d[:, 8:].astype(F32)
        lg = np.log(u1.astype(np.float64)).astype(F32)
        radius = np.sqrt((-2.0 * lg.astype(np.float64)).astype(F32).astype(np.float64)).astype(F32)
        theta = (2.0 * math.pi * u2.astype(np.float64)).astype(F32)
        d[:, :8] = radius * np.cos(theta.astype(np.float64)).astype(F32)
        d[:, 8:] = radius * np.sin(theta.astype(np.float64)).astype(F32)

    def randn(self, n: int) -> np.ndarray:
        if n < 16:
            raise ValueError("n >= 16")
        d = self._uniform(n)
        full = n // 16 * 16
        self._fill16(d[:full].reshape(-1, 16))
        if n % 16:
            tail = self._uniform(16)
            self._fill16(tail.reshape(1, 16))
            d[n - 16:] = tail
        return d


# ------------------------------------------------------------------ sampler steps (samplers.js:104-218)

SAMPLER_KIND = {"euler": 0, "euler_a": 1, "dpmpp_2m": 2, "er_sde": 3}


def _er_scaler(v: float) -> float:
    return v * (math.exp(v ** 0.3) + 10)


def plan(name: str, sigmas: list, shift: float = 3.0) -> list:
    """Per-step coefficients, one dict per step: kind, sigma (the denoiser's input), final, stage,
    noise and c[10] (the layout of anima_sampler_desc)."""
    if name not in SAMPLER_KIND:
        raise ValueError(name)
    n = len(sigmas) - 1
    steps = []
    sg = list(sigmas)
    lam = None
    if name == "er_sde":  # samplers.js:170-175
        if sg[0] >= 1:
            sg[0] = float(F32(time_shift(shift, 1 - 1e-4)))
        lam = [0.0 if v == 0 else v / (1 - v) for v in sg]
    for i in range(n):
        c = [0.0] * 10
        st = dict(kind=SAMPLER_KIND[name], sigma=sg[i], final=False, stage=0, noise=False, c=c)
        s, s1 = sigmas[i], sigmas[i + 1]
        if name == "euler":  # samplers.js:109-116
            if s1 == 0:
                st["final"] = True
            else:
                c[0], c[1] = s1 / s, 1 - s1 / s
        elif name == "euler_a":  # samplers.js:118-139
            if s1 == 0:
                st["final"] = True
            else:
                sigma_down = s1 * (s1 / s)
                alpha_ip1 = 1 - s1
                alpha_down = 1 - sigma_down
                renoise = math.sqrt(s1 * s1 - (sigma_down * sigma_down * alpha_ip1 * alpha_ip1)
                                    / (alpha_down * alpha_down))
                r = sigma_down / s
                c[0], c[1], c[2], c[3] = r, 1 - r, alpha_ip1 / alpha_down, renoise
                st["noise"] = True
        elif name == "dpmpp_2m":  # samplers.js:141-166
            st["stage"] = 1 if i > 0 else 0
            if s1 == 0:
                st["final"] = True
            else:
                t = lambda v: -math.log(v)  # noqa: E731
                h = t(s1) - t(s)
                c[0], c[1] = s1 / s, -math.expm1(-h)
                if i > 0:
                    r = (t(s) - t(sigmas[i - 1])) / h
                    c[2], c[3] = 1 + 1 / (2 * r), -1 / (2 * r)
        else:  # er_sde, samplers.js:168-215
            st["stage"] = min(3, i + 1)
            if sg[i + 1] == 0:
                st["final"] = True
            else:
                ls, lt = lam[i], lam[i + 1]
                alpha_s, alpha_t = sg[i] / ls, sg[i + 1] / lt
                r = _er_scaler(lt) / _er_scaler(ls)
                c[0], c[1] = (alpha_t / alpha_s) * r, alpha_t * (1 - r)
                if st["stage"] >= 2:
                    dt = lt - ls
                    step = -dt / 200
                    s0 = su = 0.0
                    for p in range(200):
                        pos = lt + p * step
                        sp = _er_scaler(pos)
                        s0 += 1 / sp
                        su += (pos - ls) / sp
                    s0 *= step
                    su *= step
                    c[2], c[3] = 1 / (ls - lam[i - 1]), -1 / (ls - lam[i - 1])
                    c[4] = alpha_t * (dt + s0 * _er_scaler(lt))
                    if st["stage"] >= 3:
                        c[5], c[6] = 2 / (ls - lam[i - 2]), -2 / (ls - lam[i - 2])
                        c[7] = alpha_t * ((dt * dt) / 2 + su * _er_scaler(lt))
                nz = math.sqrt(max(0.0, lt * lt - ls * ls * r * r))
                if nz > 0:
                    st["noise"] = True
                    c[8], c[9] = alpha_t, nz
        steps.append(st)
    return steps


def _axpby(a, x, b, y):
    """Float32Array o[i] = a * x[i] + b * y[i] (doubles, one rounding to float)."""
    return (a * x.astype(np.float64) + b * y.astype(np.float64)).astype(F32)


def cfg_denoised(x, v, v_uncond, cfg, sigma):
    """pipeline.js:276-282: v = vu + cfg (v - vu) (float), den = x - sigma v (float)."""
    v = np.asarray(v, F32)
    if v_uncond is not None:
        vu = np.asarray(v_uncond, F32).astype(np.float64)
        v = (vu + cfg * (v.astype(np.float64) - vu)).astype(F32)
    return (np.asarray(x, F32).astype(np.float64) - sigma * v.astype(np.float64)).astype(F32)


def apply(st: dict, x, den, state: dict, eps=None):
    """One sampler update (samplers.js:109-215) given den; state carries old / old_d.  Returns
    the new x (float32)."""
    c = st["c"]
    x = np.asarray(x, F32)
    den = np.asarray(den, F32)
    if st["final"]:
        state["old"] = den
        return den.copy()
    k = st["kind"]
    if k == 0:
        o = _axpby(c[0], x, c[1], den)
    elif k == 1:
        t = _axpby(c[0], x, c[1], den)
        o = (c[2] * t.astype(np.float64) + eps.astype(np.float64) * c[3]).astype(F32)
    elif k == 2:
        dd = _axpby(c[2], den, c[3], state["old"]) if st["stage"] else den
        o = _axpby(c[0], x, c[1], dd)
    else:
        o = _axpby(c[0], x, c[1], den)
        if st["stage"] >= 2:
            dD = _axpby(c[2], den, c[3], state["old"])
            o = (o.astype(np.float64) + c[4] * dD.astype(np.float64)).astype(F32)
            if st["stage"] >= 3:
                dU = _axpby(c[5], dD, c[6], state["old_d"])
                o = (o.astype(np.float64) + c[7] * dU.astype(np.float64)).astype(F32)
            state["old_d"] = dD
        if eps is not None:
            o = (o.astype(np.float64) + c[8] * eps.astype(np.float64) * c[9]).astype(F32)
    state["old"] = den
    return o


def sample(name: str, denoise, x, sigmas: list, seed: int = 0, shift: float = 3.0, steps=None):
    """samplers.js:104: denoise(x, sigma, i) -> den; the noise comes from the sampler's own
    generator seeded with `seed`, drawn only on steps that use it.  `steps` replaces plan(...)
    (to run on coefficients computed elsewhere)."""
    gen = TorchRandnStream(seed)
    state = {}
    x = np.asarray(x, F32)
    for i, st in enumerate(steps if steps is not None else plan(name, sigmas, shift)):
        den = np.asarray(denoise(x, st["sigma"], i), F32)
        x = apply(st, x, den, state, gen.randn(x.size) if st["noise"] else None)
    return x
