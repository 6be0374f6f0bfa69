"""Shared test helpers: package loader, seeded inputs, error metrics (check.js:24-37)."""

import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "anima-studio_amd")
RUN_CASE = os.path.join(ROOT, "tests", "js", "run_case.mjs")  # the JS op-case harness of the GPU tests


def amd():
    """The anima-studio_amd package (its directory name is not an identifier)."""
    if "anima_studio_amd" in sys.modules:
        return sys.modules["anima_studio_amd"]
    spec = importlib.util.spec_from_file_location("anima_studio_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["anima_studio_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def rel_l2(got, ref):
    """rel L2 = ||got - ref|| / ||ref|| (tools/check.js:24-37)."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    return float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))


def max_abs(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))))


def report(name, got, ref):
    r, m = rel_l2(got, ref), max_abs(got, ref)
    print(f"{name}: rel L2 {r:.3e}  max|d| {m:.3e}", flush=True)
    return r, m
