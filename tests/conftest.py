"""Shared test plumbing: the `gpu` marker, seeded inputs, and module loading.

The product package lives in the directory `burn-deltanet_amd/`, whose name is
not a Python identifier; `load_package()` registers it as `burn_deltanet_amd`.
"""

from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    name = "burn_deltanet_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "burn-deltanet_amd"
    spec = importlib.util.spec_from_file_location(
        name, pkg_dir / "__init__.py", submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def fla_fixture():
    fx = json.loads((ROOT / "tests" / "golden" / "fla_fixture.json").read_text())
    arrays = {k: np.array(fx[k], dtype=np.float64).reshape(fx["shapes"][k])
              for k in fx["shapes"]}
    return fx["dims"], arrays


def l2(x, eps=1e-6):
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def random_raw(rng, B, S, H, K, V, beta_max=0.95, gated=True, random_state=True,
               channel=False, dtype=np.float64):
    """Inputs shaped the way a block hands them over (mirrors random_raw_gates,
    src/delta/tests.rs:69-139): q/k L2-normalised, gates squashed, g <= 0."""
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    kw, vw = (K, V) if channel else (1, 1)
    erase = rng.uniform(0.05, beta_max, (B, S, H, kw))
    write = rng.uniform(0.05, 1.0, (B, S, H, vw)) if channel else erase.copy()
    g = rng.uniform(-0.5, -0.01, (B, S, H, kw)) if gated else None
    state = (rng.normal(0.0, 0.2, (B, H, K, V)) if random_state
             else np.zeros((B, H, K, V)))
    cast = lambda a: None if a is None else a.astype(dtype)
    return [cast(a) for a in (q, k, v, erase, write, g, state)]


def rel_err(a, b):
    """Normwise relative error max|a-b| / max|b| (b is the reference)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    denom = max(float(np.abs(b).max()), 1e-30) if b.size else 1.0
    return float(np.abs(a - b).max()) / denom if b.size else 0.0


@pytest.fixture
def rng():
    return np.random.default_rng(20260826)
