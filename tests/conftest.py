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


def clamp_regime_case(K=64, V=64, c=10.0):
    """Per-channel decay in the regime where the block-decay clamp binds
    (decay.rs:41-49: each factor's exponent capped at MAX_EXPONENT = 48,
    reference row m/2 = 8 of each 16-row block), with closed-form outputs and
    gradients (combined_backward.rs:480-496: a clamped exponent passes no
    gradient).

    One 64-token chunk, g = −c on every token and channel, so the in-chunk
    cumulative gate is G_t = −c(t+1); erase = write = 1; zero initial state.
    Two isolated key → query pairs in block 0, on channels and value columns
    0 and 1: key/value at token 0, query at token 2 (row exponent
    G_2 − G_8 = 6c = 60, clamped to 48; column exponent G_8 − G_0 = −8c),
    and key/value at token 13, query at token 14 (row exponent −6c; column
    exponent G_8 − G_13 = 5c = 50, clamped). With T = I (the keys are
    orthogonal) the outputs are y₁ = scale·e^{48−8c} and
    y₂ = scale·e^{−6c+48}, against scale·e^{−2c} and scale·e^{−c} unclamped.

    Backward with dy = 1 at those two outputs and no state cotangent:
    d_q, d_k, d_v and d_write are y₁ / y₂ at the pair's entries. d_g is the
    reverse in-chunk sum of dG: pair 1's clamped row factor passes nothing,
    its column factor gives dG_8 = +y₁, dG_0 = −y₁, so d_g[1…8][0] = y₁; pair
    2's clamped column factor passes nothing, its row factor gives
    dG_14 = +y₂, dG_8 = −y₂, so d_g[9…14][1] = y₂. Every other entry of every
    output and gradient is zero (or below e^{−400})."""
    S = 64
    q = np.zeros((1, S, 1, K))
    k = np.zeros((1, S, 1, K))
    v = np.zeros((1, S, 1, V))
    q[0, 2, 0, 0] = k[0, 0, 0, 0] = v[0, 0, 0, 0] = 1.0
    q[0, 14, 0, 1] = k[0, 13, 0, 1] = v[0, 13, 0, 1] = 1.0
    args = [q, k, v, np.ones((1, S, 1, K)), np.ones((1, S, 1, V)), np.full((1, S, 1, K), -c),
            np.zeros((1, 1, K, V))]
    scale = 1.0 / np.sqrt(K)
    y1, y2 = scale * np.exp(48.0 - 8 * c), scale * np.exp(48.0 - 6 * c)
    dy = np.zeros((1, S, 1, V))
    dy[0, 2, 0, 0] = dy[0, 14, 0, 1] = 1.0
    y = np.zeros((1, S, 1, V))
    y[0, 2, 0, 0], y[0, 14, 0, 1] = y1, y2
    pair = lambda shape, a, b: _entries(shape, {a: y1, b: y2})
    dg = np.zeros((1, S, 1, K))
    dg[0, 1:9, 0, 0] = y1
    dg[0, 9:15, 0, 1] = y2
    want = {
        "y": y,
        "d_q": pair(q.shape, (0, 2, 0, 0), (0, 14, 0, 1)),
        "d_k": pair(k.shape, (0, 0, 0, 0), (0, 13, 0, 1)),
        "d_v": pair(v.shape, (0, 0, 0, 0), (0, 13, 0, 1)),
        "d_erase": np.zeros((1, S, 1, K)),
        "d_write": pair(v.shape, (0, 0, 0, 0), (0, 13, 0, 1)),
        "d_g": dg,
    }
    return args, dy, want


def _entries(shape, values):
    out = np.zeros(shape)
    for idx, val in values.items():
        out[idx] = val
    return out


def closed_form_err(got, want):
    """Largest relative error over want's nonzero entries, and the largest
    magnitude elsewhere relative to want's smallest nonzero entry."""
    got = np.asarray(got, dtype=np.float64)
    nz = want != 0
    if not nz.any():
        return 0.0, float(np.abs(got).max())
    rel = float((np.abs(got[nz] - want[nz]) / np.abs(want[nz])).max())
    rest = float(np.abs(got[~nz]).max()) / float(np.abs(want[nz]).min()) if (~nz).any() else 0.0
    return rel, rest


def rel_err(a, b):
    """Normwise relative error max|a-b| / max|b| (b is the reference)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    denom = max(float(np.abs(b).max()), 1e-30) if b.size else 1.0
    return float(np.abs(a - b).max()) / denom if b.size else 0.0


@pytest.fixture
def rng():
    return np.random.default_rng(20260826)
