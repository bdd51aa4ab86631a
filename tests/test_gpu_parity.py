"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bars: normwise relative error max|a−b|/max|ref|
≤ 1e-4 for fp32 inputs, ≤ 2e-2 for bf16 inputs with fp32 state; the FLA
fixture at the reference's own 1e-4 absolute.
"""

import numpy as np
import pytest
import torch

from conftest import fla_fixture, l2, random_raw, rel_err
from gpu_util import DEV, announce, as_oracle_inputs, np_of, pkg, to_gpu
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GENERIC = pkg.abi.DN_ALGO_GENERIC
AUTO = pkg.abi.DN_ALGO_AUTO


def gpu_chunk(args, L, algo=AUTO, y_dtype=None, scale=None):
    q, k, v, e, w, g, s = args
    K = q.shape[3]
    sc = 1.0 / np.sqrt(K) if scale is None else scale
    y, st = pkg.delta_chunk_recalculated(q, k, v, e, w, g, s, g is not None, L, sc, algo=algo,
                                         y_dtype=y_dtype)
    torch.cuda.synchronize()
    return np_of(y), np_of(st)


# ---------------------------------------------------------------------------
# The reference's FLA fixture (src/delta/tests.rs:533-568, 760-812)
# ---------------------------------------------------------------------------

def fixture_inputs(case):
    _, a = fla_fixture()
    beta = a["IN_BETA"][..., None]
    if case == "ungated":
        return [a["IN_Q"], a["IN_K"], a["IN_V"], beta, beta, None, a["IN_STATE"]], "UNGATED"
    if case == "gated":
        return [a["IN_Q"], a["IN_K"], a["IN_V"], beta, beta, a["IN_G"][..., None],
                a["IN_STATE"]], "GATED"
    return [a["IN_Q"], a["IN_K"], a["IN_V"], a["IN_B"], a["IN_W"], a["IN_GK"],
            a["IN_STATE"]], "GDN2"


@pytest.mark.parametrize("case", ["ungated", "gated", "gdn2"])
def test_fixture_through_every_path(case):
    args, tag = fixture_inputs(case)
    _, a = fla_fixture()
    want_y, want_s = a[tag + "_Y"], a[tag + "_STATE"]
    announce(f"fixture {case}")
    g_args = to_gpu(args)
    for path in [pkg.DeltaPath.recurrent(), pkg.DeltaPath.with_chunk_len(3),
                 pkg.DeltaPath.with_chunk_len(4), pkg.DeltaPath.with_chunk_len(16)]:
        y, s = pkg.DeltaInput(*g_args).run(path)
        torch.cuda.synchronize()
        assert np.abs(np_of(y) - want_y).max() < 1e-4, path
        assert np.abs(np_of(s) - want_s).max() < 1e-4, path


# ---------------------------------------------------------------------------
# Chunk forward vs the oracle (shapes of src/delta/tests.rs and
# chunk_recalculated/tests.rs)
# ---------------------------------------------------------------------------

FWD_CASES = [
    # B, S, H, K, V, L, beta_max, gated, random_state, channel
    (2, 16, 3, 8, 8, 8, 0.95, False, False, False),
    (2, 16, 3, 8, 8, 8, 0.95, True, False, False),
    (2, 12, 2, 8, 16, 4, 0.95, True, True, False),
    (2, 12, 2, 8, 8, 6, 1.95, True, True, False),
    (2, 13, 2, 8, 8, 8, 0.95, True, True, False),
    (1, 5, 1, 4, 4, 8, 0.95, False, False, False),
    (2, 16, 3, 8, 8, 8, 0.95, True, True, True),
    (2, 40, 2, 8, 8, 32, 0.95, True, True, True),
    (1, 37, 1, 4, 6, 16, 1.95, True, True, True),
    (2, 24, 2, 8, 8, 1, 0.95, True, True, True),
    (2, 128, 2, 8, 8, 128, 0.95, True, True, False),
    (1, 200, 2, 64, 64, 64, 0.95, True, True, False),
    (1, 130, 2, 128, 256, 64, 0.95, True, True, False),
    (1, 70, 2, 32, 48, 64, 0.95, True, True, True),
]


@pytest.mark.parametrize("case", FWD_CASES)
def test_chunk_fwd_matches_oracle(rng, case):
    B, S, H, K, V, L, bmax, gated, rstate, channel = case
    announce(f"chunk fwd generic {case}")
    args = random_raw(rng, B, S, H, K, V, bmax, gated, rstate, channel)
    y, s = gpu_chunk(to_gpu(args), L, algo=GENERIC)
    y0, s0 = O.chunk_fwd(*args, chunk_len=L)
    assert rel_err(y, y0) < 1e-4 and rel_err(s, s0) < 1e-4


@pytest.mark.parametrize("case", FWD_CASES[6:10])
def test_chunk_fwd_bf16_inputs(rng, case):
    B, S, H, K, V, L, bmax, gated, rstate, channel = case
    announce(f"chunk fwd bf16 {case}")
    g_args = to_gpu(random_raw(rng, B, S, H, K, V, bmax, gated, rstate, channel),
                    torch.bfloat16)
    y, s = gpu_chunk(g_args, L, algo=GENERIC, y_dtype=torch.float32)
    y0, s0 = O.chunk_fwd(*as_oracle_inputs(g_args), chunk_len=L)
    assert rel_err(y, y0) < 2e-2 and rel_err(s, s0) < 2e-2


def test_config1_chunk_and_step_agree(rng):
    """B=1, H=4, T=512, dk=dv=64, chunk 64, fp32; S₀ = 0.
    The chunk forward matches the oracle, and 512 dn_step calls match both."""
    announce("config 1")
    B, S, H, K, V = 1, 512, 4, 64, 64
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, 1))))
    g = -np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * 0.1
    s0 = np.zeros((B, H, K, V))
    args = [q, k, v, beta, beta, g, s0]
    y, s = gpu_chunk(to_gpu(args), 64)
    y0, st0 = O.chunk_fwd(*args, chunk_len=64)
    assert rel_err(y, y0) < 1e-4 and rel_err(s, st0) < 1e-4
    yr, sr = pkg.DeltaInput(*to_gpu(args)).run(pkg.DeltaPath.recurrent())
    torch.cuda.synchronize()
    assert rel_err(np_of(yr), y0) < 1e-4 and rel_err(np_of(sr), st0) < 1e-4
    assert rel_err(np_of(yr), y) < 1e-4 and rel_err(np_of(sr), s) < 1e-4


# ---------------------------------------------------------------------------
# dn_step vs the oracle
# ---------------------------------------------------------------------------

STEP_CASES = [
    # B, H, K, V, ew, ww, dw, dtype
    (2, 2, 4, 6, 1, 1, 0, torch.float32),
    (2, 3, 4, 6, 4, 6, 4, torch.float32),
    (3, 2, 8, 12, 1, 1, 1, torch.float32),
    (4, 4, 128, 256, 1, 1, 1, torch.float32),
    (2, 4, 128, 128, 128, 128, 128, torch.float32),
    (2, 2, 64, 100, 1, 100, 1, torch.float32),
    (2, 2, 600, 40, 1, 1, 1, torch.float32),
    (4, 4, 128, 256, 1, 1, 1, torch.bfloat16),
]


@pytest.mark.parametrize("case", STEP_CASES)
def test_step_matches_oracle(rng, case):
    B, H, K, V, ew, ww, dw, dt = case
    announce(f"dn_step {case}")
    q = l2(rng.standard_normal((B, H, K)))
    k = l2(rng.standard_normal((B, H, K)))
    v = rng.standard_normal((B, H, V))
    e = rng.uniform(0.05, 1.9, (B, H, ew))
    w = rng.uniform(0.05, 1.0, (B, H, ww))
    g = rng.uniform(-0.5, -0.01, (B, H, dw)) if dw else None
    s = rng.normal(0, 0.2, (B, H, K, V))
    gq = [torch.tensor(a, dtype=torch.float32, device=DEV).to(dt) for a in (q, k, v)]
    gg = [None if a is None else torch.tensor(a, dtype=torch.float32, device=DEV)
          for a in (e, w, g, s)]
    y, s1 = pkg.delta_step(*gq, *gg, 1.0 / np.sqrt(K), y_dtype=torch.float32)
    torch.cuda.synchronize()
    ref_in = [t.float().cpu().numpy().astype(np.float64) for t in gq]
    y0, s0 = O.delta_step(*ref_in, e, w, g, s)
    tol = 1e-4 if dt == torch.float32 else 2e-2
    assert rel_err(np_of(y), y0) < tol and rel_err(np_of(s1), s0) < tol


def test_step_in_place_state(rng):
    """state_out may alias state_in (the in-place read-modify-write)."""
    announce("dn_step in place")
    B, H, K, V = 2, 2, 128, 256
    args = [l2(rng.standard_normal((B, H, K))), l2(rng.standard_normal((B, H, K))),
            rng.standard_normal((B, H, V)), rng.uniform(0.05, 1, (B, H, 1)),
            rng.uniform(0.05, 1, (B, H, 1)), rng.uniform(-0.5, -0.01, (B, H, 1))]
    s = rng.normal(0, 0.2, (B, H, K, V))
    t = [torch.tensor(a, dtype=torch.float32, device=DEV) for a in args]
    st = torch.tensor(s, dtype=torch.float32, device=DEV)
    y, st2 = pkg.delta_step(*t, st, 0.1, in_place=True)
    torch.cuda.synchronize()
    assert st2.data_ptr() == st.data_ptr()
    y0, s0 = O.delta_step(*args, s, scale=0.1)
    assert rel_err(np_of(y), y0) < 1e-4 and rel_err(np_of(st), s0) < 1e-4


# ---------------------------------------------------------------------------
# Backward vs the oracle (chunk_recalculated/tests.rs shapes)
# ---------------------------------------------------------------------------

BWD_CASES = [
    (2, 16, 3, 8, 8, 8, 0.95, False, False),
    (2, 16, 3, 8, 8, 8, 0.95, True, False),
    (2, 16, 3, 8, 8, 8, 0.95, True, True),
    (2, 40, 2, 8, 8, 32, 0.95, True, True),
    (2, 12, 2, 8, 8, 6, 1.95, True, False),
    (2, 12, 2, 8, 8, 6, 1.95, True, True),
    (2, 13, 2, 8, 8, 8, 0.95, True, False),
    (1, 5, 1, 4, 4, 8, 0.95, False, False),
    (2, 37, 2, 4, 6, 16, 0.95, True, True),
    (2, 16, 2, 8, 16, 8, 0.95, True, False),
    (2, 16, 2, 16, 8, 8, 0.95, True, True),
    (2, 24, 2, 8, 8, 1, 0.95, True, True),
    (1, 150, 2, 64, 64, 64, 0.95, True, True),
]


@pytest.mark.parametrize("case", BWD_CASES)
def test_chunk_bwd_matches_oracle(rng, case):
    B, S, H, K, V, L, bmax, gated, channel = case
    announce(f"chunk bwd {case}")
    args = random_raw(rng, B, S, H, K, V, bmax, gated, True, channel)
    dy = rng.standard_normal((B, S, H, V))
    ds = rng.standard_normal((B, H, K, V))
    g_args = to_gpu(args)
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)
    got = pkg.combined_backward(t(dy), t(ds), *g_args, L, 1.0 / np.sqrt(K))
    torch.cuda.synchronize()
    want = O.chunk_bwd(dy, ds, *args, chunk_len=L)
    names = ["d_q", "d_k", "d_v", "d_erase", "d_write", "d_g", "d_state"]
    vals = [got.d_q_bshk, got.d_k_bshk, got.d_v_bshv, got.d_erase_bshK, got.d_write_bshV,
            got.d_g_bshK, got.d_state_bhkv]
    for name, a, b in zip(names, vals, want):
        if b is None:
            assert a is None
            continue
        assert rel_err(np_of(a), b) < 1e-4, name


def test_autograd_node_matches_oracle(rng):
    """DeltaInput.run under torch autograd takes the custom node (backward.rs)."""
    announce("autograd node")
    B, S, H, K, V, L = 2, 20, 2, 8, 8, 8
    args = random_raw(rng, B, S, H, K, V, 0.95, True, True, True)
    leaves = [torch.tensor(a, dtype=torch.float32, device=DEV, requires_grad=True)
              for a in args]
    y_head = rng.standard_normal((B, S, H, V))
    s_head = rng.standard_normal((B, H, K, V))
    y, s = pkg.DeltaInput(*leaves).run(pkg.DeltaPath.with_chunk_len(L))
    loss = (y * torch.tensor(y_head, dtype=torch.float32, device=DEV)).sum() + \
        (s * torch.tensor(s_head, dtype=torch.float32, device=DEV)).sum()
    loss.backward()
    want = O.chunk_bwd(y_head, s_head, *args, chunk_len=L)
    for leaf, b in zip(leaves, want):
        assert rel_err(np_of(leaf.grad), b) < 1e-4


# ---------------------------------------------------------------------------
# Invariants on the GPU path
# ---------------------------------------------------------------------------

def test_split_calls_match_a_single_call(rng):
    announce("split stream")
    q, k, v, e, w, g, s = to_gpu(random_raw(rng, 2, 20, 2, 8, 8, 0.95, True, False))
    P = pkg.DeltaPath.with_chunk_len(4)
    y_all, s_all = pkg.DeltaInput(q, k, v, e, w, g, s).run(P)
    cut = lambda a, sl: a[:, sl].contiguous()
    y1, s_mid = pkg.DeltaInput(*(cut(a, slice(0, 7)) for a in (q, k, v, e, w, g)), s).run(P)
    y2, s_end = pkg.DeltaInput(*(cut(a, slice(7, 20)) for a in (q, k, v, e, w, g)),
                               s_mid).run(P)
    torch.cuda.synchronize()
    assert (torch.cat([y1, y2], 1) - y_all).abs().max().item() < 1e-4
    assert (s_end - s_all).abs().max().item() < 1e-4


def test_zero_gate_is_the_ungated_rule(rng):
    announce("zero gate")
    q, k, v, e, w, _, s = to_gpu(random_raw(rng, 2, 12, 2, 8, 8, 0.95, False, True))
    zeros = torch.zeros((2, 12, 2, 1), device=DEV)
    for P in [pkg.DeltaPath.recurrent(), pkg.DeltaPath.with_chunk_len(5)]:
        y0, s0 = pkg.DeltaInput(q, k, v, e, w, None, s).run(P)
        y1, s1 = pkg.DeltaInput(q, k, v, e, w, zeros, s).run(P)
        torch.cuda.synchronize()
        assert (y0 - y1).abs().max().item() < 1e-5 and (s0 - s1).abs().max().item() < 1e-5


def test_nonfinite_guard(rng):
    announce("nonfinite guard")
    args = to_gpu(random_raw(rng, 1, 8, 1, 4, 4, 0.95, True, True))
    args[0][0, 3, 0, 1] = float("nan")
    with pytest.raises(pkg.DeltaError, match="NaN or Inf found in the inputs"):
        pkg.DeltaInput(*args).run(pkg.DeltaPath.with_chunk_len(4), check_finite=True)
