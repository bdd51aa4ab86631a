"""GPU parity of dn_recurrent: delta_step over a whole sequence in one call.

Checked against the oracle's recurrent pass (recurrent.rs:107-142) and against
the same tokens run as one dn_step per token, across the shapes the kernel
specialises on: rows per lane (head_k_dim up to 64 / 128 / 256 / 512), one or two
columns per lane (head_v_dim below 128 or odd vs even from 128), every gate
width, fp32 and bf16 inputs, and a state updated in place. Bars: normwise
relative error 1e-4 for fp32 inputs, 2e-2 for bf16 inputs (BASELINE.json
north_star); 1e-5 between dn_recurrent and the dn_step loop, which evaluate
the same arithmetic.
"""

import numpy as np
import pytest
import torch

from conftest import l2, rel_err
from gpu_util import DEV, announce, np_of, pkg
from oracle import oracle as O

pytestmark = pytest.mark.gpu

abi = pkg.abi

CASES = [
    # B, S, H, K, V, ew, ww, dw, dtype
    (2, 7, 3, 4, 6, 1, 1, 0, torch.float32),
    (2, 9, 2, 8, 12, 8, 12, 8, torch.float32),
    (1, 33, 2, 64, 64, 1, 1, 1, torch.float32),
    (2, 16, 2, 128, 128, 128, 128, 128, torch.float32),
    (1, 12, 2, 256, 256, 1, 1, 1, torch.float32),
    (1, 10, 2, 100, 70, 1, 70, 100, torch.float32),
    (1, 10, 2, 192, 129, 192, 1, 1, torch.float32),
    (1, 5, 1, 1, 1, 1, 1, 1, torch.float32),
    (2, 24, 4, 128, 256, 1, 1, 1, torch.bfloat16),
    (1, 2, 16, 128, 128, 1, 1, 1, torch.bfloat16),
    # above 256 state rows: 64 rows a lane, one column a lane
    (1, 9, 2, 384, 160, 384, 1, 384, torch.float32),
    (2, 6, 2, 512, 128, 1, 128, 1, torch.float32),
    (1, 8, 2, 512, 256, 1, 1, 1, torch.bfloat16),
]


def inputs(rng, B, S, H, K, V, ew, ww, dw, gamma=1.9):
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    e = rng.uniform(0.05, gamma, (B, S, H, ew))
    w = rng.uniform(0.05, 1.0, (B, S, H, ww))
    g = rng.uniform(-0.5, -0.01, (B, S, H, dw)) if dw else None
    s = rng.normal(0, 0.2, (B, H, K, V))
    return q, k, v, e, w, g, s


def on_gpu(q, k, v, e, w, g, s, dt):
    t = lambda a, d=torch.float32: None if a is None else torch.tensor(a, dtype=torch.float32,
                                                                      device=DEV).to(d)
    return [t(q, dt), t(k, dt), t(v, dt), t(e), t(w), t(g), t(s)]


def run_recurrent(gq, gk, gv, ge, gw, gg, gs, scale, y_dtype=torch.float32, state_out=None):
    B, S, H, _ = gq.shape
    y = torch.empty((B, S, H, gv.shape[3]), dtype=y_dtype, device=DEV)
    s1 = torch.empty_like(gs) if state_out is None else state_out
    abi.run_recurrent(abi.recurrent_args(gq, gk, gv, ge, gw, gg, gs, y, s1, scale))
    torch.cuda.synchronize()
    return y, s1


@pytest.mark.parametrize("case", CASES)
def test_recurrent_matches_oracle(rng, case):
    B, S, H, K, V, ew, ww, dw, dt = case
    announce(f"dn_recurrent {case}")
    q, k, v, e, w, g, s = inputs(rng, B, S, H, K, V, ew, ww, dw)
    g_args = on_gpu(q, k, v, e, w, g, s, dt)
    scale = 1.0 / np.sqrt(K)
    y, s1 = run_recurrent(*g_args, scale)
    ref_qkv = [t.float().cpu().numpy().astype(np.float64) for t in g_args[:3]]
    y0, s0 = O.recurrent(*ref_qkv, e, w, g, s, scale=scale)
    tol = 1e-4 if dt == torch.float32 else 2e-2
    assert rel_err(np_of(y), y0) < tol
    assert rel_err(np_of(s1), s0) < tol


@pytest.mark.parametrize("case", [CASES[1], CASES[4], CASES[6], CASES[8]])
def test_recurrent_matches_a_dn_step_loop(rng, case):
    """One dn_recurrent call = S dn_step calls on the token slices."""
    B, S, H, K, V, ew, ww, dw, dt = case
    announce(f"dn_recurrent vs dn_step loop {case}")
    g_args = on_gpu(*inputs(rng, B, S, H, K, V, ew, ww, dw), dt)
    y, s1 = run_recurrent(*g_args, 0.3)
    st = g_args[6].clone()
    ys = []
    for t in range(S):
        sl = [None if a is None else a[:, t].contiguous() for a in g_args[:6]]
        yt, st = pkg.delta_step(*sl, st, 0.3, y_dtype=torch.float32, in_place=True)
        ys.append(yt)
    torch.cuda.synchronize()
    assert rel_err(np_of(y), np_of(torch.stack(ys, 1))) < 1e-5
    assert rel_err(np_of(s1), np_of(st)) < 1e-5


def test_recurrent_bf16_output_and_in_place_state(rng):
    """y in bf16 (the reference's output dtype for bf16 inputs) and
    state_out aliasing state_in."""
    B, S, H, K, V = 2, 6, 2, 64, 128
    announce("dn_recurrent bf16 y, in-place state")
    q, k, v, e, w, g, s = inputs(rng, B, S, H, K, V, 1, 1, 1)
    g_args = on_gpu(q, k, v, e, w, g, s, torch.bfloat16)
    st = g_args[6]
    y, s1 = run_recurrent(*g_args, 0.125, y_dtype=torch.bfloat16, state_out=st)
    assert s1.data_ptr() == st.data_ptr() and y.dtype == torch.bfloat16
    ref_qkv = [t.float().cpu().numpy().astype(np.float64) for t in g_args[:3]]
    y0, s0 = O.recurrent(*ref_qkv, e, w, g, s, scale=0.125)
    assert rel_err(np_of(y), y0) < 2e-2 and rel_err(np_of(st), s0) < 2e-2


def test_delta_product_decode_is_a_short_recurrent_run(rng):
    """DeltaProduct decode (delta_product.rs:270-305): u Householder
    micro-steps per token, the first carrying the token's decay and the
    others none, fold into a u-token sequence. Two decode tokens with u = 3
    through dn_recurrent equal six dn_step calls and the oracle."""
    B, H, K, V, u = 2, 4, 128, 128, 3
    announce("DeltaProduct decode via dn_recurrent")
    q, k, v, e, w, _, s = inputs(rng, B, 2 * u, H, K, V, 1, 1, 0)
    g = np.zeros((B, 2 * u, H, 1))
    g[:, ::u] = rng.uniform(-0.5, -0.01, (B, 2, H, 1))
    g_args = on_gpu(q, k, v, e, w, g, s, torch.float32)
    y, s1 = run_recurrent(*g_args, 0.1)
    y0, s0 = O.recurrent(q, k, v, e, w, g, s, scale=0.1)
    assert rel_err(np_of(y), y0) < 1e-4 and rel_err(np_of(s1), s0) < 1e-4


def test_wide_heads_fall_back_to_the_step_loop(rng):
    """head_k_dim above dn_recurrent's limit: the C ABI refuses it and
    DeltaInput's recurrent path runs dn_step per token instead."""
    B, S, H, K, V = 1, 4, 2, abi.RECURRENT_MAX_K + 44, 48
    announce("dn_recurrent wide-head fallback")
    q, k, v, e, w, g, s = inputs(rng, B, S, H, K, V, 1, 1, 1)
    g_args = on_gpu(q, k, v, e, w, g, s, torch.float32)
    with pytest.raises(Exception, match="head_k_dim up to"):
        run_recurrent(*g_args, 0.1)
    yr, sr = pkg.DeltaInput(*g_args).run(pkg.DeltaPath.recurrent())
    torch.cuda.synchronize()
    y0, s0 = O.recurrent(q, k, v, e, w, g, s)
    assert rel_err(np_of(yr), y0) < 1e-4 and rel_err(np_of(sr), s0) < 1e-4


def test_recurrent_path_reads_bf16_gates_as_their_fp32_values():
    """DeltaPath::Recurrent with gates and state in bf16 (a Burn backend whose
    float dtype is bf16 hands them over so) gives the result of the same
    values upcast to fp32: the host mirror converts them before the call."""
    announce("dn_recurrent through DeltaPath.recurrent(): bf16 gates and state")
    rng = np.random.default_rng(31)
    q, k, v, e, w, g, s = inputs(rng, 2, 9, 3, 16, 24, 16, 1, 16)
    gq, gk, gv, ge, gw, gg, gs = on_gpu(q, k, v, e, w, g, s, torch.float32)
    b = lambda t: t.to(torch.bfloat16)
    y_b, s_b = pkg.DeltaInput(gq, gk, gv, b(ge), b(gw), b(gg), b(gs)).run(
        pkg.DeltaPath.recurrent())
    up = lambda t: b(t).float()
    y_f, s_f = pkg.DeltaInput(gq, gk, gv, up(ge), up(gw), up(gg), up(gs)).run(
        pkg.DeltaPath.recurrent())
    torch.cuda.synchronize()
    assert torch.equal(y_b, y_f) and torch.equal(s_b, s_f)
