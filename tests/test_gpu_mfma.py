"""The MFMA (bf16) chunk forward against the oracle, at the north_star's bf16
bar (normwise relative ≤ 2e-2, fp32 state), on the shapes it serves:
Gated DeltaNet / DeltaNet / DeltaProduct with per-head gates.

The oracle is fed the bf16-rounded q/k/v the GPU actually reads."""

import numpy as np
import pytest
import torch

from conftest import clamp_regime_case, closed_form_err, l2, rel_err
from gpu_util import DEV, announce, as_oracle_inputs, np_of, pkg, to_gpu
from oracle import oracle as O

pytestmark = pytest.mark.gpu

MFMA = pkg.abi.DN_ALGO_MFMA
TOL = 2e-2


def gdn_inputs(rng, B, S, H, K, V, gated=True, beta_scale=1.0, state_std=0.0, split=False,
               g_scale=0.05):
    """Config-2 distributions: q,k L2(N(0,1)), v N(0,1), β = σ(N), g = −softplus(N)·g_scale."""
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    beta = beta_scale / (1.0 + np.exp(-rng.standard_normal((B, S, H, 1))))
    write = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, 1))))) if split else beta
    g = (-np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * g_scale) if gated else None
    s0 = rng.normal(0.0, state_std, (B, H, K, V)) if state_std else np.zeros((B, H, K, V))
    return [q, k, v, beta, write, g, s0]


def run_mfma(g_args, y_dtype=torch.bfloat16, in_place=False):
    q, k, v, e, w, g, s = g_args
    B, S, H, K = q.shape
    V = v.shape[3]
    y = torch.empty((B, S, H, V), dtype=y_dtype, device=DEV)
    s_out = s if in_place else torch.empty_like(s)
    a = pkg.abi.chunk_fwd_args(q, k, v, e, w, g, s, y, s_out, 64, None, algo=MFMA)
    assert pkg.abi.lib().dn_chunk_fwd_algo(a) == MFMA
    pkg.abi.run_chunk_fwd(a)
    torch.cuda.synchronize()
    return np_of(y), np_of(s_out)


CASES = [
    # B, S, H, K, V, gated, beta_scale, state_std, split(erase≠write)
    (1, 64, 1, 128, 64, True, 1.0, 0.0, False),
    (2, 256, 4, 128, 256, True, 1.0, 0.0, False),
    (1, 300, 2, 128, 128, True, 1.0, 0.02, False),
    (2, 192, 2, 64, 64, True, 1.0, 0.02, False),
    (1, 256, 2, 64, 192, False, 1.0, 0.02, False),
    (1, 200, 3, 128, 128, True, 2.0, 0.02, False),
    (1, 128, 2, 128, 64, True, 1.0, 0.02, True),
    (1, 1000, 2, 128, 256, True, 1.0, 0.02, False),
    # head_k_dim 256 (one 128-column workgroup per head and value block)
    (1, 300, 2, 256, 256, True, 1.0, 0.02, False),
    (2, 128, 3, 256, 128, False, 2.0, 0.02, False),
    (1, 200, 1, 256, 512, True, 1.0, 0.0, False),
]


@pytest.mark.parametrize("case", CASES)
def test_mfma_fwd_matches_oracle(rng, case):
    B, S, H, K, V, gated, bs, sstd, split = case
    announce(f"mfma fwd {case}")
    args = gdn_inputs(rng, B, S, H, K, V, gated, bs, sstd, split)
    g_args = to_gpu(args, torch.bfloat16)
    y, s = run_mfma(g_args)
    y0, s0 = O.chunk_fwd(*as_oracle_inputs(g_args), chunk_len=64, dtype=np.float32)
    ey, es = rel_err(y, y0), rel_err(s, s0)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL and es < TOL


def test_mfma_fwd_in_place_state_fp32_y(rng):
    announce("mfma fwd in place, fp32 y")
    args = gdn_inputs(rng, 1, 256, 2, 128, 128, True, 1.0, 0.02)
    g_args = to_gpu(args, torch.bfloat16)
    ref_in = as_oracle_inputs(g_args)  # before the state buffer is overwritten
    y, s = run_mfma(g_args, y_dtype=torch.float32, in_place=True)
    y0, s0 = O.chunk_fwd(*ref_in, chunk_len=64, dtype=np.float32)
    assert rel_err(y, y0) < TOL and rel_err(s, s0) < TOL


def test_mfma_head_k_dim_256_fp32_y_in_place_and_chunk_len(rng):
    """head_k_dim 256: fp32 y with the state updated in place, and a request
    for chunk_len 128 served by the 64-token kernels, against the oracle's
    chunk forward at the requested length; the backward at this width takes
    the MFMA kernels under AUTO."""
    announce("mfma fwd head_k_dim 256: fp32 y in place, chunk_len 128")
    args = gdn_inputs(rng, 1, 260, 2, 256, 128, True, 1.0, 0.02)
    g_args = to_gpu(args, torch.bfloat16)
    ref_in = as_oracle_inputs(g_args)
    y, s = run_mfma(g_args, y_dtype=torch.float32, in_place=True)
    y0, s0 = O.chunk_fwd(*ref_in, chunk_len=64, dtype=np.float64)
    ey, es = rel_err(y, y0), rel_err(s, s0)
    print(f"  in place: rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL and es < TOL
    g_args = to_gpu(args, torch.bfloat16)
    q, k, v, e, w, g, s_in = g_args
    yb = torch.empty((1, 260, 2, 128), dtype=torch.bfloat16, device=DEV)
    s_out = torch.empty_like(s_in)
    a = pkg.abi.chunk_fwd_args(q, k, v, e, w, g, s_in, yb, s_out, 128, None)
    assert pkg.abi.lib().dn_chunk_fwd_algo(a) == MFMA
    pkg.abi.run_chunk_fwd(a)
    torch.cuda.synchronize()
    y0, s0 = O.chunk_fwd(*as_oracle_inputs(g_args), chunk_len=128, dtype=np.float64)
    ey, es = rel_err(np_of(yb), y0), rel_err(np_of(s_out), s0)
    print(f"  chunk_len 128: rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL and es < TOL
    dy = torch.zeros((1, 260, 2, 128), device=DEV)
    grads = (torch.empty(q.shape, device=DEV), torch.empty(k.shape, device=DEV),
             torch.empty(v.shape, device=DEV), torch.empty_like(e), torch.empty_like(w),
             torch.empty_like(g), torch.empty_like(s_in))
    b = pkg.abi.chunk_bwd_args(dy, None, q, k, v, e, w, g, s_in, grads, 64, None)
    assert pkg.abi.lib().dn_chunk_bwd_algo(b) == MFMA


def test_mfma_matches_generic_path(rng):
    """Both GPU algorithms on one bf16 input; generic is fp32 arithmetic."""
    announce("mfma vs generic")
    g_args = to_gpu(gdn_inputs(rng, 2, 512, 2, 128, 256, True, 1.0, 0.02), torch.bfloat16)
    y_m, s_m = run_mfma(g_args, y_dtype=torch.float32)
    q, k, v, e, w, g, s = g_args
    y_g, s_g = pkg.delta_chunk_recalculated(q, k, v, e, w, g, s, True, 64, None,
                                            algo=pkg.abi.DN_ALGO_GENERIC, y_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err(y_m, np_of(y_g)) < TOL and rel_err(s_m, np_of(s_g)) < TOL


def test_mfma_constant_keys_stay_bounded(rng):
    """src/delta/tests.rs:373-460 at chunk 64: the WY inverse of a constant-key
    chunk must stay exact (blocked substitution, never a series)."""
    announce("mfma constant keys")
    B, S, H, K, V = 1, 256, 2, 128, 64
    hold = lambda a: np.broadcast_to(a, (B, S, H, a.shape[-1])).copy()
    q = hold(l2(rng.standard_normal((B, 1, H, K))))
    k = hold(l2(rng.standard_normal((B, 1, H, K))))
    v = hold(rng.standard_normal((B, 1, H, V)))
    for beta in (0.9, 1.8):
        e = np.full((B, S, H, 1), beta)
        g = np.full((B, S, H, 1), -0.05)
        args = [q, k, v, e, e, g, np.zeros((B, H, K, V))]
        g_args = to_gpu(args, torch.bfloat16)
        y, s = run_mfma(g_args, y_dtype=torch.float32)
        assert np.isfinite(y).all()
        y0, s0 = O.recurrent(*as_oracle_inputs(g_args), dtype=np.float64)
        assert rel_err(y, y0) < TOL and rel_err(s, s0) < TOL


def test_other_shapes_take_the_generic_path(rng):
    """dk outside {64, 128}, or a per-channel forget gate at a chunk length
    other than 64, is served by the generic kernels under AUTO."""
    announce("mfma coverage")
    for K, L, gates in [(96, 64, "head"), (128, 32, "channel")]:
        if gates == "head":
            g_args = to_gpu(gdn_inputs(rng, 1, 100, 2, K, 64, True), torch.bfloat16)
        else:
            g_args = to_gpu(gdn2_inputs(rng, 1, 100, 2, K, 64, K, 64), torch.bfloat16)
        q, k, v, e, w, g, s = g_args
        y = torch.empty((1, 100, 2, 64), dtype=torch.bfloat16, device=DEV)
        a = pkg.abi.chunk_fwd_args(q, k, v, e, w, g, s, y, torch.empty_like(s), L, None)
        assert pkg.abi.lib().dn_chunk_fwd_algo(a) == pkg.abi.DN_ALGO_GENERIC


CHUNK_LEN_CASES = [
    # chunk_len, B, S, H, K, V, gated: any chunk length runs the MFMA kernels'
    # 64-token chunks when the forget gate is per head (or absent)
    (32, 2, 256, 2, 128, 256, True),
    (128, 1, 300, 2, 128, 128, True),
    (16, 1, 200, 2, 64, 64, False),
    (100, 2, 250, 2, 128, 128, True),
    (1, 1, 70, 2, 128, 64, True),
]


@pytest.mark.parametrize("case", CHUNK_LEN_CASES)
def test_mfma_serves_other_chunk_lengths(rng, case):
    """path.rs:15-19: the chunk length trades intra-chunk work against serial
    steps; the chunk form computes the token recurrence at any length. The
    MFMA path serves a request for chunk_len L (per-head gates) with its own
    64-token chunks: against the oracle's chunk forward at L itself, forward
    and all seven gradients, at the bf16 bar."""
    L, B, S, H, K, V, gated = case
    announce(f"mfma at chunk_len {L}: {case[1:]}")
    args = gdn_inputs(rng, B, S, H, K, V, gated, state_std=0.02)
    g_args = to_gpu(args, torch.bfloat16)
    q, k, v, e, w, g, s = g_args
    y = torch.empty((B, S, H, V), dtype=torch.float32, device=DEV)
    s_out = torch.empty_like(s)
    a = pkg.abi.chunk_fwd_args(q, k, v, e, w, g, s, y, s_out, L, None)
    assert pkg.abi.lib().dn_chunk_fwd_algo(a) == MFMA
    pkg.abi.run_chunk_fwd(a)
    torch.cuda.synchronize()
    ref = as_oracle_inputs(g_args)
    y0, s0 = O.chunk_fwd(*ref, chunk_len=L, dtype=np.float64)
    ey, es = rel_err(np_of(y), y0), rel_err(np_of(s_out), s0)
    print(f"  forward rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL and es < TOL
    dy = rng.standard_normal((B, S, H, V))
    ds = rng.standard_normal((B, H, K, V)) * 0.5
    tdy = torch.tensor(dy, dtype=torch.float32, device=DEV)
    tds = torch.tensor(ds, dtype=torch.float32, device=DEV)
    grads = (torch.empty(q.shape, device=DEV), torch.empty(k.shape, device=DEV),
             torch.empty(v.shape, device=DEV), torch.empty_like(e), torch.empty_like(w),
             None if g is None else torch.empty_like(g), torch.empty_like(s))
    assert pkg.abi.lib().dn_chunk_bwd_algo(
        pkg.abi.chunk_bwd_args(tdy, tds, q, k, v, e, w, g, s, grads, L, None)) == MFMA
    got = pkg.combined_backward(tdy, tds, q, k, v, e, w, g, s, L, 1.0 / np.sqrt(K))
    torch.cuda.synchronize()
    want = O.chunk_bwd(dy, ds, *ref, chunk_len=L)
    names = ["d_q", "d_k", "d_v", "d_erase", "d_write", "d_g", "d_state"]
    vals = [got.d_q_bshk, got.d_k_bshk, got.d_v_bshv, got.d_erase_bshK, got.d_write_bshV,
            got.d_g_bshK, got.d_state_bhkv]
    for name, a_, b in zip(names, vals, want):
        if b is None:
            assert a_ is None
            continue
        err = rel_err(np_of(a_), b)
        print(f"  {name} rel err {err:.2e}", flush=True)
        assert err < TOL, name


def gdn2_inputs(rng, B, S, H, K, V, ew, ww, state_std=0.0, g_scale=0.05, beta_scale=1.0):
    """Config-5 distributions: per-key-channel erase b and decay α = e^g, per-value-channel
    write w (widths ew, ww; 1 means one value per head)."""
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    e = beta_scale / (1.0 + np.exp(-rng.standard_normal((B, S, H, ew))))
    w = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, ww))))
    g = -np.log1p(np.exp(rng.standard_normal((B, S, H, K)))) * g_scale
    s0 = rng.normal(0.0, state_std, (B, H, K, V)) if state_std else np.zeros((B, H, K, V))
    return [q, k, v, e, w, g, s0]


PC_CASES = [
    # B, S, H, K, V, ew, ww, state_std, g_scale
    (1, 64, 1, 128, 64, 128, 64, 0.0, 0.05),
    (2, 256, 2, 128, 128, 128, 128, 0.02, 0.05),
    (1, 300, 2, 128, 128, 128, 128, 0.02, 0.05),
    (1, 192, 2, 128, 64, 1, 64, 0.02, 0.05),
    (1, 200, 2, 128, 128, 128, 1, 0.02, 0.05),
    (1, 256, 2, 128, 128, 128, 128, 0.02, 1.0),
    (2, 130, 2, 64, 64, 64, 64, 0.05, 0.1),
    (1, 100, 2, 64, 64, 1, 1, 0.02, 0.05),
]


@pytest.mark.parametrize("case", PC_CASES)
def test_mfma_fwd_channel_gates_match_oracle(rng, case):
    """GDN-2 gate widths on the MFMA path (block-decay scores, kg/qg tiles)."""
    B, S, H, K, V, ew, ww, sstd, gs = case
    announce(f"mfma fwd per-channel {case}")
    g_args = to_gpu(gdn2_inputs(rng, B, S, H, K, V, ew, ww, sstd, gs), torch.bfloat16)
    y, s = run_mfma(g_args)
    y0, s0 = O.chunk_fwd(*as_oracle_inputs(g_args), chunk_len=64, dtype=np.float64)
    ey, es = rel_err(y, y0), rel_err(s, s0)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL and es < TOL


HD_CASES = [
    # B, S, H, K, V, ew, ww, forget gate ("head" | None), g scale: per-channel
    # erase or write gates beside a per-head (or no) forget gate, on the
    # per-channel kernels with the head mask
    (1, 256, 2, 128, 128, 128, 128, "head", 0.05),
    (2, 200, 2, 128, 256, 128, 1, "head", 0.05),
    (1, 130, 2, 64, 64, 1, 64, "head", 0.05),
    (1, 192, 2, 128, 128, 128, 128, None, 0.0),
    # decay of ~8 nats per token: the block decay's clamp would bind here, the
    # head mask is exact (the reference runs head_decay_mask for these widths)
    (1, 128, 2, 128, 64, 128, 64, "head", 8.0),
]


@pytest.mark.parametrize("case", HD_CASES)
def test_mfma_fwd_channel_write_gates_head_decay(rng, case):
    """WriteGate::Channel blocks (erase [.., dk], write [.., dv]) with a
    per-head forget gate: AUTO runs MFMA, against the oracle."""
    B, S, H, K, V, ew, ww, decay, gs = case
    announce(f"mfma fwd channel gates, head decay {case}")
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    e = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, ew))))
    w = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, ww))))
    g = None
    if decay == "head":
        g = (-np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * gs if gs < 1
             else np.full((B, S, H, 1), -gs))
    s0 = rng.normal(0.0, 0.02, (B, H, K, V))
    g_args = to_gpu([q, k, v, e, w, g, s0], torch.bfloat16)
    y, s = run_mfma(g_args)
    y0, s0r = O.chunk_fwd(*as_oracle_inputs(g_args), chunk_len=64, dtype=np.float64)
    ey, es = rel_err(y, y0), rel_err(s, s0r)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL and es < TOL
    # The backward for these widths runs the generic kernels under AUTO.
    qq, kk, vv, ee, ww_, gg, ss = g_args
    grads = tuple(torch.empty_like(x) if x is not None else None
                  for x in (qq, kk, vv, ee, ww_, gg, ss))
    a = pkg.abi.chunk_bwd_args(torch.zeros((B, S, H, V), device=DEV), None, qq, kk, vv, ee, ww_,
                               gg, ss, grads, 64, None)
    assert pkg.abi.lib().dn_chunk_bwd_algo(a) == pkg.abi.DN_ALGO_GENERIC


def test_mfma_channel_gates_constant_keys(rng):
    """Constant keys with β up to 1.8 per channel: the cancelling retrieval
    and the WY inverse stay within the bar (kg and S carry lo parts)."""
    announce("mfma per-channel constant keys")
    B, S, H, K, V = 1, 256, 2, 128, 64
    hold = lambda a: np.broadcast_to(a, (B, S, H, a.shape[-1])).copy()
    q = hold(l2(rng.standard_normal((B, 1, H, K))))
    k = hold(l2(rng.standard_normal((B, 1, H, K))))
    v = hold(rng.standard_normal((B, 1, H, V)))
    e = hold(1.8 / (1.0 + np.exp(-rng.standard_normal((B, 1, H, K)))))
    w = hold(1.0 / (1.0 + np.exp(-rng.standard_normal((B, 1, H, V)))))
    g = hold(-np.log1p(np.exp(rng.standard_normal((B, 1, H, K)))) * 0.05)
    g_args = to_gpu([q, k, v, e, w, g, np.zeros((B, H, K, V))], torch.bfloat16)
    y, s = run_mfma(g_args, y_dtype=torch.float32)
    assert np.isfinite(y).all()
    y0, s0 = O.recurrent(*as_oracle_inputs(g_args), dtype=np.float64)
    ey, es = rel_err(y, y0), rel_err(s, s0)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL and es < TOL


# ---------------------------------------------------------------------------
# Backward with the MFMA scans (bf16 q/k/v): all seven gradients
# ---------------------------------------------------------------------------

BWD_CASES = [
    # B, S, H, K, V, gates: None (ungated) | "head" | (ew, ww) with a per-channel decay
    (1, 256, 2, 128, 128, "head"),
    (2, 200, 2, 128, 64, "head"),
    (1, 192, 2, 64, 128, None),
    (1, 256, 2, 128, 128, (128, 128)),
    (1, 130, 2, 128, 64, (1, 64)),
    (2, 128, 2, 64, 64, (64, 1)),
    (1, 100, 2, 64, 128, (1, 128)),
    # a repeated key in every chunk (the retrieval cancels), β ∈ (0, 2)
    (1, 256, 2, 128, 128, "head", {"const_keys": True}),
    (1, 256, 2, 128, 128, (128, 128), {"const_keys": True}),
    (1, 192, 2, 128, 128, "head", {"beta_scale": 2.0}),
    # head_v_dim a multiple of 128 above 128: the chunk-local kernel in passes
    # of 128 value columns, the value-summed gradients added across them, and
    # (per-head gates) dattn and dT handed to the last pass, which runs the
    # score backward once
    (1, 128, 2, 128, 256, "head"),
    (1, 150, 2, 64, 256, "head"),
    (1, 128, 2, 64, 384, None),
    (1, 200, 2, 128, 256, (128, 256)),
    (1, 130, 2, 128, 256, (1, 1)),
    (1, 192, 2, 128, 384, "head"),
    (1, 96, 2, 64, 512, "head"),  # two middle passes, each adding to the handed-on sums
    (1, 128, 2, 128, 256, None),
    (1, 256, 2, 128, 256, "head", {"const_keys": True}),
    # an odd multiple of 64 above 128: passes of 128 columns and a last of 64
    (1, 128, 2, 128, 192, "head"),
    (1, 130, 2, 128, 192, (128, 192)),
    (1, 100, 2, 64, 320, "head"),  # 128, 128 (a middle pass), then 64
    (1, 96, 2, 128, 192, None),
    (1, 128, 2, 64, 192, (1, 1)),
    # head_k_dim 256 (per-head gates): each value pass as two launches over
    # the halves of the key channels, d_g and d_erase summed across them
    (1, 128, 2, 256, 128, "head"),
    (1, 200, 2, 256, 128, None),
    (1, 192, 2, 256, 128, "head", {"beta_scale": 2.0}),
    (1, 256, 2, 256, 128, "head", {"const_keys": True}),
    (1, 128, 2, 256, 256, "head"),
    (1, 130, 2, 256, 256, None),
    (1, 150, 2, 256, 384, "head"),  # a middle value pass
]


@pytest.mark.parametrize("algo", [MFMA, pkg.abi.DN_ALGO_GENERIC])
def test_channel_decay_clamp_closed_form(algo):
    """The per-channel decay where its clamp binds (decay.rs:41-49,
    combined_backward.rs:480-496), forward and backward on the MFMA and
    generic kernels, against the closed forms of conftest.clamp_regime_case
    (also the oracle's, tests/test_oracle_invariants.py). Relative 2e-2 on
    the MFMA path (bf16 operands), 1e-5 on the fp32 generic path; every
    other entry below 1e-3 of the smallest expected one."""
    announce(f"channel decay clamp closed form, algo {algo}")
    args, dy, want = clamp_regime_case()
    q, k, v, e, w, g, s = to_gpu(args, torch.bfloat16)
    V = v.shape[3]
    y = torch.empty(v.shape, dtype=torch.float32, device=DEV)
    s_out = torch.empty_like(s)
    a = pkg.abi.chunk_fwd_args(q, k, v, e, w, g, s, y, s_out, 64, None, algo=algo)
    assert pkg.abi.lib().dn_chunk_fwd_algo(a) == algo
    pkg.abi.run_chunk_fwd(a)
    torch.cuda.synchronize()
    tol = TOL if algo == MFMA else 1e-5
    rel, rest = closed_form_err(np_of(y), want["y"])
    print(f"  y rel {rel:.2e} rest {rest:.2e}", flush=True)
    assert rel < tol and rest < 1e-3
    assert np_of(s_out).max() == 0.0 and np_of(s_out).min() == 0.0
    tdy = torch.tensor(dy, dtype=torch.float32, device=DEV)
    grads = pkg.combined_backward(tdy, torch.zeros_like(s), q, k, v, e, w, g, s, 64,
                                  1.0 / np.sqrt(q.shape[3]), algo=algo)
    torch.cuda.synchronize()
    got = dict(zip(["d_q", "d_k", "d_v", "d_erase", "d_write", "d_g"],
                   [grads.d_q_bshk, grads.d_k_bshk, grads.d_v_bshv, grads.d_erase_bshK,
                    grads.d_write_bshV, grads.d_g_bshK]))
    for name, t in got.items():
        rel, rest = closed_form_err(np_of(t), want[name])
        print(f"  {name} rel {rel:.2e} rest {rest:.2e}", flush=True)
        assert rel < tol and rest < 1e-3, name


def bwd_inputs(rng, B, S, H, K, V, gates, opts=None):
    opts = opts or {}
    beta_scale = opts.get("beta_scale", 1.0)
    if gates is None or gates == "head":
        args = gdn_inputs(rng, B, S, H, K, V, gated=gates == "head", state_std=0.05,
                          beta_scale=beta_scale)
    else:
        args = gdn2_inputs(rng, B, S, H, K, V, gates[0], gates[1], state_std=0.05,
                           beta_scale=beta_scale)
    if opts.get("const_keys"):
        args[1] = np.repeat(args[1][:, :1], S, axis=1)
    dy = rng.standard_normal((B, S, H, V))
    ds = rng.standard_normal((B, H, K, V)) * 0.5
    return args, dy, ds


@pytest.mark.parametrize("case", BWD_CASES)
@pytest.mark.parametrize("dy_dtype", [torch.float32, torch.bfloat16])
def test_mfma_bwd_matches_oracle(rng, case, dy_dtype):
    B, S, H, K, V, gates = case[:6]
    announce(f"mfma bwd {case} dy {dy_dtype}")
    args, dy, ds = bwd_inputs(rng, B, S, H, K, V, gates, case[6] if len(case) > 6 else None)
    g_args = to_gpu(args, torch.bfloat16)
    tdy = torch.tensor(dy, dtype=torch.float32, device=DEV).to(dy_dtype)
    tds = torch.tensor(ds, dtype=torch.float32, device=DEV)
    q, k, v, e, w, g, s = g_args
    grads = pkg.combined_backward(tdy, tds, q, k, v, e, w, g, s, 64, 1.0 / np.sqrt(K))
    torch.cuda.synchronize()
    want = O.chunk_bwd(np_of(tdy), ds, *as_oracle_inputs(g_args), chunk_len=64)
    names = ["d_q", "d_k", "d_v", "d_erase", "d_write", "d_g", "d_state"]
    vals = [grads.d_q_bshk, grads.d_k_bshk, grads.d_v_bshv, grads.d_erase_bshK,
            grads.d_write_bshV, grads.d_g_bshK, grads.d_state_bhkv]
    for name, a, b in zip(names, vals, want):
        if b is None:
            assert a is None
            continue
        err = rel_err(np_of(a), b)
        print(f"  {name} rel err {err:.2e}", flush=True)
        assert err < TOL, name


@pytest.mark.parametrize("V,gates", [(128, "head"), (256, None)])
def test_mfma_bwd_head_k_dim_256_is_chosen(rng, V, gates):
    """AUTO runs the MFMA backward at head_k_dim 256 with per-head gates
    (the generic fp32 kernels before: 103 ms at the config-2 shape)."""
    announce(f"mfma bwd head_k_dim 256 chosen V={V} gates={gates}")
    args, dy, ds = bwd_inputs(rng, 1, 128, 2, 256, V, gates)
    q, k, v, e, w, g, s = to_gpu(args, torch.bfloat16)
    tdy = torch.tensor(dy, dtype=torch.float32, device=DEV)
    tds = torch.tensor(ds, dtype=torch.float32, device=DEV)
    grads = (torch.empty(q.shape, device=DEV), torch.empty(k.shape, device=DEV),
             torch.empty(v.shape, device=DEV), torch.empty_like(e), torch.empty_like(w),
             torch.empty_like(g) if g is not None else None, torch.empty_like(s))
    a = pkg.abi.chunk_bwd_args(tdy, tds, q, k, v, e, w, g, s, grads, 64, None)
    assert pkg.abi.lib().dn_chunk_bwd_algo(a) == MFMA


def test_mfma_bwd_is_chosen_and_matches_generic(rng):
    announce("mfma bwd vs generic")
    B, S, H, K, V = 1, 256, 2, 128, 128
    args, dy, ds = bwd_inputs(rng, B, S, H, K, V, "head")
    g_args = to_gpu(args, torch.bfloat16)
    q, k, v, e, w, g, s = g_args
    tdy = torch.tensor(dy, dtype=torch.float32, device=DEV)
    tds = torch.tensor(ds, dtype=torch.float32, device=DEV)
    grads = (torch.empty(q.shape, device=DEV), torch.empty(k.shape, device=DEV),
             torch.empty(v.shape, device=DEV), torch.empty_like(e), torch.empty_like(w),
             torch.empty_like(g), torch.empty_like(s))
    a = pkg.abi.chunk_bwd_args(tdy, tds, q, k, v, e, w, g, s, grads, 64, None)
    assert pkg.abi.lib().dn_chunk_bwd_algo(a) == MFMA
    out = {}
    for algo in (MFMA, pkg.abi.DN_ALGO_GENERIC):
        got = pkg.combined_backward(tdy, tds, q, k, v, e, w, g, s, 64, 1.0 / np.sqrt(K),
                                    algo=algo)
        torch.cuda.synchronize()
        out[algo] = [np_of(x) for x in (got.d_q_bshk, got.d_k_bshk, got.d_v_bshv,
                                         got.d_erase_bshK, got.d_write_bshV, got.d_g_bshK,
                                         got.d_state_bhkv)]
    for m, gnr in zip(out[MFMA], out[pkg.abi.DN_ALGO_GENERIC]):
        assert rel_err(m, gnr) < TOL


@pytest.mark.parametrize("V,gates", [(256, "head"), (192, "head"), (192, (128, 192))])
def test_mfma_chunk_local_backward_runs_in_value_passes(rng, V, gates):
    """head_v_dim 256 runs the MFMA chunk-local kernel (two 128-column passes
    under one profiler scope), not the generic one; 192 likewise, as a pass of
    128 columns and one of 64."""
    announce(f"mfma bwd, dv {V} {gates}: kernels")
    args, dy, ds = bwd_inputs(rng, 1, 128, 2, 128, V, gates)
    q, k, v, e, w, g, s = to_gpu(args, torch.bfloat16)
    tdy = torch.tensor(dy, dtype=torch.float32, device=DEV).to(torch.bfloat16)
    tds = torch.tensor(ds, dtype=torch.float32, device=DEV)
    torch.cuda.synchronize()
    pkg.abi.profile_enable(True)
    pkg.combined_backward(tdy, tds, q, k, v, e, w, g, s, 64, 1.0 / np.sqrt(128))
    torch.cuda.synchronize()
    prof = pkg.abi.profile_read()
    pkg.abi.profile_enable(False)
    assert "dn_mfma_chunk_bwd" in prof, prof
    assert not any(n.startswith("dn_generic") for n in prof), prof
