"""dn_frontend_chunk_fwd: QkvProjection::forward (qkv.rs:373-449) followed by
the chunk forward on its outputs (chunk_recalculated.rs:115-151), as the
families run them (gated_deltanet_1.rs:162-177).

Where the MFMA path applies (per-head gates, head_k_dim 128, conv 4 with the
default SiLU, bf16),
the front-end's q/k half runs in the intra kernel's load stage, with
dn_frontend's lane layout and order of operations: every output (y, the
final state, q, k, v, the gates and the next conv window) must equal
dn_frontend followed by dn_chunk_fwd bit for bit. Against the oracle
composition (oracle/frontend.py's frontend, then the oracle's chunk forward
in float64 on the bf16 values the GPU reads) at the bf16 bar, 2e-2. Shapes
outside the fused path run the two calls, checked the same way."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from gpu_util import DEV, announce, np_of, pkg
from oracle import frontend as F
from oracle import oracle as O

pytestmark = pytest.mark.gpu

abi = pkg.abi
TOL = 2e-2

CASES = [
    # B, S, H, dk, dv, conv_act, qk_act, qk_norm, gate, bias, gated, chunk, extra, window_scale
    (2, 300, 2, 128, 256, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False, True,
     64, 6, 0.0),                                  # partial last chunk, zero window
    (1, 256, 4, 128, 128, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, True, True,
     64, 36, 1.0),                                 # bias, a carried window, extra columns
    (1, 256, 4, 128, 128, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, True, True,
     64, 37, 1.0),                                 # rows off 16 bytes: the two calls
    (2, 50, 2, 128, 256, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_FIXED, False, False,
     64, 0, 1.0),                                  # one partial chunk, ungated, fixed β
    (1, 200, 2, 128, 128, F.ACT_IDENTITY, F.ACT_RELU, F.QKNORM_L2, F.WRITE_SCALAR, True,
     True, 32, 14, 1.0),                           # unfused activations: the two calls
    (1, 130, 2, 128, 128, F.ACT_SILU, F.ACT_SILU, F.QKNORM_NONE, F.WRITE_SCALAR, False,
     True, 64, 6, 1.0),                            # no q/k norm
    (2, 100, 2, 64, 64, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False, True,
     64, 0, 1.0),                                  # head_k_dim 64: the two calls
    (1, 96, 2, 128, 128, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_CHANNEL, False, True,
     64, 0, 1.0),                                  # per-channel gates: the two calls
]


def width_of(case):
    (B, S, H, dk, dv, cact, qact, qn, gate, bias, gated, L, extra, wscale) = case
    return F.conv_dim(H, dk, dv, 1) + F.gate_width(H, dk, dv, 1, gate) + extra


def make(rng, case):
    (B, S, H, dk, dv, cact, qact, qn, gate, bias, gated, L, extra, wscale) = case
    cd = F.conv_dim(H, dk, dv, 1)
    width = width_of(case)
    bf = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV).to(torch.bfloat16)
    # Without the q/k norm, keys of unit-scale entries make β·K·Kᵀ entries of
    # order dk and (I + A)⁻¹ overflow: that case takes small projections.
    pscale = 1.0 if qn == F.QKNORM_L2 else 0.05
    proj = bf(rng.standard_normal((B, S, width)) * pscale)
    w = torch.tensor(rng.standard_normal((cd, 4)) * 0.5, dtype=torch.float32, device=DEV)
    b = (torch.tensor(rng.standard_normal(cd) * 0.1, dtype=torch.float32, device=DEV)
         if bias else None)
    win = bf(rng.standard_normal((B, cd, 4)) * wscale)
    g = (torch.tensor(-np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * 0.05,
                      dtype=torch.float32, device=DEV) if gated else None)
    s0 = torch.tensor(rng.normal(0.0, 0.02, (B, H, dk, dv)), dtype=torch.float32, device=DEV)
    return proj, w, b, win, g, s0


def outputs(B, S, H, dk, dv, gate):
    q = torch.empty((B, S, H, dk), dtype=torch.bfloat16, device=DEV)
    k = torch.empty_like(q)
    v = torch.empty((B, S, H, dv), dtype=torch.bfloat16, device=DEV)
    if gate == F.WRITE_CHANNEL:
        e = torch.empty((B, S, H, dk), device=DEV)
        wr = torch.empty((B, S, H, dv), device=DEV)
    else:
        e = torch.empty((B, S, H, 1), device=DEV)
        wr = e
    y = torch.empty((B, S, H, dv), dtype=torch.bfloat16, device=DEV)
    return dict(q=q, k=k, v=v, erase=e, write=wr, y=y)


def run(case, inputs, fused, win_out=None):
    (B, S, H, dk, dv, cact, qact, qn, gate, bias, gated, L, extra, wscale) = case
    proj, w, b, win, g, s0 = inputs
    o = outputs(B, S, H, dk, dv, gate)
    o["window"] = torch.empty_like(win) if win_out is None else win_out
    o["state"] = torch.empty_like(s0)
    fe = abi.frontend_args(proj, w, b, win, o["window"], o["q"], o["k"], o["v"], o["erase"],
                           o["write"], nheads=H, head_k_dim=dk, head_v_dim=dv, n_householder=1,
                           conv_activation=cact, qk_activation=qact, qk_norm=qn,
                           write_gate=gate, allow_neg_eigval=False)
    fwd = abi.chunk_fwd_args(o["q"], o["k"], o["v"], o["erase"], o["write"], g, s0, o["y"],
                             o["state"], L, None)
    if fused:
        a = abi.frontend_chunk_fwd_args(fe, fwd)
        ws = torch.empty(max(abi.lib().dn_frontend_chunk_fwd_workspace_bytes(a), 1),
                         dtype=torch.uint8, device=DEV)
        a.fwd.workspace, a.fwd.workspace_bytes = ws.data_ptr(), ws.numel()
        abi.run_frontend_chunk_fwd(a)
    else:
        abi.run_frontend(fe)
        abi.run_chunk_fwd(fwd)
    torch.cuda.synchronize()
    return o


@pytest.mark.parametrize("case", CASES)
def test_frontend_chunk_fwd_equals_the_two_calls(rng, case):
    announce(f"dn_frontend_chunk_fwd {case}")
    inputs = make(rng, case)
    abi.profile_enable(True)
    got = run(case, inputs, True)
    prof = abi.profile_read()
    abi.profile_enable(False)
    # The fused path: head_k_dim 128, per-head gates, the default activations
    # (SiLU in the conv, fused with the q/k one), projection rows on 16 bytes.
    fusable = (case[3] == 128 and case[8] != F.WRITE_CHANNEL and width_of(case) % 8 == 0 and
               case[5] == F.ACT_SILU and case[6] == F.ACT_SILU)
    assert ("dn_mfma_intra_fe" in prof) == fusable, prof
    want = run(case, inputs, False)
    for name in ["q", "k", "v", "erase", "write", "window", "y", "state"]:
        assert torch.equal(got[name], want[name]), name


@pytest.mark.parametrize("case", CASES[:6])
def test_frontend_chunk_fwd_matches_oracle(rng, case):
    (B, S, H, dk, dv, cact, qact, qn, gate, bias, gated, L, extra, wscale) = case
    announce(f"dn_frontend_chunk_fwd vs oracle {case}")
    inputs = make(rng, case)
    proj, w, b, win, g, s0 = inputs
    got = run(case, inputs, True)
    d = lambda t: None if t is None else t.double().cpu().numpy()
    fe = F.frontend(d(proj), nheads=H, head_k_dim=dk, head_v_dim=dv, n_householder=1,
                    conv=dict(weight=d(w), bias=d(b), window=d(win), activation=cact),
                    qk_activation=qact, qk_norm_kind=qn, write_gate=gate,
                    allow_neg_eigval=False)
    # The chunk forward's oracle on the bf16 q/k/v the GPU path reads.
    rbf = lambda a: torch.tensor(a, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    y0, s1 = O.chunk_fwd(rbf(fe["q"]), rbf(fe["k"]), rbf(fe["v"]), fe["erase"], fe["write"],
                         d(g), d(s0), chunk_len=L, dtype=np.float64)
    for name, want in [("q", fe["q"]), ("k", fe["k"]), ("v", fe["v"]), ("y", y0), ("state", s1)]:
        err = rel_err(np_of(got[name]), want)
        print(f"  {name}: rel err {err:.2e}", flush=True)
        assert err < TOL, name
    assert np.array_equal(np_of(got["window"]).astype(np.float64), fe["window"])


def test_frontend_chunk_fwd_window_in_place(rng):
    """window_out aliasing window_in (the cache updated in place): the intra
    kernel reads the old window before the next one is written."""
    case = CASES[1]
    announce("dn_frontend_chunk_fwd, window in place")
    inputs = make(rng, case)
    win = inputs[3]
    want = run(case, inputs, False)
    alias = win.clone()
    got = run(case, inputs[:3] + (alias,) + inputs[4:], True, win_out=alias)
    for name in ["q", "k", "y", "state", "window"]:
        assert torch.equal(got[name], want[name]), name


def test_frontend_chunk_fwd_config2_shape(rng):
    """BASELINE config 2's shape (B=8, T=4096, H=16, dk=128, dv=256) with the
    reference's default front-end (conv 4 with SiLU, L2 norm, scalar β): the
    fused call equals the two calls bit for bit."""
    case = (8, 4096, 16, 128, 256, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR,
            False, True, 64, 0, 1.0)
    announce("dn_frontend_chunk_fwd at the config-2 shape")
    inputs = make(rng, case)
    got = run(case, inputs, True)
    want = run(case, inputs, False)
    for name in ["q", "k", "v", "erase", "window", "y", "state"]:
        assert torch.equal(got[name], want[name]), name
