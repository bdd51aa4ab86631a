"""GPU parity of dn_frontend (the projection front-end, qkv.rs:373-516) with
the CPU oracle (oracle/frontend.py), through the C ABI and its Python mirror
QkvProjection.

Bars: normwise relative error 1e-5 for fp32 in and out (the arithmetic is a
handful of fp32 operations per element); 1e-2 where q, k, v are written in
bf16 (one rounding: 2⁻⁹ relative) — below the 2e-2 of BASELINE.json's
north_star for bf16 inputs. Gates are fp32 at 1e-5 in every case. The next
conv window is compared exactly (it is a copy of inputs)."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from gpu_util import DEV, announce, np_of, pkg
from oracle import frontend as F

pytestmark = pytest.mark.gpu

abi = pkg.abi

CASES = [
    # B, S, H, dk, dv, u, K, conv_act, qk_act, qk_norm, gate, neg, bias, in, out, extra
    (2, 37, 4, 128, 256, 1, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False,
     False, torch.bfloat16, torch.bfloat16, 0),
    (2, 40, 2, 64, 64, 1, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False,
     True, torch.float32, torch.float32, 0),
    (1, 33, 2, 128, 128, 2, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_CHANNEL, True,
     False, torch.float32, torch.float32, 5),
    (2, 19, 3, 32, 48, 1, 3, F.ACT_IDENTITY, F.ACT_RELU, F.QKNORM_L2, F.WRITE_FIXED, True,
     True, torch.float32, torch.float32, 0),
    (1, 21, 2, 16, 16, 1, 0, F.ACT_SILU, F.ACT_ELU_PLUS_ONE, F.QKNORM_NONE, F.WRITE_SCALAR,
     True, False, torch.float32, torch.float32, 3),
    (2, 18, 2, 100, 36, 1, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_CHANNEL, False,
     True, torch.float32, torch.float32, 0),
    (1, 25, 2, 64, 64, 1, 6, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False,
     True, torch.float32, torch.float32, 0),
    (1, 9, 2, 64, 64, 1, 1, F.ACT_SILU, F.ACT_IDENTITY, F.QKNORM_L2, F.WRITE_SCALAR, False,
     False, torch.float32, torch.float32, 0),
    (2, 5, 1, 4, 6, 3, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_CHANNEL, True,
     True, torch.float32, torch.float32, 0),
    (2, 30, 2, 256, 128, 1, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False,
     False, torch.bfloat16, torch.float32, 0),
    (2, 2, 2, 64, 64, 1, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False,
     False, torch.float32, torch.float32, 0),
    # short sequences (decode steps) take the row-per-token kernel
    (3, 1, 4, 128, 256, 1, 4, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False,
     False, torch.bfloat16, torch.bfloat16, 0),
    (2, 3, 2, 64, 128, 2, 4, F.ACT_IDENTITY, F.ACT_RELU, F.QKNORM_L2, F.WRITE_CHANNEL, True,
     True, torch.float32, torch.float32, 0),
    (4, 16, 2, 32, 32, 1, 6, F.ACT_SILU, F.ACT_SILU, F.QKNORM_L2, F.WRITE_SCALAR, False,
     True, torch.float32, torch.bfloat16, 2),
]


def make_case(rng, case):
    (B, S, H, dk, dv, u, K, cact, qact, qn, gate, neg, bias, din, dout, extra) = case
    cd = F.conv_dim(H, dk, dv, u)
    width = cd + F.gate_width(H, dk, dv, u, gate) + extra
    # The oracle sees the values the GPU sees: inputs rounded to their dtype.
    rd = lambda a, d: torch.tensor(a, dtype=torch.float32).to(d).double().numpy()
    p = rd(rng.standard_normal((B, S, width)), din)
    conv = None
    if K:
        w = rd(rng.standard_normal((cd, K)) * 0.5, torch.float32)
        window = rd(rng.standard_normal((B, cd, K)), din)
        conv = dict(weight=w, bias=rd(rng.standard_normal(cd) * 0.1, torch.float32)
                    if bias else None, window=window, activation=cact)
    return p, conv


def oracle_of(p, conv, case):
    (B, S, H, dk, dv, u, K, cact, qact, qn, gate, neg, *_rest) = case
    return F.frontend(p, nheads=H, head_k_dim=dk, head_v_dim=dv, n_householder=u, conv=conv,
                      qk_activation=qact, qk_norm_kind=qn, write_gate=gate,
                      allow_neg_eigval=neg)


def run_abi(p, conv, case, alias_window=False):
    (B, S, H, dk, dv, u, K, cact, qact, qn, gate, neg, bias, din, dout, extra) = case
    t = lambda a, d=torch.float32: torch.tensor(a, dtype=torch.float32, device=DEV).to(d)
    gp = t(p, din)
    q = torch.empty((B, S, H, dk), dtype=dout, device=DEV)
    k = torch.empty((B, S * u, H, dk), dtype=dout, device=DEV)
    v = torch.empty((B, S * u, H, dv), dtype=dout, device=DEV)
    if gate == F.WRITE_CHANNEL:
        e = torch.empty((B, S * u, H, dk), device=DEV)
        w = torch.empty((B, S * u, H, dv), device=DEV)
    else:
        e = torch.empty((B, S * u, H, 1), device=DEV)
        w = torch.empty_like(e)
    weight = bias_t = win_in = win_out = None
    if conv is not None:
        weight = t(conv["weight"])
        bias_t = None if conv["bias"] is None else t(conv["bias"])
        win_in = t(conv["window"], din)
        win_out = win_in if alias_window else torch.empty_like(win_in)
    abi.run_frontend(abi.frontend_args(
        gp, weight, bias_t, win_in, win_out, q, k, v, e, w, nheads=H, head_k_dim=dk,
        head_v_dim=dv, n_householder=u, conv_activation=cact if K else F.ACT_IDENTITY,
        qk_activation=qact, qk_norm=qn, write_gate=gate, allow_neg_eigval=neg))
    torch.cuda.synchronize()
    return dict(q=q, k=k, v=v, erase=e, write=w, window=win_out)


def check(got, want, dout):
    tol = 1e-5 if dout == torch.float32 else 1e-2
    for name in ["q", "k", "v"]:
        err = rel_err(np_of(got[name]), want[name])
        assert err < tol, f"{name}: rel err {err:.2e}"
    for name in ["erase", "write"]:
        err = rel_err(np_of(got[name]), want[name])
        assert err < 1e-5, f"{name}: rel err {err:.2e}"
    if want["window"] is not None:
        assert np.array_equal(np_of(got["window"]).astype(np.float64), want["window"])


@pytest.mark.parametrize("case", CASES)
def test_frontend_matches_oracle(rng, case):
    announce(f"dn_frontend {case[:12]}")
    p, conv = make_case(rng, case)
    check(run_abi(p, conv, case), oracle_of(p, conv, case), case[14])


@pytest.mark.parametrize("ci", [1, 11, 12])
def test_frontend_window_in_place(rng, ci):
    """window_out aliasing window_in (the decode cache updated in place): a
    sequence, a one-token step (whose kernel writes the next window itself)
    and a 3-token call. Case 11 (B = 3, one token) is the regression case
    for the row kernel's padded rows: its workgroup holds 16 (batch, token)
    rows over four waves, 13 of them padded onto the last real row, and only
    real rows may write the window (a padded row in another wave could read
    the window after the real row replaced it and write it shifted twice)."""
    case = CASES[ci]
    announce(f"dn_frontend in-place window, case {ci}")
    p, conv = make_case(rng, case)
    want = oracle_of(p, conv, case)
    check(run_abi(p, conv, case, alias_window=True), want, case[14])


def test_step_chain_equals_forward(rng):
    """QkvProjection.step token by token, carrying the window, equals one
    forward over the sequence (the reference's forward/step parity)."""
    announce("QkvProjection step chain")
    B, S, H, dk, dv = 2, 6, 2, 64, 128
    proj = pkg.QkvProjection(nheads=H, head_k_dim=dk, head_v_dim=dv, has_gate=True,
                             extra_channels=4)
    cd = proj.conv_dim()
    proj.conv = pkg.ShortConv(torch.tensor(rng.standard_normal((cd, 4)) * 0.5,
                                           dtype=torch.float32, device=DEV))
    p = torch.tensor(rng.standard_normal((B, S, proj.d_in_proj())), dtype=torch.float32,
                     device=DEV)
    win0 = torch.tensor(rng.standard_normal((B, cd, 4)), dtype=torch.float32, device=DEV)
    full, wfull = proj.forward_projected(p, win0)
    win = win0
    for t in range(S):
        st, win = proj.step_projected(p[:, t].contiguous(), win)
        assert rel_err(np_of(st.q_bhk), np_of(full.q_bshk[:, t])) < 1e-6
        assert rel_err(np_of(st.k_buhk[:, 0]), np_of(full.k_bShk[:, t])) < 1e-6
        assert rel_err(np_of(st.v_buhv[:, 0]), np_of(full.v_bShv[:, t])) < 1e-6
        assert torch.equal(st.erase_buhK[:, 0], full.erase_bShK[:, t])
        assert torch.equal(st.gate_bhv, full.gate_bshv[:, t])
    torch.cuda.synchronize()
    assert torch.equal(win, wfull)
    # The mirror's gate and extra views are the projection's own columns.
    c = cd + proj.write_gate_width()
    assert torch.equal(full.gate_bshv.reshape(B, S, -1), p[:, :, c:c + H * dv])
    assert torch.equal(full.extra_bsx, p[:, :, c + H * dv:])


def test_projection_forward_runs_in_proj(rng):
    """QkvProjection.forward = in_proj (a library GEMM) + dn_frontend."""
    announce("QkvProjection forward with in_proj")
    B, S, D, H, dk, dv = 2, 8, 48, 2, 32, 32
    proj = pkg.QkvProjection(nheads=H, head_k_dim=dk, head_v_dim=dv)
    cd = proj.conv_dim()
    wproj = rng.standard_normal((D, proj.d_in_proj())) * 0.2
    wconv = rng.standard_normal((cd, 4)) * 0.5
    proj.in_proj = torch.tensor(wproj, dtype=torch.float32, device=DEV)
    proj.conv = pkg.ShortConv(torch.tensor(wconv, dtype=torch.float32, device=DEV))
    x = rng.standard_normal((B, S, D))
    qkv, win = proj.forward(torch.tensor(x, dtype=torch.float32, device=DEV),
                            proj.zero_conv_window(B, DEV))
    want = F.frontend(x @ wproj, nheads=H, head_k_dim=dk, head_v_dim=dv,
                      conv=dict(weight=wconv, bias=None, window=np.zeros((B, cd, 4)),
                                activation=F.ACT_SILU))
    # The GEMM runs in fp32 on the GPU (rocBLAS/hipBLASLt order): 1e-4.
    assert rel_err(np_of(qkv.q_bshk), want["q"]) < 1e-4
    assert rel_err(np_of(qkv.k_bShk), want["k"]) < 1e-4
    assert rel_err(np_of(qkv.v_bShv), want["v"]) < 1e-4
    assert rel_err(np_of(qkv.erase_bShK), want["erase"]) < 1e-4
    assert qkv.write_bShV.data_ptr() == qkv.erase_bShK.data_ptr()


# ---------------------------------------------------------------------------
# dn_out_norm: OutNorm::forward (norm.rs:106-144)
# ---------------------------------------------------------------------------

NORM_CASES = [
    # tokens shape, H, D, gated, x dtype, out dtype, gate as a projection view
    ((2, 33), 4, 256, True, torch.bfloat16, torch.bfloat16, True),
    ((2, 17), 3, 128, True, torch.float32, torch.float32, False),
    ((5,), 16, 256, True, torch.float32, torch.bfloat16, True),
    ((3, 9), 2, 128, False, torch.float32, torch.float32, False),
    ((2, 7), 2, 100, True, torch.float32, torch.float32, True),
    ((1, 6), 3, 6, True, torch.float32, torch.float32, False),
    ((2, 4), 2, 512, True, torch.bfloat16, torch.float32, False),
]


@pytest.mark.parametrize("case", NORM_CASES)
def test_out_norm_matches_oracle(rng, case):
    lead, H, D, gated, dx, do, view = case
    announce(f"dn_out_norm {case}")
    rd = lambda a, d: torch.tensor(a, dtype=torch.float32).to(d).double().numpy()
    x = rd(rng.standard_normal((*lead, H, D)) * 2.0, dx)
    w = rd(rng.standard_normal(D), torch.float32)
    gx = torch.tensor(x, dtype=torch.float32, device=DEV).to(dx)
    gate = g_np = None
    if gated:
        g_np = rd(rng.standard_normal((*lead, H, D)), dx)
        if view:  # the gate as the projection's column range (qkv.rs:429)
            W = H * D + 37
            proj = torch.zeros((*lead, W), dtype=dx, device=DEV)
            proj[..., 5:5 + H * D] = torch.tensor(g_np, dtype=torch.float32,
                                                  device=DEV).to(dx).reshape(*lead, H * D)
            gate = proj[..., 5:5 + H * D].unflatten(-1, (H, D))
        else:
            gate = torch.tensor(g_np, dtype=torch.float32, device=DEV).to(dx)
    norm = pkg.OutNorm(torch.tensor(w, dtype=torch.float32, device=DEV), gated=gated, eps=1e-5)
    y = norm.forward(gx, gate, out_dtype=do)
    torch.cuda.synchronize()
    want = F.out_norm(x, g_np, w, 1e-5)
    tol = 1e-5 if do == torch.float32 else 1e-2
    assert rel_err(np_of(y), want) < tol


def test_out_norm_in_place(rng):
    """out may alias x."""
    announce("dn_out_norm in place")
    H, D = 4, 128
    x = rng.standard_normal((6, H, D))
    w = rng.standard_normal(D)
    g = rng.standard_normal((6, H, D))
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)
    gx, gg, gw = t(x), t(g), t(w)
    abi.run_out_norm(abi.out_norm_args(gx, gg, gw, gx, 1e-5))
    torch.cuda.synchronize()
    assert rel_err(np_of(gx), F.out_norm(x, g, w, 1e-5)) < 1e-5


def test_out_norm_gate_presence_mirrors_the_reference(rng):
    """norm.rs:131-132: a gated norm without a gate, or the reverse, panics."""
    x = torch.zeros((2, 2, 8), device=DEV)
    with pytest.raises(pkg.DeltaError, match="needs an output gate"):
        pkg.OutNorm.init(8, True, DEV).forward(x)
    with pytest.raises(pkg.DeltaError, match="takes no output gate"):
        pkg.OutNorm.init(8, False, DEV).forward(x, x)
