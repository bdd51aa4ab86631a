"""dn_block_step, one decode token of a delta-rule block in one launch,
against the same token through the three separate calls it fuses: the
front-end's step (dn_frontend, QkvProjection::step, qkv.rs:454-516),
delta_step (dn_step, recurrent.rs:41-99) and the output norm (dn_out_norm,
norm.rs:127-134), each pinned against the oracle by its own tests. The fused
path keeps q, k, v and y in fp32 between the stages, so the bar is the
composition with fp32 intermediates at 1e-5 normwise; the next conv window
must match bit for bit (it is the projection's values, moved). The fused
step also meets the oracle's own composition (oracle/frontend.py's
front-end, the C++ oracle's delta_step, oracle/frontend.py's out_norm) in
float64 at 1e-4. A chain of
decode tokens must match the block's forward over the sequence (the forward
≡ step contract of gated_deltanet_1/tests.rs:61-155) at 1e-4 absolute."""

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, pkg
from oracle import frontend as F
from oracle import oracle as O

pytestmark = pytest.mark.gpu

abi = pkg.abi
A = pkg.QkActivation
WG = pkg.WriteGate


def rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def make_block(rng, H, dk, dv, *, conv_k=4, conv_act=pkg.ConvActivation.SILU, conv_bias=False,
               qk_act=A.SILU, qk_norm=pkg.QkNorm.L2, write_gate=WG.SCALAR, neg=False,
               gated=True):
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)
    proj = pkg.QkvProjection(nheads=H, head_k_dim=dk, head_v_dim=dv, qk_activation=qk_act,
                             qk_norm=qk_norm, write_gate=write_gate, has_gate=gated,
                             allow_neg_eigval=neg)
    if conv_k:
        proj.conv = pkg.ShortConv(t(rng.standard_normal((proj.conv_dim(), conv_k)) * 0.5),
                                  t(rng.standard_normal(proj.conv_dim()) * 0.1) if conv_bias
                                  else None, conv_act)
    norm = pkg.OutNorm(t(1.0 + 0.1 * rng.standard_normal(dv)), gated=gated, eps=1e-5)
    return proj, norm


def three_calls(proj, norm, p, win, g, s, scale):
    """The same token through dn_frontend (fp32 outputs), dn_step, dn_out_norm."""
    st, win2 = proj.step_projected(p, win, out_dtype=torch.float32)
    y, s2 = pkg.delta_step(st.q_bhk, st.k_buhk[:, 0].contiguous(), st.v_buhv[:, 0].contiguous(),
                           st.erase_buhK[:, 0].contiguous(), st.write_buhV[:, 0].contiguous(),
                           g, s, scale)
    gate = None if st.gate_bhv is None else st.gate_bhv
    return norm.forward(y, gate, out_dtype=torch.float32), win2, s2, y


CASES = [
    # id, B, H, dk, dv, block options, input dtype, decay width (0: no forget gate)
    ("config3-like", 3, 2, 128, 256, {}, torch.float32, 1),
    ("channel-gates", 2, 3, 64, 128, dict(write_gate=WG.CHANNEL, neg=True, conv_k=3),
     torch.bfloat16, "K"),
    ("plain", 2, 2, 32, 48, dict(conv_k=0, write_gate=WG.FIXED, gated=False, qk_act=A.RELU,
                                 qk_norm=pkg.QkNorm.NONE), torch.float32, 0),
    ("wide-odd", 1, 2, 200, 200, dict(conv_bias=True, qk_act=A.ELU_PLUS_ONE), torch.float32, 1),
    ("unfused-silu", 2, 1, 16, 64, dict(conv_k=2, conv_act=pkg.ConvActivation.IDENTITY),
     torch.bfloat16, 1),
    ("k256", 1, 1, 256, 256, dict(write_gate=WG.CHANNEL), torch.float32, "K"),
]


def case_inputs(rng, B, H, dk, dv, opts, in_dtype, dw):
    proj, norm = make_block(rng, H, dk, dv, **opts)
    p = torch.tensor(rng.standard_normal((B, proj.d_in_proj())), dtype=torch.float32,
                     device=DEV).to(in_dtype)
    win = None
    if proj.conv is not None:
        win = torch.tensor(rng.standard_normal((B, proj.conv_dim(), proj.conv_kernel())),
                           dtype=torch.float32, device=DEV).to(in_dtype)
    width = dk if dw == "K" else dw
    g = None if width == 0 else torch.tensor(
        -np.log1p(np.exp(rng.standard_normal((B, H, width)))) * 0.1, dtype=torch.float32,
        device=DEV)
    s = torch.tensor(rng.standard_normal((B, H, dk, dv)) * 0.1, dtype=torch.float32, device=DEV)
    return proj, norm, p, win, g, s


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_block_step_equals_the_three_calls(rng, case):
    name, B, H, dk, dv, opts, in_dtype, dw = case
    announce(f"block step {name}")
    proj, norm, p, win, g, s = case_inputs(rng, B, H, dk, dv, opts, in_dtype, dw)
    scale = 1.0 / np.sqrt(dk)
    want_out, want_win, want_s, want_y = three_calls(proj, norm, p, win, g, s, scale)
    out, win2, s2, y = pkg.block_step(proj, norm, p, win, g, s, scale, out_dtype=torch.float32,
                                      return_y=True)
    torch.cuda.synchronize()
    e = (rel(out, want_out), rel(s2, want_s), rel(y, want_y))
    print(f"  out {e[0]:.2e} state {e[1]:.2e} y {e[2]:.2e}", flush=True)
    assert torch.isfinite(out).all()
    assert max(e) < 1e-5
    if win is not None:
        assert torch.equal(win2, want_win.to(win2.dtype))


def oracle_block_step(proj, norm, p, win, g, s, scale):
    """The same token through the oracle's composition, in float64: the
    front-end's forward over a one-token sequence (oracle/frontend.py,
    QkvProjection::step ≡ forward on one token, qkv.rs:454-516), delta_step
    (oracle.cpp, recurrent.rs:41-99), then OutNorm::forward (norm.rs:106-144)
    with the output gate read from the projection row after the write
    gates (qkv.rs:237-262)."""
    npf = lambda t: None if t is None else t.double().cpu().numpy()
    H, dk, dv = proj.nheads, proj.head_k_dim, proj.head_v_dim
    pn = npf(p)
    conv = None
    if proj.conv is not None:
        conv = dict(weight=npf(proj.conv.weight), bias=npf(proj.conv.bias), window=npf(win),
                    activation=int(proj.conv.activation))
    fr = F.frontend(pn[:, None], nheads=H, head_k_dim=dk, head_v_dim=dv, conv=conv,
                    qk_activation=int(proj.qk_activation), qk_norm_kind=int(proj.qk_norm),
                    write_gate=int(proj.write_gate), allow_neg_eigval=proj.allow_neg_eigval)
    y, s2 = O.delta_step(fr["q"][:, 0], fr["k"][:, 0], fr["v"][:, 0], fr["erase"][:, 0],
                         fr["write"][:, 0], npf(g), npf(s), scale=scale)
    gate = None
    if norm.gated:
        g0 = F.conv_dim(H, dk, dv, 1) + F.gate_width(H, dk, dv, 1, int(proj.write_gate))
        gate = pn[:, g0:g0 + H * dv].reshape(-1, H, dv)
    out = F.out_norm(y, gate, npf(norm.weight), norm.eps)
    return out, fr["window"], s2, y


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_block_step_matches_the_oracle_composition(rng, case):
    """dn_block_step straight against the oracle's front-end step, delta_step
    and output norm (float64), at 1e-4 normwise: its stages keep fp32
    intermediates, so the difference is fp32 rounding."""
    name, B, H, dk, dv, opts, in_dtype, dw = case
    announce(f"block step vs oracle composition: {name}")
    proj, norm, p, win, g, s = case_inputs(rng, B, H, dk, dv, opts, in_dtype, dw)
    scale = 1.0 / np.sqrt(dk)
    out, win2, s2, y = pkg.block_step(proj, norm, p, win, g, s, scale, out_dtype=torch.float32,
                                      return_y=True)
    torch.cuda.synchronize()
    w_out, w_win, w_s, w_y = oracle_block_step(proj, norm, p, win, g, s, scale)
    npd = lambda t: t.double().cpu().numpy()
    re = lambda a, b: float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))
    e = (re(npd(out), w_out), re(npd(s2), w_s), re(npd(y), w_y))
    print(f"  out {e[0]:.2e} state {e[1]:.2e} y {e[2]:.2e}", flush=True)
    assert max(e) < 1e-4
    if win is not None:
        assert np.array_equal(npd(win2), w_win)


def test_block_step_bf16_out_and_in_place(rng):
    announce("block step bf16 out, in place")
    proj, norm, p, win, g, s = case_inputs(rng, 4, 4, 128, 256, {}, torch.bfloat16, 1)
    out_f, win_f, s_f = pkg.block_step(proj, norm, p, win, g, s, out_dtype=torch.float32)
    s_in, w_in = s.clone(), win.clone()
    out_b, win_b, s_b = pkg.block_step(proj, norm, p, w_in, g, s_in, out_dtype=torch.bfloat16,
                                       in_place=True)
    torch.cuda.synchronize()
    assert s_b.data_ptr() == s_in.data_ptr() and win_b.data_ptr() == w_in.data_ptr()
    assert torch.equal(s_b, s_f) and torch.equal(win_b, win_f)
    assert torch.equal(out_b, out_f.to(torch.bfloat16))


def test_block_step_chain_matches_the_block_forward(rng):
    """forward ≡ step (gated_deltanet_1/tests.rs:61-155): eight decode tokens
    through dn_block_step against the sequence through dn_frontend, the
    recurrent path and dn_out_norm."""
    announce("block step chain vs block forward")
    B, S, H, dk, dv = 2, 8, 2, 64, 128
    proj, norm = make_block(rng, H, dk, dv)
    p = torch.tensor(rng.standard_normal((B, S, proj.d_in_proj())), dtype=torch.float32,
                     device=DEV)
    g = torch.tensor(-np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * 0.1,
                     dtype=torch.float32, device=DEV)
    s0 = torch.zeros((B, H, dk, dv), device=DEV)
    win0 = proj.zero_conv_window(B, DEV)
    qkv, win_f = proj.forward_projected(p, win0)
    y, s_f = pkg.DeltaInput(qkv.q_bshk, qkv.k_bShk, qkv.v_bShv, qkv.erase_bShK, qkv.write_bShV,
                            g, s0).run(pkg.DeltaPath.recurrent())
    out_f = norm.forward(y, qkv.gate_bshv)
    s, win, outs = s0.clone(), win0.clone(), []
    for t in range(S):
        o, win, s = pkg.block_step(proj, norm, p[:, t].contiguous(), win, g[:, t].contiguous(), s,
                                   in_place=True)
        outs.append(o)
    torch.cuda.synchronize()
    assert (out_f - torch.stack(outs, 1)).abs().max().item() < 1e-4
    assert (s_f - s).abs().max().item() < 1e-4
    assert torch.equal(win, win_f)


def test_block_step_refuses_what_it_does_not_serve(rng):
    announce("block step refusals")
    proj, norm = make_block(rng, 2, 16, 64)
    proj.n_householder = 2
    with pytest.raises(pkg.DeltaError, match="n_householder"):
        pkg.block_step(proj, norm, torch.zeros(1, proj.d_in_proj(), device=DEV),
                       proj.zero_conv_window(1, DEV), None, torch.zeros(1, 2, 16, 64, device=DEV))
    proj, norm = make_block(rng, 1, 16, 130)
    with pytest.raises(pkg.DeltaError, match="multiple of 4"):
        pkg.block_step(proj, norm, torch.zeros(1, proj.d_in_proj(), device=DEV),
                       proj.zero_conv_window(1, DEV), None, torch.zeros(1, 1, 16, 130, device=DEV))


def test_block_step_check_finite(rng):
    announce("block step check_finite")
    proj, norm, p, win, g, s = case_inputs(rng, 2, 2, 32, 64, {}, torch.float32, 1)
    p[1, 3] = float("nan")
    with pytest.raises(pkg.DeltaError, match="NaN or Inf"):
        pkg.block_step(proj, norm, p, win, g, s, check_finite=True)
