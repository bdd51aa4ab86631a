"""A delta-rule block assembled from this library's pieces keeps forward ≡
step, the reference's block contract (gated_deltanet_1/tests.rs:61-155,
delta_product/tests.rs:75-227): QkvProjection (in_proj as a library GEMM,
then dn_frontend), the delta rule (the chunk path, or dn_recurrent for a
DeltaProduct decode token's micro-steps), and OutNorm (dn_out_norm). The
forget gate is a synthetic log-decay tensor: the families' own gate
parameterisation lies outside the core. Bars: 1e-4 absolute on outputs and
caches in fp32, as the reference's test asserts."""

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, pkg

pytestmark = pytest.mark.gpu


def make_block(rng, d_model, H, dk, dv, u=1, neg=False):
    proj = pkg.QkvProjection(nheads=H, head_k_dim=dk, head_v_dim=dv, n_householder=u,
                             has_gate=True, allow_neg_eigval=neg)
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)
    proj.in_proj = t(rng.standard_normal((d_model, proj.d_in_proj())) / np.sqrt(d_model))
    proj.conv = pkg.ShortConv(t(rng.standard_normal((proj.conv_dim(), 4)) * 0.5))
    norm = pkg.OutNorm(t(1.0 + 0.1 * rng.standard_normal(dv)), gated=True, eps=1e-5)
    return proj, norm


def max_abs(a, b):
    return (a.float() - b.float()).abs().max().item()


@pytest.mark.parametrize("path", ["recurrent", 4, 64])
def test_gated_deltanet_block_forward_matches_step(rng, path):
    announce(f"block forward vs step, path {path}")
    B, S, D, H, dk, dv = 2, 10, 48, 2, 16, 32
    proj, norm = make_block(rng, D, H, dk, dv)
    x = torch.tensor(rng.standard_normal((B, S, D)), dtype=torch.float32, device=DEV)
    g = torch.tensor(-np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * 0.1,
                     dtype=torch.float32, device=DEV)
    s0 = torch.zeros((B, H, dk, dv), device=DEV)
    win0 = proj.zero_conv_window(B, DEV)
    # forward over the sequence
    qkv, win_f = proj.forward(x, win0)
    P = pkg.DeltaPath.recurrent() if path == "recurrent" else pkg.DeltaPath.with_chunk_len(path)
    y, s_f = pkg.DeltaInput(qkv.q_bshk, qkv.k_bShk, qkv.v_bShv, qkv.erase_bShK, qkv.write_bShV,
                            g, s0).run(P)
    out_f = norm.forward(y, qkv.gate_bshv)
    # token by token
    s, win, outs = s0.clone(), win0, []
    for t in range(S):
        st, win = proj.step(x[:, t].contiguous(), win)
        yt, s = pkg.delta_step(st.q_bhk, st.k_buhk[:, 0].contiguous(), st.v_buhv[:, 0].contiguous(),
                               st.erase_buhK[:, 0].contiguous(), st.write_buhV[:, 0].contiguous(),
                               g[:, t].contiguous(), s, 1.0 / np.sqrt(dk))
        outs.append(norm.forward(yt, st.gate_bhv))
    torch.cuda.synchronize()
    assert max_abs(out_f, torch.stack(outs, 1)) < 1e-4
    assert max_abs(s_f, s) < 1e-4
    # The window holds raw projections: the sequence's one GEMM and the
    # per-token GEMMs may round differently, so caches compare at the bar too.
    assert max_abs(win_f, win) < 1e-4


def test_deltaproduct_block_forward_matches_decode(rng):
    """DeltaProduct, u = 2 with allow_neg_eigval: forward folds the micro-steps
    into the sequence (q on the last, the forget gate on the first,
    delta_product.rs:178-205) and runs the chunk path; decode runs each
    token's two micro-steps as one dn_recurrent call (delta_product.rs:270-303)."""
    announce("DeltaProduct block forward vs decode")
    B, S, D, H, dk, dv, u = 2, 9, 48, 2, 16, 32, 2
    proj, norm = make_block(rng, D, H, dk, dv, u=u, neg=True)
    x = torch.tensor(rng.standard_normal((B, S, D)), dtype=torch.float32, device=DEV)
    g_tok = torch.tensor(-np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * 0.1,
                         dtype=torch.float32, device=DEV)
    s0 = torch.zeros((B, H, dk, dv), device=DEV)
    win0 = proj.zero_conv_window(B, DEV)
    qkv, win_f = proj.forward(x, win0)
    # The fold: q only on the last micro-step of a token, g only on the first.
    q_f = torch.zeros((B, S, u, H, dk), device=DEV)
    q_f[:, :, u - 1] = qkv.q_bshk
    g_f = torch.zeros((B, S, u, H, 1), device=DEV)
    g_f[:, :, 0] = g_tok
    y, s_f = pkg.DeltaInput(q_f.reshape(B, S * u, H, dk), qkv.k_bShk, qkv.v_bShv,
                            qkv.erase_bShK, qkv.write_bShV, g_f.reshape(B, S * u, H, 1),
                            s0).run(pkg.DeltaPath.with_chunk_len(8))
    out_f = norm.forward(y.reshape(B, S, u, H, dv)[:, :, u - 1].contiguous(), qkv.gate_bshv)
    s, win, outs = s0.clone(), win0, []
    for t in range(S):
        st, win = proj.step(x[:, t].contiguous(), win)
        q_u = torch.zeros((B, u, H, dk), device=DEV)
        q_u[:, u - 1] = st.q_bhk
        g_u = torch.zeros((B, u, H, 1), device=DEV)
        g_u[:, 0] = g_tok[:, t]
        yu, s = pkg.DeltaInput(q_u, st.k_buhk, st.v_buhv, st.erase_buhK, st.write_buhV, g_u,
                               s).run(pkg.DeltaPath.recurrent())
        outs.append(norm.forward(yu[:, u - 1].contiguous(), st.gate_bhv))
    torch.cuda.synchronize()
    assert max_abs(out_f, torch.stack(outs, 1)) < 1e-4
    assert max_abs(s_f, s) < 1e-4
    # The window holds raw projections: the sequence's one GEMM and the
    # per-token GEMMs may round differently, so caches compare at the bar too.
    assert max_abs(win_f, win) < 1e-4
