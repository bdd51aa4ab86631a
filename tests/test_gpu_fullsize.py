"""BASELINE's own shapes on the GPU, checked through properties that hold at
any size (the CPU oracle would take hours at these sizes; it pins the same
kernels at small sizes in the other GPU tests):

- config 2 (B=8, T=4096, H=16, dk=128, dv=256, bf16 q/k/v): a sequence split
  at a chunk boundary and carried through the returned fp32 state gives the
  same bits as one call, since the scan walks the chunks in order from an
  fp32 state. The MFMA chunk path agrees with `dn_recurrent`, an independent
  kernel that walks the tokens one by one: both arms of `DeltaPath`
  (path.rs:215-231) compute one recurrence.
- config 3 (decode: batch 256, H=16, dk=128, dv=256, fp32 state): 1000
  consecutive `dn_step` calls agree with the chunk forward over the same
  1000 tokens (the config's own check), and one step is affine in the state:
  f(S1 + S2) = f(S1) + f(S2) − f(0), for the next state and for y.
- config 4 (DeltaProduct u = 2 fold) and config 5 (GDN-2 per-channel gates):
  the MFMA forward, and for config 5 the MFMA backward, agree with the
  generic fp32 kernels, which share no code with them (so does the backward
  at the config-2 shape, head_v_dim 256 in two value passes); the MFMA forward
  also agrees with `dn_recurrent`, the token-by-token recurrence.
- the projection front-end at the config-2 shape: a sequence split in two,
  with the conv window carried across (conv.rs:14-20), gives the same bits
  as one call. The output norm at config 2's output shape agrees with its
  formula restated in torch fp32 (norm.rs:106-144).

Bars: bit-exact where the arithmetic is the same, 1e-4 relative between fp32
paths and for the affine identity, and 2e-2 (the bf16-input bar) across the
MFMA and fp32 paths."""

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, pkg

pytestmark = pytest.mark.gpu

GENERIC, MFMA = pkg.abi.DN_ALGO_GENERIC, pkg.abi.DN_ALGO_MFMA
TOL_BF16, TOL_F32 = 2e-2, 1e-4


def rel_err(a, b):
    """Normwise relative error max|a − b| / max|b| (b is the reference), on the GPU."""
    a, b = a.float(), b.float()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def gen(seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


def l2(x):
    return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def gdn_inputs(gr, B, T, H, K, V, dtype, g_scale=0.05):
    """Config-2 distributions: q, k L2(N(0,1)); v N(0,1); β = σ(N(0,1)); g = −softplus(N)·g_scale."""
    q = l2(torch.randn((B, T, H, K), generator=gr, device=DEV)).to(dtype)
    k = l2(torch.randn((B, T, H, K), generator=gr, device=DEV)).to(dtype)
    v = torch.randn((B, T, H, V), generator=gr, device=DEV).to(dtype)
    beta = torch.sigmoid(torch.randn((B, T, H, 1), generator=gr, device=DEV))
    g = -torch.nn.functional.softplus(torch.randn((B, T, H, 1), generator=gr, device=DEV)) * g_scale
    return q, k, v, beta, g


def chunk(q, k, v, e, w, g, s, algo=pkg.abi.DN_ALGO_AUTO):
    return pkg.delta_chunk_recalculated(q, k, v, e, w, g, s, g is not None, 64,
                                        1.0 / np.sqrt(q.shape[3]), algo=algo)


def test_config2_split_call_is_bit_exact():
    announce("config 2 full size: split at a chunk boundary vs one call")
    B, T, H, K, V = 8, 4096, 16, 128, 256
    q, k, v, beta, g = gdn_inputs(gen(2), B, T, H, K, V, torch.bfloat16)
    s0 = torch.zeros((B, H, K, V), device=DEV)
    assert pkg.abi.lib().dn_chunk_fwd_algo(pkg.abi.chunk_fwd_args(
        q, k, v, beta, beta, g, s0, torch.empty((B, T, H, V), dtype=torch.bfloat16, device=DEV),
        torch.empty_like(s0), 64, None)) == MFMA
    y, s = chunk(q, k, v, beta, beta, g, s0)
    half = T // 2
    cut = lambda x, a, b: x[:, a:b].contiguous()
    y1, s1 = chunk(cut(q, 0, half), cut(k, 0, half), cut(v, 0, half), cut(beta, 0, half),
                   cut(beta, 0, half), cut(g, 0, half), s0)
    y2, s2 = chunk(cut(q, half, T), cut(k, half, T), cut(v, half, T), cut(beta, half, T),
                   cut(beta, half, T), cut(g, half, T), s1)
    torch.cuda.synchronize()
    assert torch.equal(y[:, :half], y1)
    assert torch.equal(y[:, half:], y2)
    assert torch.equal(s, s2)


def test_config2_chunk_path_agrees_with_recurrent_kernel():
    announce("config 2 full size: MFMA chunk path vs dn_recurrent")
    B, T, H, K, V = 8, 4096, 16, 128, 256
    q, k, v, beta, g = gdn_inputs(gen(3), B, T, H, K, V, torch.bfloat16)
    s0 = torch.zeros((B, H, K, V), device=DEV)
    y, s = chunk(q, k, v, beta, beta, g, s0)
    yr, sr = pkg.DeltaInput(q, k, v, beta, beta, g, s0).delta_recurrent()
    torch.cuda.synchronize()
    ey, es = rel_err(y, yr), rel_err(s, sr)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL_BF16 and es < TOL_BF16


def decode_inputs(gr, Bd, T, H, K, V):
    q, k, v, beta, _ = gdn_inputs(gr, Bd, T, H, K, V, torch.float32)
    # α = exp(−softplus(N)·0.05) per (token, head), passed as the log-decay g.
    g = -torch.nn.functional.softplus(torch.randn((Bd, T, H, 1), generator=gr, device=DEV)) * 0.05
    return q, k, v, beta, g


def test_config3_step_chain_agrees_with_chunk_forward():
    """BASELINE config 3's own check: 1000 consecutive in-place dn_step calls
    on a 1000-token sequence, every y row and the final state compared with
    the chunk forward over the same tokens from the same S0 (fp32 inputs, so
    the chunk forward runs the generic fp32 kernels)."""
    Bd, H, K, V, T = 256, 16, 128, 256, 1000
    announce(f"config 3 full size: {T} dn_step calls vs the chunk forward")
    gr = gen(4)
    q, k, v, beta, g = decode_inputs(gr, Bd, T, H, K, V)
    s0 = torch.randn((Bd, H, K, V), generator=gr, device=DEV) * 0.02
    y_c, s_c = chunk(q, k, v, beta, beta, g, s0)
    s = s0.clone()
    y_steps = torch.empty_like(y_c)
    at = lambda x, t: x[:, t].contiguous()
    scale = 1.0 / np.sqrt(K)
    for t in range(T):
        yt, s = pkg.delta_step(at(q, t), at(k, t), at(v, t), at(beta, t), at(beta, t), at(g, t),
                               s, scale, in_place=True)
        y_steps[:, t] = yt
    torch.cuda.synchronize()
    ey = rel_err(y_steps, y_c)
    es = rel_err(s, s_c)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL_F32 and es < TOL_F32


def test_config3_step_is_affine_in_the_state():
    announce("config 3 full size: f(S1 + S2) = f(S1) + f(S2) - f(0)")
    Bd, H, K, V = 256, 16, 128, 256
    gr = gen(5)
    q, k, v, beta, g = (x[:, 0].contiguous() for x in decode_inputs(gr, Bd, 1, H, K, V))
    s1 = torch.randn((Bd, H, K, V), generator=gr, device=DEV) * 0.02
    s2 = torch.randn((Bd, H, K, V), generator=gr, device=DEV) * 0.02
    f = lambda s: pkg.delta_step(q, k, v, beta, beta, g, s, 1.0 / np.sqrt(K))
    y12, n12 = f(s1 + s2)
    ya, na = f(s1)
    yb, nb = f(s2)
    y0, n0 = f(torch.zeros_like(s1))
    torch.cuda.synchronize()
    ey = rel_err(ya + yb - y0, y12)
    es = rel_err(na + nb - n0, n12)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL_F32 and es < TOL_F32


def test_config4_mfma_forward_agrees_with_generic():
    announce("config 4 full size: DeltaProduct u=2 fold, MFMA vs generic forward")
    B, T, u, H, K, V = 4, 8192, 2, 16, 128, 128
    S = T * u
    gr = gen(6)
    q = torch.zeros((B, T, u, H, K), device=DEV)
    q[:, :, u - 1] = l2(torch.randn((B, T, H, K), generator=gr, device=DEV))
    q = q.reshape(B, S, H, K).to(torch.bfloat16)
    k = l2(torch.randn((B, S, H, K), generator=gr, device=DEV)).to(torch.bfloat16)
    v = torch.randn((B, S, H, V), generator=gr, device=DEV).to(torch.bfloat16)
    beta = 2 * torch.sigmoid(torch.randn((B, S, H, 1), generator=gr, device=DEV))
    g = torch.zeros((B, T, u, H, 1), device=DEV)
    # BASELINE config 4 draws g as config 1 does: −softplus(N(0,1))·0.1.
    g[:, :, 0] = -torch.nn.functional.softplus(
        torch.randn((B, T, H, 1), generator=gr, device=DEV)) * 0.1
    g = g.reshape(B, S, H, 1)
    s0 = torch.zeros((B, H, K, V), device=DEV)
    y_m, s_m = chunk(q, k, v, beta, beta, g, s0, algo=MFMA)
    y_g, s_g = chunk(q, k, v, beta, beta, g, s0, algo=GENERIC)
    torch.cuda.synchronize()
    ey, es = rel_err(y_m, y_g), rel_err(s_m, s_g)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL_BF16 and es < TOL_BF16
    del y_g, s_g
    # An independent algorithm: the token-by-token recurrence (dn_recurrent).
    y_r, s_r = pkg.DeltaInput(q, k, v, beta, beta, g, s0).delta_recurrent()
    torch.cuda.synchronize()
    ey, es = rel_err(y_m, y_r), rel_err(s_m, s_r)
    print(f"  vs dn_recurrent: rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL_BF16 and es < TOL_BF16


def test_config5_mfma_forward_and_backward_agree_with_generic():
    announce("config 5 full size: GDN-2 per-channel gates, MFMA vs generic, forward + backward")
    B, T, H, K, V = 2, 16384, 16, 128, 128
    gr = gen(7)
    q = l2(torch.randn((B, T, H, K), generator=gr, device=DEV)).to(torch.bfloat16)
    k = l2(torch.randn((B, T, H, K), generator=gr, device=DEV)).to(torch.bfloat16)
    v = torch.randn((B, T, H, V), generator=gr, device=DEV).to(torch.bfloat16)
    e = torch.sigmoid(torch.randn((B, T, H, K), generator=gr, device=DEV))
    w = torch.sigmoid(torch.randn((B, T, H, V), generator=gr, device=DEV))
    g = -torch.nn.functional.softplus(torch.randn((B, T, H, K), generator=gr, device=DEV)) * 0.05
    s0 = torch.zeros((B, H, K, V), device=DEV)
    y_m, s_m = chunk(q, k, v, e, w, g, s0, algo=MFMA)
    y_g, s_g = chunk(q, k, v, e, w, g, s0, algo=GENERIC)
    torch.cuda.synchronize()
    ey, es = rel_err(y_m, y_g), rel_err(s_m, s_g)
    print(f"  forward rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL_BF16 and es < TOL_BF16
    del y_g, s_g
    # An independent algorithm: the token-by-token recurrence (dn_recurrent).
    y_r, s_r = pkg.DeltaInput(q, k, v, e, w, g, s0).delta_recurrent()
    torch.cuda.synchronize()
    ey, es = rel_err(y_m, y_r), rel_err(s_m, s_r)
    print(f"  forward vs dn_recurrent: rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert ey < TOL_BF16 and es < TOL_BF16
    del y_m, s_m, y_r, s_r
    dy = torch.randn((B, T, H, V), generator=gr, device=DEV)
    ds = torch.randn((B, H, K, V), generator=gr, device=DEV) * 0.5
    scale = 1.0 / np.sqrt(K)
    got = {}
    for algo in (MFMA, GENERIC):
        r = pkg.combined_backward(dy, ds, q, k, v, e, w, g, s0, 64, scale, algo=algo)
        torch.cuda.synchronize()
        got[algo] = [x.clone() for x in (r.d_q_bshk, r.d_k_bshk, r.d_v_bshv, r.d_erase_bshK,
                                        r.d_write_bshV, r.d_g_bshK, r.d_state_bhkv)]
        del r
    for name, m, gn in zip(["dq", "dk", "dv", "d_erase", "d_write", "dg", "d_state"],
                           got[MFMA], got[GENERIC]):
        err = rel_err(m, gn)
        print(f"  backward {name} rel err {err:.2e}", flush=True)
        assert err < TOL_BF16, name


def test_config2_shape_mfma_backward_agrees_with_generic():
    """The backward at the config-2 shape (per-head gates, head_v_dim 256: the
    chunk-local kernel runs two value passes, the first handing its partial
    dattn and dT to the second) against the generic fp32 kernels, all seven
    gradients, with a nonzero initial state and final-state cotangent."""
    announce("config 2 shape: backward, MFMA (two value passes) vs generic")
    B, T, H, K, V = 8, 4096, 16, 128, 256
    gr = gen(10)
    q, k, v, beta, g = gdn_inputs(gr, B, T, H, K, V, torch.bfloat16)
    s0 = torch.randn((B, H, K, V), generator=gr, device=DEV) * 0.02
    dy = torch.randn((B, T, H, V), generator=gr, device=DEV).to(torch.bfloat16)
    ds = torch.randn((B, H, K, V), generator=gr, device=DEV) * 0.5
    scale = 1.0 / np.sqrt(K)
    got = {}
    for algo in (MFMA, GENERIC):
        r = pkg.combined_backward(dy, ds, q, k, v, beta, beta, g, s0, 64, scale, algo=algo)
        torch.cuda.synchronize()
        got[algo] = [x.clone() for x in (r.d_q_bshk, r.d_k_bshk, r.d_v_bshv, r.d_erase_bshK,
                                        r.d_write_bshV, r.d_g_bshK, r.d_state_bhkv)]
        del r
    for name, m, gn in zip(["dq", "dk", "dv", "d_erase", "d_write", "dg", "d_state"],
                           got[MFMA], got[GENERIC]):
        err = rel_err(m, gn)
        print(f"  backward {name} rel err {err:.2e}", flush=True)
        assert err < TOL_BF16, name


def test_frontend_split_with_carried_window_is_bit_exact():
    announce("dn_frontend at the config-2 shape: two halves with the window carried vs one call")
    abi = pkg.abi
    B, T, H, K, V, KC = 8, 4096, 16, 128, 256, 4
    gr = gen(8)
    conv_dim = H * K * 2 + H * V
    width = conv_dim + H
    proj = torch.randn((B, T, width), generator=gr, device=DEV).to(torch.bfloat16)
    weight = torch.randn((conv_dim, KC), generator=gr, device=DEV) * 0.5
    win0 = torch.randn((B, conv_dim, KC), generator=gr, device=DEV).to(torch.bfloat16)

    def run(p, win):
        S = p.shape[1]
        q = torch.empty((B, S, H, K), dtype=torch.bfloat16, device=DEV)
        k, v = torch.empty_like(q), torch.empty((B, S, H, V), dtype=torch.bfloat16, device=DEV)
        beta = torch.empty((B, S, H, 1), device=DEV)
        wout = torch.empty_like(win)
        abi.run_frontend(abi.frontend_args(
            p, weight, None, win, wout, q, k, v, beta, beta, nheads=H, head_k_dim=K,
            head_v_dim=V, n_householder=1, conv_activation=abi.DN_ACT_SILU,
            qk_activation=abi.DN_ACT_SILU, qk_norm=abi.DN_QKNORM_L2,
            write_gate=abi.DN_WRITE_SCALAR, allow_neg_eigval=False))
        return (q, k, v, beta), wout

    full, wfull = run(proj, win0)
    half = T // 2
    a, wa = run(proj[:, :half].contiguous(), win0)
    b, wb = run(proj[:, half:].contiguous(), wa)
    torch.cuda.synchronize()
    for f, x, y in zip(full, a, b):
        assert torch.equal(f, torch.cat([x, y], 1))
    assert torch.equal(wfull, wb)


def test_out_norm_agrees_with_its_formula_in_fp32():
    announce("dn_out_norm at config 2's output shape vs torch fp32")
    abi = pkg.abi
    B, T, H, V = 8, 4096, 16, 256
    gr = gen(9)
    x = torch.randn((B, T, H, V), generator=gr, device=DEV).to(torch.bfloat16)
    gate = torch.randn((B, T, H, V), generator=gr, device=DEV).to(torch.bfloat16)
    w = 1.0 + 0.1 * torch.randn((V,), generator=gr, device=DEV)
    out = torch.empty_like(x)
    abi.run_out_norm(abi.out_norm_args(x, gate, w, out, 1e-5))
    xf, gf = x.float(), gate.float()
    want = xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + 1e-5) * w * (gf * torch.sigmoid(gf))
    torch.cuda.synchronize()
    err = rel_err(out, want)
    print(f"  rel err {err:.2e}", flush=True)
    assert err < 1e-2  # bf16 output: a rounding of 2^-9 relative per element
