"""dn_chunk_fwd_out_norm: the chunk forward with OutNorm (norm.rs:106-144)
applied in the scan's output write, as the families run the two back to
back (gated_deltanet_1.rs:183-186).

Against the oracle's composition: the C++ oracle's chunk forward
(chunk_recalculated.rs:115-177) followed by oracle/frontend.py's out_norm,
in float64 on the bf16-rounded inputs the GPU reads, at the bf16 bar
(normwise 2e-2; bf16 output rounds each value to 2^-9), both with the norm
in the scan's output write (in_scan) and as a pass of its own. The cases
cover one
scan workgroup per head row and rows split over 2, 4 and 8 workgroups (whose
per-token sums cross workgroups mid-kernel), the segmented scan, per-head
and per-channel gates, the gated and plain norms, the gate as a strided
column view of a projection, fp32 gate and output, partial chunks, chunk
lengths other than 64, and the generic fallback; at BASELINE config 2's
shape the fused call against dn_chunk_fwd followed by dn_out_norm. Every
test ends with no cross-workgroup wait having given up."""

import numpy as np
import pytest
import torch

from conftest import l2, rel_err
from gpu_util import DEV, announce, as_oracle_inputs, np_of, pkg, to_gpu
from oracle import frontend as F
from oracle import oracle as O

pytestmark = pytest.mark.gpu

abi = pkg.abi
TOL = 2e-2


def inputs(rng, B, S, H, K, V, gates, state_std=0.02):
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    if gates == "channel":
        e = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, K))))
        w = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, V))))
        g = -np.log1p(np.exp(rng.standard_normal((B, S, H, K)))) * 0.05
    else:
        e = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, 1))))
        w = e
        g = -np.log1p(np.exp(rng.standard_normal((B, S, H, 1)))) * 0.05
    s0 = rng.normal(0.0, state_std, (B, H, K, V))
    return [q, k, v, e, w, g, s0]


def run_fused(g_args, gate, gamma, eps, y_dtype, chunk_len=64, in_scan=True):
    q, k, v, e, w, g, s = g_args
    B, S, H, _ = q.shape
    V = v.shape[3]
    y = torch.empty((B, S, H, V), dtype=y_dtype, device=DEV)
    s_out = torch.empty_like(s)
    fa = abi.chunk_fwd_args(q, k, v, e, w, g, s, y, s_out, chunk_len, None)
    na = abi.chunk_fwd_out_norm_args(fa, gate, gamma, eps, in_scan=in_scan)
    ws_bytes = abi.lib().dn_chunk_fwd_out_norm_workspace_bytes(na)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    na.fwd.workspace, na.fwd.workspace_bytes = ws.data_ptr(), ws.numel()
    abi.run_chunk_fwd_out_norm(na)
    torch.cuda.synchronize()
    return y, s_out


def oracle_of(g_args, gate, gamma, eps, chunk_len=64):
    ref = as_oracle_inputs(g_args)
    y0, s0 = O.chunk_fwd(*ref, chunk_len=chunk_len, dtype=np.float64)
    gt = None if gate is None else gate.double().cpu().numpy()
    return F.out_norm(y0, gt, gamma.double().cpu().numpy(), eps), s0


CASES = [
    # B, S, H, K, V, gates, gate form, y dtype, chunk_len
    (1, 256, 2, 128, 128, "head", "bf16", torch.bfloat16, 64),
    (2, 200, 2, 128, 256, "head", "bf16", torch.bfloat16, 64),   # partial last chunk
    (1, 64, 1, 64, 64, "head", "bf16", torch.bfloat16, 64),
    (1, 256, 2, 128, 128, "channel", "bf16", torch.bfloat16, 64),
    (2, 130, 3, 64, 128, "channel", "f32", torch.float32, 64),
    (1, 192, 2, 128, 256, "head", None, torch.bfloat16, 64),      # OutNorm::Plain
    (1, 300, 2, 128, 128, "head", "proj", torch.bfloat16, 64),    # gate: projection columns
    (1, 250, 2, 128, 256, "head", "bf16", torch.float32, 32),     # another chunk length
    (1, 4096, 2, 128, 128, "head", "bf16", torch.bfloat16, 64),   # segmented scan
    (1, 4096, 2, 128, 128, "channel", "bf16", torch.bfloat16, 64),
    (1, 4096, 2, 128, 256, "head", "bf16", torch.bfloat16, 64),   # segmented, rows split
]


def make_gate(rng, B, S, H, V, form):
    if form is None:
        return None, None
    if form == "proj":
        # The gate as the projection's column range: tokens W elements apart.
        W = H * V + 37 * 4
        proj = torch.tensor(rng.standard_normal((B, S, W)), dtype=torch.float32,
                            device=DEV).to(torch.bfloat16)
        return proj[:, :, 20 * 4:20 * 4 + H * V].unflatten(2, (H, V)), proj
    dt = torch.bfloat16 if form == "bf16" else torch.float32
    return torch.tensor(rng.standard_normal((B, S, H, V)), dtype=torch.float32,
                        device=DEV).to(dt), None


@pytest.mark.parametrize("in_scan", [True, False])
@pytest.mark.parametrize("case", CASES)
def test_fused_out_norm_matches_oracle(rng, case, in_scan):
    B, S, H, K, V, gates, form, y_dtype, L = case
    announce(f"chunk fwd + out norm {case}, in scan {in_scan}")
    g_args = to_gpu(inputs(rng, B, S, H, K, V, gates), torch.bfloat16)
    gate, keep = make_gate(rng, B, S, H, V, form)
    gamma = torch.tensor(1.0 + 0.1 * rng.standard_normal(V), dtype=torch.float32, device=DEV)
    y, s = run_fused(g_args, gate, gamma, 1e-5, y_dtype, L, in_scan)
    want_y, want_s = oracle_of(g_args, gate, gamma, 1e-5, L)
    ey, es = rel_err(np_of(y), want_y), rel_err(np_of(s), want_s)
    print(f"  rel err out {ey:.2e} state {es:.2e}", flush=True)
    assert np.isfinite(np_of(y)).all()
    assert ey < TOL and es < TOL
    assert abi.wait_give_ups() == 0


def test_generic_fallback_matches_oracle(rng):
    """fp32 q/k/v (outside the MFMA path): dn_chunk_fwd then dn_out_norm."""
    announce("chunk fwd + out norm, generic fallback")
    B, S, H, K, V = 1, 100, 2, 32, 48
    g_args = to_gpu(inputs(rng, B, S, H, K, V, "head"), torch.float32)
    gate, _ = make_gate(rng, B, S, H, V, "f32")
    gamma = torch.tensor(1.0 + 0.1 * rng.standard_normal(V), dtype=torch.float32, device=DEV)
    y, s = run_fused(g_args, gate, gamma, 1e-5, torch.float32, 16)
    want_y, want_s = oracle_of(g_args, gate, gamma, 1e-5, 16)
    assert rel_err(np_of(y), want_y) < 1e-4 and rel_err(np_of(s), want_s) < 1e-4


def test_config2_shape_fused_equals_two_calls():
    """BASELINE config 2's shape (B=8, T=4096, H=16, dk=128, dv=256: each head
    row over two scan workgroups that exchange per-token sums): the fused
    call against dn_chunk_fwd followed by dn_out_norm on its y. The fused
    scan takes the sums of squares from the fp32 y where the two calls take
    them from the bf16 y, hence a bar of 1e-2 rather than bit equality. The
    profile shows the norm inside the scan (no dn_out_norm launch)."""
    announce("config 2 shape: fused out norm vs dn_chunk_fwd + dn_out_norm")
    B, T, H, K, V = 8, 4096, 16, 128, 256
    l2 = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    gr = torch.Generator(device=DEV)
    gr.manual_seed(11)
    q = l2(torch.randn((B, T, H, K), generator=gr, device=DEV)).to(torch.bfloat16)
    k = l2(torch.randn((B, T, H, K), generator=gr, device=DEV)).to(torch.bfloat16)
    v = torch.randn((B, T, H, V), generator=gr, device=DEV).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn((B, T, H, 1), generator=gr, device=DEV))
    g = -torch.nn.functional.softplus(torch.randn((B, T, H, 1), generator=gr, device=DEV)) * 0.05
    s0 = torch.zeros((B, H, K, V), device=DEV)
    z = torch.randn((B, T, H, V), generator=gr, device=DEV).to(torch.bfloat16)
    gamma = 1.0 + 0.1 * torch.randn((V,), generator=gr, device=DEV)
    abi.profile_enable(True)
    y_f, s_f = run_fused([q, k, v, beta, beta, g, s0], z, gamma, 1e-5, torch.bfloat16)
    prof = abi.profile_read()
    abi.profile_enable(False)
    assert "dn_mfma_scan_norm" in prof and "dn_out_norm" not in prof, prof
    y = torch.empty((B, T, H, V), dtype=torch.bfloat16, device=DEV)
    s1 = torch.empty_like(s0)
    abi.run_chunk_fwd(abi.chunk_fwd_args(q, k, v, beta, beta, g, s0, y, s1, 64, None))
    out = torch.empty_like(y)
    abi.run_out_norm(abi.out_norm_args(y, z, gamma, out, 1e-5))
    torch.cuda.synchronize()
    err = float((y_f.float() - out.float()).abs().max() / out.float().abs().max())
    print(f"  fused vs two calls: rel err {err:.2e}", flush=True)
    assert err < 1e-2
    assert torch.equal(s_f, s1)
    assert abi.wait_give_ups() == 0
