"""dn_chunk_fwd_noalloc against dn_chunk_fwd through the C ABI.

The no-allocation entry point runs dn_chunk_fwd's kernels on the library's
fixed scratch array instead of a workspace, so its outputs must equal
dn_chunk_fwd's bit for bit, on the MFMA path and on the generic fp32 path.
Two calls in a row share the array; the second, with a smaller input, must
not be affected by what the first left there. Arguments above the array's
size are refused with DN_ERR_WORKSPACE before anything runs.
"""

import pytest
import torch

from gpu_util import DEV, announce, pkg

pytestmark = pytest.mark.gpu

abi = pkg.abi


def inputs(seed, B, S, H, K, V, dtype, channel=False):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    l2 = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q = l2(torch.randn((B, S, H, K), generator=g, device=DEV)).to(dtype)
    k = l2(torch.randn((B, S, H, K), generator=g, device=DEV)).to(dtype)
    v = torch.randn((B, S, H, V), generator=g, device=DEV).to(dtype)
    kw, vw = (K, V) if channel else (1, 1)
    e = torch.sigmoid(torch.randn((B, S, H, kw), generator=g, device=DEV))
    w = torch.sigmoid(torch.randn((B, S, H, vw), generator=g, device=DEV))
    gg = -torch.nn.functional.softplus(torch.randn((B, S, H, kw), generator=g, device=DEV)) * 0.1
    s0 = torch.randn((B, H, K, V), generator=g, device=DEV) * 0.1
    return q, k, v, e, w, gg, s0


def both(q, k, v, e, w, gg, s0, algo=abi.DN_ALGO_AUTO):
    """(y, state) of dn_chunk_fwd with its own workspace, and of the no-alloc entry."""
    B, S, H, K = q.shape
    V = v.shape[3]
    outs = []
    for noalloc in (False, True):
        y = torch.full((B, S, H, V), float("nan"), dtype=q.dtype, device=DEV)
        s1 = torch.full((B, H, K, V), float("nan"), device=DEV)
        args = abi.chunk_fwd_args(q, k, v, e, w, gg, s0, y, s1, 64, None, algo=algo)
        if noalloc:
            assert abi.lib().dn_chunk_fwd_workspace_bytes(args) <= abi.NOALLOC_SCRATCH_BYTES
            abi.run_chunk_fwd_noalloc(args)
        else:
            ws = torch.empty(max(abi.lib().dn_chunk_fwd_workspace_bytes(args), 1),
                             dtype=torch.uint8, device=DEV)
            args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
            abi.run_chunk_fwd(args)
            chosen = abi.lib().dn_chunk_fwd_algo(args)
        torch.cuda.synchronize()
        outs.append((y, s1))
    return outs, chosen


@pytest.mark.parametrize("case", [
    # (B, S, H, K, V, dtype, channel): the first call, then a smaller second one
    ((2, 1000, 4, 128, 256, torch.bfloat16, False), (1, 130, 2, 128, 128, torch.bfloat16, False)),
    ((1, 700, 2, 128, 128, torch.bfloat16, True), (1, 77, 1, 64, 64, torch.bfloat16, True)),
    ((1, 200, 2, 64, 48, torch.float32, False), (1, 37, 1, 16, 24, torch.float32, False)),
])
@pytest.mark.parametrize("fused", [False, True])
def test_noalloc_forward_equals_dn_chunk_fwd_on_two_calls_in_a_row(case, fused):
    if fused and any(K != 128 or dtype != torch.bfloat16 or channel
                     for _, _, _, K, _, dtype, channel in case):
        pytest.skip("DN_ALGO_MFMA_FUSED serves per-head gates at head_k_dim 128, bf16 q/k/v")
    for n, (B, S, H, K, V, dtype, channel) in enumerate(case):
        announce(f"dn_chunk_fwd_noalloc call {n + 1}: B={B} S={S} H={H} K={K} V={V} "
                 f"{dtype} channel={channel} fused={fused}")
        algo = abi.DN_ALGO_MFMA_FUSED if fused else abi.DN_ALGO_AUTO
        (ref, got), chosen = both(*inputs(40 + n, B, S, H, K, V, dtype, channel), algo=algo)
        assert chosen == (abi.DN_ALGO_MFMA_FUSED if fused else
                          abi.DN_ALGO_MFMA if dtype == torch.bfloat16 else abi.DN_ALGO_GENERIC)
        assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])


def test_noalloc_refuses_arguments_above_its_scratch():
    announce("dn_chunk_fwd_noalloc: too large for the scratch array")
    # BASELINE config 5 (GDN-2 per-channel gates): 737 MB of workspace.
    B, S, H, K, V = 2, 16384, 16, 128, 128
    q = torch.empty((B, S, H, K), dtype=torch.bfloat16, device=DEV)
    v = torch.empty((B, S, H, V), dtype=torch.bfloat16, device=DEV)
    e = torch.empty((B, S, H, K), device=DEV)
    w = torch.empty((B, S, H, V), device=DEV)
    s0 = torch.empty((B, H, K, V), device=DEV)
    args = abi.chunk_fwd_args(q, q, v, e, w, e, s0, v, s0, 64, None)
    assert abi.lib().dn_chunk_fwd_workspace_bytes(args) > abi.NOALLOC_SCRATCH_BYTES
    with pytest.raises(pkg.DeltaError, match="above its maximum"):
        abi.run_chunk_fwd_noalloc(args)
