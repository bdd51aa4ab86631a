"""HIP-graph capture of the MFMA forward and backward.

A captured dn_chunk_fwd + dn_chunk_bwd replays to the eager results. The
backward forks its reverse scan onto the library's second stream and joins it
back, so the capture holds a branch. The graph is replayed several times, with
the outputs poisoned and other eager work and synchronisations between the
replays, and every replay is checked. Workspaces are caller-owned, so nothing
allocates under capture."""

import numpy as np
import pytest
import torch

from conftest import rel_err
from gpu_util import DEV, announce, np_of, pkg, to_gpu
from test_gpu_mfma import gdn2_inputs, gdn_inputs

pytestmark = pytest.mark.gpu

MFMA = pkg.abi.DN_ALGO_MFMA


def _workspace(nbytes):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=DEV)


@pytest.mark.parametrize("gates", ["head", (128, 128)])
def test_graph_replays_match_eager(rng, gates):
    announce(f"graph capture fwd+bwd, gates {gates}")
    B, S, H, K, V = 1, 256, 2, 128, 128
    if gates == "head":
        args = gdn_inputs(rng, B, S, H, K, V, gated=True, state_std=0.05)
    else:
        args = gdn2_inputs(rng, B, S, H, K, V, gates[0], gates[1], state_std=0.05)
    q, k, v, e, w, g, s = to_gpu(args, torch.bfloat16)
    dy = torch.tensor(rng.standard_normal((B, S, H, V)), dtype=torch.float32,
                      device=DEV).to(torch.bfloat16)
    abi = pkg.abi
    y = torch.empty((B, S, H, V), dtype=torch.bfloat16, device=DEV)
    s1 = torch.empty_like(s)
    fa = abi.chunk_fwd_args(q, k, v, e, w, g, s, y, s1, 64, None)
    wsf = _workspace(abi.lib().dn_chunk_fwd_workspace_bytes(fa))
    fa.workspace, fa.workspace_bytes = wsf.data_ptr(), wsf.numel()
    grads = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
             torch.empty_like(e), torch.empty_like(w), torch.empty_like(g), torch.empty_like(s))
    ba = abi.chunk_bwd_args(dy, None, q, k, v, e, w, g, s, grads, 64, None)
    wsb = _workspace(abi.lib().dn_chunk_bwd_workspace_bytes(ba))
    ba.workspace, ba.workspace_bytes = wsb.data_ptr(), wsb.numel()
    assert abi.lib().dn_chunk_fwd_algo(fa) == MFMA
    assert abi.lib().dn_chunk_bwd_algo(ba) == MFMA

    def run():
        abi.run_chunk_fwd(fa)
        abi.run_chunk_bwd(ba)

    outs = (y, s1) + grads
    names = ["y", "state", "d_q", "d_k", "d_v", "d_erase", "d_write", "d_g", "d_state"]
    run()
    torch.cuda.synchronize()
    want = [np_of(o) for o in outs]

    # Warm-up on a side stream, then capture (torch's capture protocol).
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    torch.cuda.synchronize()

    # Eager work between replays: another forward on its own buffers.
    y2, s2 = torch.empty_like(y), torch.empty_like(s1)
    fa2 = abi.chunk_fwd_args(k, q, v, e, w, g, s, y2, s2, 64, None)
    ws2 = _workspace(abi.lib().dn_chunk_fwd_workspace_bytes(fa2))
    fa2.workspace, fa2.workspace_bytes = ws2.data_ptr(), ws2.numel()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        abi.run_chunk_fwd(fa2)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, o, ref in zip(names, outs, want):
            got = np_of(o)
            assert np.isfinite(got).all(), f"replay {rep}: {name} not written"
            err = rel_err(got, ref)
            # Row sums over channels use LDS atomics (per-head gates): their
            # order may differ between runs, at fp32 rounding level.
            assert err < 1e-5, f"replay {rep}: {name} rel err {err:.2e}"
        print(f"  replay {rep} matches", flush=True)
