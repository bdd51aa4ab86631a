"""The segmented MFMA scan against the oracle.

When batch × heads × head_v_dim/128 leaves most of the device's 256 CUs idle,
the two-kernel forward cuts each sequence into P segments of whole chunks
(P a power of two, at least 16 chunks per segment, head_k_dim 128): one scan
forms every segment's transition M and offset H (the affine map the chunk
updates compose to), a carry kernel walks the segments in order (start(s+1)
= M_s·start(s) + H_s, as bf16 hi + lo MFMAs), and a second scan produces y
and the final state from the carried starts. The shapes below give P = 2, 4
and 8 on a 256-CU MI355X; the library's per-kernel profiler confirms the
carry ran. Bar: the north_star's bf16 bar (normwise relative ≤ 2e-2, fp32
state) against the oracle fed the bf16-rounded q/k/v the GPU reads."""

import numpy as np
import pytest
import torch

from conftest import l2, rel_err
from gpu_util import DEV, announce, as_oracle_inputs, np_of, pkg, to_gpu
from oracle import oracle as O

pytestmark = pytest.mark.gpu

abi = pkg.abi
TOL = 2e-2


def inputs(rng, B, S, H, K, V, gates, state_std):
    """gates: None (DeltaNet), "head" (Gated DeltaNet) or "channel" (GDN-2)."""
    q = l2(rng.standard_normal((B, S, H, K)))
    k = l2(rng.standard_normal((B, S, H, K)))
    v = rng.standard_normal((B, S, H, V))
    ew, ww, dw = (K, V, K) if gates == "channel" else (1, 1, 1)
    e = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, ew))))
    w = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, S, H, ww)))) if gates == "channel" else e
    g = None if gates is None else -np.log1p(np.exp(rng.standard_normal((B, S, H, dw)))) * 0.05
    s0 = rng.normal(0.0, state_std, (B, H, K, V)) if state_std else np.zeros((B, H, K, V))
    return [q, k, v, e, w, g, s0]


def run(g_args, y_dtype=torch.bfloat16, in_place=False):
    q, k, v, e, w, g, s = g_args
    B, S, H, K = q.shape
    V = v.shape[3]
    y = torch.full((B, S, H, V), float("nan"), dtype=y_dtype, device=DEV)
    s_out = s if in_place else torch.full_like(s, float("nan"))
    a = abi.chunk_fwd_args(q, k, v, e, w, g, s, y, s_out, 64, None)
    assert abi.lib().dn_chunk_fwd_algo(a) == abi.DN_ALGO_MFMA
    torch.cuda.synchronize()
    abi.profile_enable(True)
    abi.run_chunk_fwd(a)
    torch.cuda.synchronize()
    kernels = set(abi.profile_read())
    abi.profile_enable(False)
    return np_of(y), np_of(s_out), kernels


CASES = [
    # B, S, H, K, V, gates, state_std: segments on a 256-CU device
    (1, 4096, 2, 128, 128, "head", 0.02),      # P = 4
    (1, 8192, 1, 128, 128, "channel", 0.02),   # P = 8, GDN-2 gate widths
    (1, 2048, 1, 128, 256, "head", 0.0),       # P = 2, two 128-column tiles
    (2, 4096, 1, 128, 128, None, 0.02),        # P = 4, ungated
    (1, 4096, 1, 128, 128, "channel", 0.5),    # P = 4, a large initial state
]


@pytest.mark.parametrize("case", CASES)
def test_segmented_scan_matches_oracle(rng, case):
    B, S, H, K, V, gates, sstd = case
    announce(f"segmented scan {case}")
    g_args = to_gpu(inputs(rng, B, S, H, K, V, gates, sstd), torch.bfloat16)
    ref = as_oracle_inputs(g_args)
    y, s, kern = run(g_args)
    assert "dn_mfma_seg_carry" in kern, kern
    y0, s0 = O.chunk_fwd(*ref, chunk_len=64, dtype=np.float64)
    ey, es = rel_err(y, y0), rel_err(s, s0)
    print(f"  rel err y {ey:.2e} state {es:.2e}", flush=True)
    assert np.isfinite(y).all() and np.isfinite(s).all()
    assert ey < TOL and es < TOL


def test_segmented_scan_in_place_state_fp32_y(rng):
    """The carry reads the initial state before the last scan overwrites it."""
    announce("segmented scan, in-place state, fp32 y")
    g_args = to_gpu(inputs(rng, 1, 8192, 1, 128, 128, "channel", 0.1), torch.bfloat16)
    ref = as_oracle_inputs(g_args)
    y, s, kern = run(g_args, y_dtype=torch.float32, in_place=True)
    assert "dn_mfma_seg_carry" in kern
    y0, s0 = O.chunk_fwd(*ref, chunk_len=64, dtype=np.float64)
    assert rel_err(y, y0) < TOL and rel_err(s, s0) < TOL


def test_short_or_ragged_sequences_are_not_segmented(rng):
    """Fewer than 32 chunks, or a partial last chunk: one scan over the sequence."""
    announce("segmented scan: dispatch")
    for S in (1024, 4000):
        g_args = to_gpu(inputs(rng, 1, S, 1, 128, 128, "head", 0.0), torch.bfloat16)
        assert "dn_mfma_seg_carry" not in run(g_args)[2]
