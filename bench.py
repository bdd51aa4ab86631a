#!/usr/bin/env python3
"""Benchmark of the delta-rule core on one MI355X.

Headline (BASELINE.json metric "chunk fwd tokens/s + decode step µs (GDN H16
dk128) at 1 GPU; % roofline"):

* value  = chunkwise forward throughput on BASELINE config 2 (Gated DeltaNet
  prefill: B=8, H=16, T=4096, dk=128, dv=256, chunk 64; bf16 q/k/v, fp32 β/g
  and state, bf16 y). One step = one dn_chunk_fwd over the whole batch, inputs
  already resident in HBM.
* decode = config 3 (batch 256, H16, dk128, dv256, fp32 state ≈ 537 MB):
  µs per dn_step over consecutive steps, and its HBM roofline; product_u2 =
  DeltaProduct decode (2 micro-steps per token) at the same shape as one
  dn_recurrent call per token.
* roofline = the dominant kernel of the forward, timed with HIP events on its
  own stream by the library's profiler (dn_profile_*), against algorithmic
  bytes per launch (the per-unit figures are in bench_chunk_fwd).
* config4 / config5 = BASELINE configs 4 (DeltaProduct u=2, folded core
  forward) and 5 (GDN-2 per-channel gates, forward + custom backward), each
  with its own HBM roofline; not part of `value`.
* frontend / out_norm = dn_frontend (the projection front-end) and
  dn_out_norm (the gated output norm) at the config-2 shape, each with its
  HBM roofline; not part of `value`.
* cpu_baseline = the CPU oracle (a C++ restatement of the reference algorithm,
  incl. its 24·L³ ladder) on a bounded sample of config 2, all host threads.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
METRIC = "chunk fwd tokens/s + decode step µs (GDN H16 dk128) at 1 GPU; % roofline"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
ALGO_NAMES = {1: "generic", 2: "mfma (intra + scan kernels)", 3: "mfma (fused kernel)"}


def load_package():
    sys.path.insert(0, str(ROOT))
    import __graft_entry__ as ge
    return ge.load_package()


def gdn_inputs(torch, B, T, H, K, V, g_scale, seed, qkv_dtype, device):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    def l2(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q = l2(torch.randn((B, T, H, K), generator=gen, device=device)).to(qkv_dtype)
    k = l2(torch.randn((B, T, H, K), generator=gen, device=device)).to(qkv_dtype)
    v = torch.randn((B, T, H, V), generator=gen, device=device).to(qkv_dtype)
    beta = torch.sigmoid(torch.randn((B, T, H, 1), generator=gen, device=device))
    g = -torch.nn.functional.softplus(torch.randn((B, T, H, 1), generator=gen,
                                                  device=device)) * g_scale
    return q, k, v, beta, g


def bench_chunk_fwd(torch, pkg, steps, warmup, algo):
    B, T, H, K, V, L = 8, 4096, 16, 128, 256, 64
    dev = torch.device("cuda:0")
    q, k, v, beta, g = gdn_inputs(torch, B, T, H, K, V, 0.05, 20260828, torch.bfloat16, dev)
    s0 = torch.zeros((B, H, K, V), dtype=torch.float32, device=dev)
    y = torch.empty((B, T, H, V), dtype=torch.bfloat16, device=dev)
    s1 = torch.empty_like(s0)
    abi = pkg.abi
    args = abi.chunk_fwd_args(q, k, v, beta, beta, g, s0, y, s1, L, None, algo=algo)
    ws_bytes = abi.lib().dn_chunk_fwd_workspace_bytes(args)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    chosen = abi.lib().dn_chunk_fwd_algo(args)
    run = lambda: abi.run_chunk_fwd(args)
    t0 = time.perf_counter()
    ms, prof = _timed_raw(torch, abi, run, steps, warmup)
    wall = time.perf_counter() - t0
    tokens = B * T
    G = B * (T // L) * H
    # Algorithmic bytes per launch of each forward kernel: every tensor it
    # must move once.
    qk = 2 * B * T * H * K * 2          # q and k, bf16
    vb = B * T * H * V * 2              # v, bf16
    yb = B * T * H * V * 2              # y, bf16
    gates = 2 * B * T * H * 4           # β and g, fp32
    st = B * H * K * V * 4              # one fp32 state
    tri = 3 * G * 6 * 16 * 32 * 2       # T (hi, lo) and attn, bf16: their six nonzero 16x32 blocks
    gcb = G * L * 4                     # in-chunk cumulative gate, fp32
    # The bytes each kernel moves by its own design (intermediates included),
    # beside the path's algorithmic bytes. (The scan forms (e^{G_last-G} k)^T
    # from its own K tile, so it does not go through HBM.)
    kernel_bytes = {
        "dn_mfma_intra": qk + gates + tri + gcb,
        "dn_mfma_scan": qk + vb + yb + gates + tri + gcb + 2 * st,
        "dn_mfma_fused": qk + vb + yb + gates + 2 * st,
    }
    flops_unit = 6 * L * L * K + 4 * L * L * V + 6 * L * K * V + L ** 3 / 3
    # The path's algorithmic bytes (every tensor crossing the C ABI once):
    # 102,912 B per chunk-head at this shape, 843,055,104 B per launch.
    path_bytes = qk + vb + yb + gates + 2 * st
    return dict(ms=ms, wall_ms=wall * 1e3 / steps, tokens=tokens, prof=prof,
                kernel_bytes=kernel_bytes, path_bytes=path_bytes, chunk_heads=G,
                path_flops=G * flops_unit, algo=chosen, ws_bytes=ws_bytes)


def bench_decode(torch, pkg, steps, warmup):
    B, H, K, V = 256, 16, 128, 256
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260829)
    S = torch.randn((B, H, K, V), generator=gen, device=dev) * 0.02
    n_tok = steps  # one distinct token per timed step: a steps-token sequence
    l2 = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q = l2(torch.randn((n_tok, B, H, K), generator=gen, device=dev))
    k = l2(torch.randn((n_tok, B, H, K), generator=gen, device=dev))
    v = torch.randn((n_tok, B, H, V), generator=gen, device=dev)
    beta = torch.sigmoid(torch.randn((n_tok, B, H, 1), generator=gen, device=dev))
    g = -torch.nn.functional.softplus(torch.randn((n_tok, B, H, 1), generator=gen,
                                                  device=dev)) * 0.05
    y = torch.empty((B, H, V), dtype=torch.float32, device=dev)
    abi = pkg.abi
    argv = [abi.step_args(q[t], k[t], v[t], beta[t], beta[t], g[t], S, y, S, None)
            for t in range(n_tok)]
    lib = abi.lib()
    import ctypes
    stream = abi.stream_handle()
    refs = [ctypes.byref(a) for a in argv]
    it = iter(range(1 << 62))

    def run():
        rc = lib.dn_step(refs[next(it) % n_tok], stream)
        if rc:
            abi.check(rc)
    ms, prof = _timed_raw(torch, abi, run, steps, warmup)
    us = ms * 1e3
    step_bytes = 2 * B * H * K * V * 4 + B * H * (2 * K + 2 * V + 2) * 4
    name = max(prof, key=lambda n: prof[n][0]) if prof else None
    k_us = prof[name][0] * 1e3 / prof[name][1] if name else us
    return dict(us=us, kernel_us=k_us, bytes=step_bytes, prof=prof, kernel=name)


def bench_product_decode(torch, pkg, steps, warmup, u=2):
    """DeltaProduct decode at the config-3 shape (B=256, H=16, dk=128,
    dv=256, fp32 state): one decode token = u Householder micro-steps
    (delta_product.rs:270-305), folded into a u-token sequence as in
    config 4 (q on the last micro-step, the forget gate on the first,
    β = 2σ(N)) and run as one dn_recurrent call, which reads and writes
    the state once per token instead of once per micro-step."""
    B, H, K, V = 256, 16, 128, 256
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260831)
    S = torch.randn((B, H, K, V), generator=gen, device=dev) * 0.02
    n_in = min(steps, 32)  # distinct input sets, cycled
    l2 = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q = torch.zeros((n_in, B, u, H, K), device=dev)
    q[:, :, u - 1] = l2(torch.randn((n_in, B, H, K), generator=gen, device=dev))
    k = l2(torch.randn((n_in, B, u, H, K), generator=gen, device=dev))
    v = torch.randn((n_in, B, u, H, V), generator=gen, device=dev)
    beta = 2 * torch.sigmoid(torch.randn((n_in, B, u, H, 1), generator=gen, device=dev))
    g = torch.zeros((n_in, B, u, H, 1), device=dev)
    g[:, :, 0] = -torch.nn.functional.softplus(
        torch.randn((n_in, B, H, 1), generator=gen, device=dev)) * 0.05
    y = torch.empty((B, u, H, V), dtype=torch.float32, device=dev)
    abi = pkg.abi
    argv = [abi.recurrent_args(q[t], k[t], v[t], beta[t], beta[t], g[t], S, y, S, None)
            for t in range(n_in)]
    import ctypes
    lib, stream = abi.lib(), abi.stream_handle()
    refs = [ctypes.byref(a) for a in argv]
    it = iter(range(1 << 62))

    def run():
        rc = lib.dn_recurrent(refs[next(it) % n_in], stream)
        if rc:
            abi.check(rc)
    ms, kern = _timed(torch, abi, run, steps, warmup)
    nbytes = 2 * B * H * K * V * 4 + u * B * H * (2 * K + 2 * V + 2) * 4
    name = max(kern, key=lambda n: kern[n]["avg_us"]) if kern else None
    k_us = kern[name]["avg_us"] if name else ms * 1e3
    # One kernel per call, launched back to back in the timed region: the
    # region's time per call is the kernel's average launch duration (gaps
    # included). The profile pass brackets each launch with its own events,
    # whose end-of-kernel release adds to what it reads (kernel_us).
    return {"workload": f"DeltaProduct decode, u={u} micro-steps per token, config-3 shape",
            "entry_point": "dn_recurrent", "calls": steps, "us_per_token": round(ms * 1e3, 2),
            "kernel_us": k_us, "bytes_per_token": nbytes,
            "roofline": _hbm(nbytes, ms) | {"kernel": name,
                                            "avg_launch_source": "timed region, one kernel a call",
                                            "traffic": traffic_from_profiles(name)}}


def bench_frontend(torch, pkg, steps, warmup):
    """The projection front-end (dn_frontend: QkvProjection::forward after its
    in_proj, qkv.rs:373-449) at the config-2 shape: B=8, T=4096, H=16,
    dk=128, dv=256, u=1, short conv of 4 with SiLU, L2 q/k norm, scalar β;
    bf16 projection in, bf16 q/k/v out, fp32 β."""
    B, S, H, K, V, KC = 8, 4096, 16, 128, 256, 4
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260832)
    conv_dim = H * K * 2 + H * V
    width = conv_dim + H
    proj = torch.randn((B, S, width), generator=gen, device=dev).to(torch.bfloat16)
    weight = torch.randn((conv_dim, KC), generator=gen, device=dev) * 0.5
    win = torch.randn((B, conv_dim, KC), generator=gen, device=dev).to(torch.bfloat16)
    wout = torch.empty_like(win)
    q = torch.empty((B, S, H, K), dtype=torch.bfloat16, device=dev)
    k, v = torch.empty_like(q), torch.empty((B, S, H, V), dtype=torch.bfloat16, device=dev)
    beta = torch.empty((B, S, H, 1), device=dev)
    abi = pkg.abi
    args = abi.frontend_args(proj, weight, None, win, wout, q, k, v, beta, beta, nheads=H,
                             head_k_dim=K, head_v_dim=V, n_householder=1,
                             conv_activation=abi.DN_ACT_SILU, qk_activation=abi.DN_ACT_SILU,
                             qk_norm=abi.DN_QKNORM_L2, write_gate=abi.DN_WRITE_SCALAR,
                             allow_neg_eigval=False)
    ms, kern = _timed(torch, abi, lambda: abi.run_frontend(args), steps, warmup)
    # Read the conv and β columns (bf16), write q, k, v (bf16) and β (fp32);
    # the windows (read + write) are B·conv_dim·KC each.
    nbytes = B * S * (width * 2 + conv_dim * 2 + H * 4) + 2 * B * conv_dim * KC * 2
    k_ms = kern["dn_frontend"]["avg_us"] / 1e3 if "dn_frontend" in kern else ms
    return {"workload": "dn_frontend at the config-2 shape (B=8 T=4096 H=16 dk=128 dv=256, "
                        "conv 4, SiLU, L2, scalar beta; bf16)",
            "ms_per_call": round(ms, 4), "tokens_per_s": round(B * S / (ms / 1e3), 1),
            "roofline": _hbm(nbytes, k_ms) | {"kernel": "dn_frontend",
                                               "traffic": traffic_from_profiles("dn_frontend")},
            "kernels": kern}


def bench_out_norm(torch, pkg, steps, warmup):
    """The gated output norm (dn_out_norm: OutNorm::forward, norm.rs:106-144)
    on config 2's delta-rule output: y [8, 4096, 16, 256] bf16, the gate of
    the same shape in bf16, bf16 out; ε = 1e-5."""
    B, S, H, V = 8, 4096, 16, 256
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260833)
    x = torch.randn((B, S, H, V), generator=gen, device=dev).to(torch.bfloat16)
    g = torch.randn((B, S, H, V), generator=gen, device=dev).to(torch.bfloat16)
    w = torch.randn(V, generator=gen, device=dev)
    out = torch.empty_like(x)
    abi = pkg.abi
    args = abi.out_norm_args(x, g, w, out, 1e-5)
    ms, kern = _timed(torch, abi, lambda: abi.run_out_norm(args), steps, warmup)
    nbytes = 3 * B * S * H * V * 2 + V * 4
    k_ms = kern["dn_out_norm"]["avg_us"] / 1e3 if "dn_out_norm" in kern else ms
    return {"workload": "dn_out_norm (gated RMSNorm per head) on config 2's output, bf16",
            "ms_per_call": round(ms, 4), "tokens_per_s": round(B * S / (ms / 1e3), 1),
            "roofline": _hbm(nbytes, k_ms) | {"kernel": "dn_out_norm",
                                               "traffic": traffic_from_profiles("dn_out_norm")},
            "kernels": kern}


def bench_block_decode(torch, pkg, steps, warmup):
    """One decode token of a Gated DeltaNet block after in_proj at the
    config-3 shape (B=256, H=16, dk=128, dv=256; short conv of 4 with SiLU,
    L2 q/k norm, scalar β, gated output norm; bf16 projection, window and
    out, fp32 state updated in place): dn_block_step against the three calls
    it fuses, dn_frontend's step (bf16 q/k/v), dn_step and dn_out_norm."""
    B, H, K, V = 256, 16, 128, 256
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260839)
    proj = pkg.QkvProjection(nheads=H, head_k_dim=K, head_v_dim=V, has_gate=True)
    proj.conv = pkg.ShortConv(torch.randn((proj.conv_dim(), 4), generator=gen, device=dev) * 0.5)
    norm = pkg.OutNorm(torch.ones(V, device=dev), gated=True)
    W = proj.d_in_proj()
    p = torch.randn((B, W), generator=gen, device=dev).to(torch.bfloat16)
    win = torch.randn((B, proj.conv_dim(), 4), generator=gen, device=dev).to(torch.bfloat16)
    g = -torch.nn.functional.softplus(torch.randn((B, H, 1), generator=gen, device=dev)) * 0.05
    s = torch.randn((B, H, K, V), generator=gen, device=dev) * 0.02
    abi = pkg.abi
    a, out, _, _, _, kept = pkg.frontend.block_step_args(proj, norm, p, win, g, s,
                                                          out_dtype=torch.bfloat16, in_place=True)
    fused_ms, fused_k = _timed(torch, abi, lambda: abi.run_block_step(a), steps, warmup)
    # The three calls, bf16 between them.
    q = torch.empty((B, 1, H, K), dtype=torch.bfloat16, device=dev)
    k, v = torch.empty_like(q), torch.empty((B, 1, H, V), dtype=torch.bfloat16, device=dev)
    beta = torch.empty((B, 1, H, 1), device=dev)
    weight = proj.conv.weight.float().contiguous()
    fe = abi.frontend_args(p.view(B, 1, W), weight, None, win, win, q, k, v, beta, beta,
                           nheads=H, head_k_dim=K, head_v_dim=V, n_householder=1,
                           conv_activation=abi.DN_ACT_SILU, qk_activation=abi.DN_ACT_SILU,
                           qk_norm=abi.DN_QKNORM_L2, write_gate=abi.DN_WRITE_SCALAR,
                           allow_neg_eigval=False)
    y = torch.empty((B, H, V), dtype=torch.bfloat16, device=dev)
    st = abi.step_args(q.view(B, H, K), k.view(B, H, K), v.view(B, H, V), beta.view(B, H, 1),
                       beta.view(B, H, 1), g, s, y, s, None)
    c0 = proj.conv_dim() + H
    zg = p[:, c0:c0 + H * V].unflatten(1, (H, V))
    on = abi.out_norm_args(y, zg, norm.weight, torch.empty_like(y), norm.eps)

    def three():
        abi.run_frontend(fe)
        abi.check(abi.lib().dn_step(ctypes.byref(st), abi.stream_handle()))
        abi.run_out_norm(on)
    sep_ms, sep_k = _timed(torch, abi, three, steps, warmup)
    nbytes = 2 * B * H * K * V * 4 + B * W * 2 + 2 * B * proj.conv_dim() * 4 * 2 + B * H * V * 2
    del kept
    return {"workload": "Gated DeltaNet block decode token after in_proj, config-3 shape "
                        "(B=256 H=16 dk=128 dv=256), bf16 projection/window/out, fp32 state",
            "fused_us": round(fused_ms * 1e3, 2), "three_calls_us": round(sep_ms * 1e3, 2),
            "roofline": _hbm(nbytes, fused_ms), "kernels_fused": fused_k,
            "kernels_three_calls": sep_k}


def bench_unit_lower_inverse(torch, pkg, steps, warmup):
    """The standalone unit_lower_inverse (dn_unit_lower_inverse, tri.rs:66-114,
    TriSolve::Blocked) on a chunk path's batch: 8192 blocks of 64 (config 2's
    chunk-heads), and 1024 blocks of 128; float32 in and out."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260838)
    abi = pkg.abi
    out = {"workload": "dn_unit_lower_inverse (TriSolve::Blocked), float32"}
    for name, G, L in (("blocks64", 8192, 64), ("blocks128", 1024, 128)):
        n = torch.tril(torch.randn((G, L, L), generator=gen, device=dev) * 0.15, -1)
        t = torch.empty_like(n)
        args = abi.tri_args(n, t, abi.DN_TRI_BLOCKED)
        ms, kern = _timed(torch, abi, lambda: abi.run_unit_lower_inverse(args), steps, warmup)
        out[name] = {"matrices": G, "size": L, "ms_per_call": round(ms, 4),
                     "roofline": _hbm(2 * G * L * L * 4, ms), "kernels": kern}
        del n, t
    return out


MIN_STEPS, MIN_WARMUP = 20, 2  # timed calls and warm-ups of every line
# Untimed run-in before every timed region's warm-up steps: the GPU's clocks
# ramp over its first ~0.1 s of work after idling (config 2 at 5 warm-ups
# measured 0.49-0.53 ms per step, at 100 warm-ups 0.43-0.45 ms). The W
# warm-up steps the caller asks for still run right before the K timed ones.
SETTLE_S = 0.3
_EXACT = {"on": False}  # --profile-pass: run exactly the calls asked for, no profiler pass


def _timed_raw(torch, abi, fn, steps, warmup):
    """Mean ms per call of fn() over max(steps, 20) calls after a SETTLE_S
    run-in and then max(warmup, 2) warm-up calls,
    timed with HIP events on torch's current stream (the stream the library
    launches on) and nothing else recorded inside the timed region; then a
    separate pass with the library's per-kernel HIP-event profiler on, which
    gives {kernel: (total_ms, launches)}."""
    if not _EXACT["on"]:
        steps, warmup = max(steps, MIN_STEPS), max(warmup, MIN_WARMUP)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < SETTLE_S:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    if _EXACT["on"]:
        return ms, {}
    abi.profile_enable(True)
    for _ in range(min(steps, 10)):
        fn()
    torch.cuda.synchronize()
    prof = abi.profile_read()
    abi.profile_enable(False)
    return ms, prof


def _timed(torch, abi, fn, steps, warmup):
    """_timed_raw with the profile as {kernel: {avg_us, launches}}."""
    ms, prof = _timed_raw(torch, abi, fn, steps, warmup)
    kern = {n: {"avg_us": round(v[0] / v[1] * 1e3, 2), "launches": v[1]} for n, v in prof.items()}
    return ms, kern


def _hbm(nbytes, ms):
    gbs = nbytes / (ms / 1e3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": int(nbytes)}


def bench_config4(torch, pkg, steps, warmup):
    """DeltaProduct with 2 Householder micro-steps per token
    (allow_neg_eigval: β = 2σ(N)), B=4, T=8192 (core sequence 16384), H=16,
    dk=dv=128, chunk 64, bf16 q/k/v, fp32 state. The core sees the folded
    sequence of delta_product.rs:178-205: q only on the last micro-step of a
    token, the forget gate only on the first."""
    B, T, H, K, V, u = 4, 8192, 16, 128, 128, 2
    S = T * u
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260830)
    l2 = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q = torch.zeros((B, T, u, H, K), device=dev)
    q[:, :, u - 1] = l2(torch.randn((B, T, H, K), generator=gen, device=dev))
    q = q.reshape(B, S, H, K).to(torch.bfloat16)
    k = l2(torch.randn((B, S, H, K), generator=gen, device=dev)).to(torch.bfloat16)
    v = torch.randn((B, S, H, V), generator=gen, device=dev).to(torch.bfloat16)
    beta = 2 * torch.sigmoid(torch.randn((B, S, H, 1), generator=gen, device=dev))
    g = torch.zeros((B, T, u, H, 1), device=dev)
    g[:, :, 0] = -torch.nn.functional.softplus(
        torch.randn((B, T, H, 1), generator=gen, device=dev)) * 0.1
    g = g.reshape(B, S, H, 1)
    s0 = torch.zeros((B, H, K, V), device=dev)
    y = torch.empty((B, S, H, V), dtype=torch.bfloat16, device=dev)
    s1 = torch.empty_like(s0)
    abi = pkg.abi
    args = abi.chunk_fwd_args(q, k, v, beta, beta, g, s0, y, s1, 64, None)
    ws = torch.empty(max(abi.lib().dn_chunk_fwd_workspace_bytes(args), 1), dtype=torch.uint8,
                     device=dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    algo = abi.lib().dn_chunk_fwd_algo(args)
    ms, kern = _timed(torch, abi, lambda: abi.run_chunk_fwd(args), steps, warmup)
    rows = B * S * H
    nbytes = rows * (2 * K + 2 * V) * 2 + rows * 3 * 4 + 2 * B * H * K * V * 4
    return {"workload": "config 4: DeltaProduct u=2 (allow_neg_eigval), folded core forward",
            "batch": B, "seq_len": T, "core_seq_len": S, "nheads": H, "head_k_dim": K,
            "head_v_dim": V, "algo": ALGO_NAMES.get(algo, algo),
            "ms_per_step": round(ms, 4), "tokens_per_s": round(B * T / (ms / 1e3), 1),
            "roofline": _hbm(nbytes, ms), "kernels": kern}


def bench_config5(torch, pkg, steps, warmup):
    """GDN-2 forward plus the custom backward, B=2,
    T=16384, H=16, dk=dv=128, chunk 64; per-key-channel erase b and decay α,
    per-value-channel write w (fp32), bf16 q/k/v and dO."""
    B, T, H, K, V = 2, 16384, 16, 128, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260831)
    l2 = lambda x: x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    rn = lambda *shape: torch.randn(shape, generator=gen, device=dev)
    q = l2(rn(B, T, H, K)).to(torch.bfloat16)
    k = l2(rn(B, T, H, K)).to(torch.bfloat16)
    v = rn(B, T, H, V).to(torch.bfloat16)
    e = torch.sigmoid(rn(B, T, H, K))
    w = torch.sigmoid(rn(B, T, H, V))
    g = -torch.nn.functional.softplus(rn(B, T, H, K)) * 0.05
    s0 = torch.zeros((B, H, K, V), device=dev)
    y = torch.empty((B, T, H, V), dtype=torch.bfloat16, device=dev)
    s1 = torch.empty_like(s0)
    abi = pkg.abi
    fargs = abi.chunk_fwd_args(q, k, v, e, w, g, s0, y, s1, 64, None)
    wsf = torch.empty(max(abi.lib().dn_chunk_fwd_workspace_bytes(fargs), 1), dtype=torch.uint8,
                      device=dev)
    fargs.workspace, fargs.workspace_bytes = wsf.data_ptr(), wsf.numel()
    dy = rn(B, T, H, V).to(torch.bfloat16)
    grads = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(e),
             torch.empty_like(w), torch.empty_like(g), torch.empty_like(s0))
    bargs = abi.chunk_bwd_args(dy, None, q, k, v, e, w, g, s0, grads, 64, None)
    wsb = torch.empty(max(abi.lib().dn_chunk_bwd_workspace_bytes(bargs), 1), dtype=torch.uint8,
                      device=dev)
    bargs.workspace, bargs.workspace_bytes = wsb.data_ptr(), wsb.numel()
    fa, ba = abi.lib().dn_chunk_fwd_algo(fargs), abi.lib().dn_chunk_bwd_algo(bargs)
    fms, fk = _timed(torch, abi, lambda: abi.run_chunk_fwd(fargs), steps, warmup)
    bms, bk = _timed(torch, abi, lambda: abi.run_chunk_bwd(bargs), steps, warmup)
    rows = B * T * H
    st = B * H * K * V * 4
    f_bytes = rows * (2 * K + V) * 2 + rows * V * 2 + rows * (2 * K + V) * 4 + 2 * st
    # backward: reads q, k, v, dO, the gates and S0; writes dq, dk, dv, the three
    # gate gradients and dS0.
    b_bytes = rows * (2 * K + 2 * V) * 2 + rows * (2 * K + V) * 4 + st + \
        rows * (2 * K + V) * 2 + rows * (2 * K + V) * 4 + st
    # The fused chunk-local backward kernel, per chunk-head (L = 64): q, k, v,
    # dO (bf16), the three gates (fp32), S0 and dS leaving the chunk (fp32),
    # T / Tlo / Tᵀ / Tᵀlo / attnᵀ (bf16), kg hi/lo and kc (bf16) in; dq, dk,
    # dv (bf16) and the three gate gradients (fp32) out.
    L, G = 64, B * H * (T // 64)
    cb_unit = (L * (2 * K + V) * 2 + L * V * 2 + L * (2 * K + V) * 4 + 2 * K * V * 4 +
               5 * L * L * 2 + 3 * L * K * 2 + L * (2 * K + V) * 2 + L * (2 * K + V) * 4)
    cb = bk.get("dn_mfma_chunk_bwd")
    cb_roof = None
    if cb:
        cb_roof = _hbm(cb_unit * G, cb["avg_us"] / 1e3)
        cb_roof.update({"kernel": "dn_mfma_chunk_bwd", "bytes_per_chunk_head": cb_unit,
                        "chunk_heads": G})
    name = {1: "generic", 2: "mfma"}
    return {"workload": "config 5: GDN-2 per-channel gates, forward + custom backward",
            "batch": B, "seq_len": T, "nheads": H, "head_k_dim": K, "head_v_dim": V,
            "algo": {"forward": name.get(fa, fa), "backward": name.get(ba, ba)},
            "fwd_ms": round(fms, 3), "bwd_ms": round(bms, 3),
            "tokens_per_s_fwd_bwd": round(B * T / ((fms + bms) / 1e3), 1),
            "roofline_fwd": _hbm(f_bytes, fms), "roofline_bwd": _hbm(b_bytes, bms),
            "roofline_chunk_bwd": cb_roof, "kernels_fwd": fk, "kernels_bwd": bk}


def bench_config2_bwd(torch, pkg, steps, warmup, V=256, K=128):
    """The custom backward (dn_chunk_bwd: combined_backward) at the config-2
    shape: B=8, T=4096, H=16, dk=128 (or K), dv=256 (or V), per-head gates,
    bf16 q/k/v and dO, fp32 state; the gradients of all seven inputs."""
    B, T, H = 8, 4096, 16
    dev = torch.device("cuda:0")
    q, k, v, beta, g = gdn_inputs(torch, B, T, H, K, V, 0.05, 20260834, torch.bfloat16, dev)
    s0 = torch.zeros((B, H, K, V), dtype=torch.float32, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260835)
    dy = torch.randn((B, T, H, V), generator=gen, device=dev).to(torch.bfloat16)
    grads = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
             torch.empty_like(beta), torch.empty_like(beta), torch.empty_like(g),
             torch.empty_like(s0))
    abi = pkg.abi
    bargs = abi.chunk_bwd_args(dy, None, q, k, v, beta, beta, g, s0, grads, 64, None)
    ws = torch.empty(max(abi.lib().dn_chunk_bwd_workspace_bytes(bargs), 1), dtype=torch.uint8,
                     device=dev)
    bargs.workspace, bargs.workspace_bytes = ws.data_ptr(), ws.numel()
    algo = abi.lib().dn_chunk_bwd_algo(bargs)
    ms, kern = _timed(torch, abi, lambda: abi.run_chunk_bwd(bargs), steps, warmup)
    rows, st = B * T * H, B * H * K * V * 4
    # reads q, k, v, dO (bf16), erase, write, g (fp32, width 1) and S0; writes
    # dq, dk, dv (bf16), the three gate gradients (fp32) and dS0.
    nbytes = rows * (2 * K + 2 * V) * 2 + rows * 3 * 4 + st + rows * (2 * K + V) * 2 + \
        rows * 3 * 4 + st
    return {"workload": "config-2 shape backward (dn_chunk_bwd), per-head gates, bf16",
            "batch": B, "seq_len": T, "nheads": H, "head_k_dim": K, "head_v_dim": V,
            "algo": ALGO_NAMES.get(algo, algo), "ms_per_call": round(ms, 4),
            "tokens_per_s": round(B * T / (ms / 1e3), 1), "roofline": _hbm(nbytes, ms),
            "kernels": kern}


def bench_chunk_lengths(torch, pkg, steps, warmup):
    """Config 2 at other chunk lengths as AUTO serves them (the MFMA kernels'
    64-token chunks: with a per-head forget gate the chunk length orders the
    roundings only), the fp32 kernels that shapes outside the MFMA path
    fall back to, forced (DN_ALGO_GENERIC) at chunk 64, and config 2 at
    head_k_dim 256 (the MFMA forward; the generic kernels forced beside it)."""
    B, T, H, K, V = 8, 4096, 16, 128, 256
    dev = torch.device("cuda:0")
    q, k, v, beta, g = gdn_inputs(torch, B, T, H, K, V, 0.05, 20260837, torch.bfloat16, dev)
    s0 = torch.zeros((B, H, K, V), dtype=torch.float32, device=dev)
    y = torch.empty((B, T, H, V), dtype=torch.bfloat16, device=dev)
    s1 = torch.empty_like(s0)
    abi = pkg.abi
    out = {"workload": "config 2 (B=8 T=4096 H=16 dk=128 dv=256, bf16 q/k/v) at chunk_len 32 "
                       "and 128 under AUTO, on the generic fp32 kernels at 64, with "
                       "per-channel erase/write gates under AUTO, and at head_k_dim 256"}
    for name, L, algo in (("auto_chunk32", 32, 0), ("auto_chunk128", 128, 0),
                          ("forced_generic_chunk64", 64, 1)):
        a = abi.chunk_fwd_args(q, k, v, beta, beta, g, s0, y, s1, L, None, algo=algo)
        ws = torch.empty(max(abi.lib().dn_chunk_fwd_workspace_bytes(a), 1), dtype=torch.uint8,
                         device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        chosen = abi.lib().dn_chunk_fwd_algo(a)
        ms, kern = _timed(torch, abi, lambda: abi.run_chunk_fwd(a), steps, warmup)
        out[name] = {"chunk_len": L, "algo": ALGO_NAMES.get(chosen, chosen),
                     "ms_per_step": round(ms, 3), "tokens_per_s": round(B * T / (ms / 1e3), 1),
                     "kernels": kern}
        del ws
    # WriteGate::Channel (erase [.., dk], write [.., dv]) beside config 2's
    # per-head forget gate: the per-channel MFMA kernels with the head mask.
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260838)
    e = torch.sigmoid(torch.randn((B, T, H, K), generator=gen, device=dev))
    w = torch.sigmoid(torch.randn((B, T, H, V), generator=gen, device=dev))
    a = abi.chunk_fwd_args(q, k, v, e, w, g, s0, y, s1, 64, None)
    ws = torch.empty(max(abi.lib().dn_chunk_fwd_workspace_bytes(a), 1), dtype=torch.uint8,
                     device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    chosen = abi.lib().dn_chunk_fwd_algo(a)
    ms, kern = _timed(torch, abi, lambda: abi.run_chunk_fwd(a), steps, warmup)
    out["auto_channel_write_gates"] = {
        "gates": "erase [.., dk], write [.., dv], per-head forget gate",
        "algo": ALGO_NAMES.get(chosen, chosen), "ms_per_step": round(ms, 3),
        "tokens_per_s": round(B * T / (ms / 1e3), 1), "kernels": kern}
    del ws, e, w
    # head_k_dim 256 (config 2 otherwise): the MFMA forward under AUTO, and
    # the generic fp32 kernels it used to fall back to, forced.
    K2 = 256
    q2, k2, v2, beta2, g2 = gdn_inputs(torch, B, T, H, K2, V, 0.05, 20260839, torch.bfloat16, dev)
    s2 = torch.zeros((B, H, K2, V), dtype=torch.float32, device=dev)
    s3 = torch.empty_like(s2)
    wide = {"shape": "B=8 T=4096 H=16 dk=256 dv=256, per-head gates, chunk 64"}
    for name, algo in (("auto", 0), ("forced_generic", 1)):
        a = abi.chunk_fwd_args(q2, k2, v2, beta2, beta2, g2, s2, y, s3, 64, None, algo=algo)
        ws = torch.empty(max(abi.lib().dn_chunk_fwd_workspace_bytes(a), 1), dtype=torch.uint8,
                         device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        chosen = abi.lib().dn_chunk_fwd_algo(a)
        ms, kern = _timed(torch, abi, lambda: abi.run_chunk_fwd(a), steps if algo == 0 else 3,
                          warmup if algo == 0 else 1)
        wide[name] = {"algo": ALGO_NAMES.get(chosen, chosen), "ms_per_step": round(ms, 3),
                      "tokens_per_s": round(B * T / (ms / 1e3), 1), "kernels": kern}
        del ws
    # Per token against config 2 (dk = 128) on the same kernels at chunk 32.
    wide["per_token_cost_vs_config2"] = round(
        wide["auto"]["ms_per_step"] / out["auto_chunk32"]["ms_per_step"], 3)
    out["head_k_dim_256"] = wide
    return out


def bench_block_forward(torch, pkg, steps, warmup):
    """A Gated DeltaNet block's forward after in_proj at the config-2 shape
    (B=8, T=4096, H=16, dk=128, dv=256): the front-end (short conv of 4 with
    SiLU, L2 q/k norm, scalar β), the chunk forward (with a synthetic decay
    of config 2's distribution) and the gated output norm (bf16). The step is
    dn_frontend_chunk_fwd (the front-end's q/k formed in the chunk forward's
    load stage) then dn_out_norm; beside it the same block as three calls
    (dn_frontend, dn_chunk_fwd, dn_out_norm), each of them timed alone, and
    the core and the norm as one call (dn_chunk_fwd_out_norm)."""
    B, S, H, K, V, KC = 8, 4096, 16, 128, 256, 4
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260836)
    conv_dim = H * K * 2 + H * V
    width = conv_dim + H
    proj = torch.randn((B, S, width), generator=gen, device=dev).to(torch.bfloat16)
    weight = torch.randn((conv_dim, KC), generator=gen, device=dev) * 0.5
    win = torch.zeros((B, conv_dim, KC), dtype=torch.bfloat16, device=dev)
    wout = torch.empty_like(win)
    q = torch.empty((B, S, H, K), dtype=torch.bfloat16, device=dev)
    k, v = torch.empty_like(q), torch.empty((B, S, H, V), dtype=torch.bfloat16, device=dev)
    beta = torch.empty((B, S, H, 1), device=dev)
    g = -torch.nn.functional.softplus(torch.randn((B, S, H, 1), generator=gen, device=dev)) * 0.05
    z = torch.randn((B, S, H, V), generator=gen, device=dev).to(torch.bfloat16)
    gamma = torch.ones(V, device=dev)
    s0 = torch.zeros((B, H, K, V), device=dev)
    s1 = torch.empty_like(s0)
    y = torch.empty((B, S, H, V), dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(y)
    abi = pkg.abi
    fe = abi.frontend_args(proj, weight, None, win, wout, q, k, v, beta, beta, nheads=H,
                           head_k_dim=K, head_v_dim=V, n_householder=1,
                           conv_activation=abi.DN_ACT_SILU, qk_activation=abi.DN_ACT_SILU,
                           qk_norm=abi.DN_QKNORM_L2, write_gate=abi.DN_WRITE_SCALAR,
                           allow_neg_eigval=False)
    ca = abi.chunk_fwd_args(q, k, v, beta, beta, g, s0, y, s1, 64, None)
    ws = torch.empty(max(abi.lib().dn_chunk_fwd_workspace_bytes(ca), 1), dtype=torch.uint8,
                     device=dev)
    ca.workspace, ca.workspace_bytes = ws.data_ptr(), ws.numel()
    na = abi.out_norm_args(y, z, gamma, out, 1e-5)
    calls = {"frontend": lambda: abi.run_frontend(fe), "core": lambda: abi.run_chunk_fwd(ca),
             "out_norm": lambda: abi.run_out_norm(na)}

    def block():
        for f in calls.values():
            f()
    ms3, kern3 = _timed(torch, abi, block, steps, warmup)
    parts = {n: round(_timed(torch, abi, f, steps, warmup)[0], 4) for n, f in calls.items()}
    # The front-end's q/k in the chunk forward's load stage, then the norm.
    fca = abi.frontend_chunk_fwd_args(fe, ca)
    fcws = torch.empty(max(abi.lib().dn_frontend_chunk_fwd_workspace_bytes(fca), 1),
                       dtype=torch.uint8, device=dev)
    fca.fwd.workspace, fca.fwd.workspace_bytes = fcws.data_ptr(), fcws.numel()
    ona = abi.out_norm_args(y, z, gamma, out, 1e-5)

    def block_fe():
        abi.run_frontend_chunk_fwd(fca)
        abi.run_out_norm(ona)
    ms, kern = _timed(torch, abi, block_fe, steps, warmup)
    fe_core_ms = _timed(torch, abi, lambda: abi.run_frontend_chunk_fwd(fca), steps, warmup)[0]
    # The same block with the norm in the scan's output write
    # (dn_chunk_fwd_out_norm: y never round-trips through HBM).
    # The core and the norm as one call (dn_chunk_fwd_out_norm), the norm as
    # a pass of its own (the default) and in the scan's y write (in_scan).
    fa = abi.chunk_fwd_args(q, k, v, beta, beta, g, s0, out, s1, 64, None)
    cn = {}
    for mode in (False, True):
        na = abi.chunk_fwd_out_norm_args(fa, z, gamma, 1e-5, in_scan=mode)
        fws = torch.empty(max(abi.lib().dn_chunk_fwd_out_norm_workspace_bytes(na), 1),
                          dtype=torch.uint8, device=dev)
        na.fwd.workspace, na.fwd.workspace_bytes = fws.data_ptr(), fws.numel()
        cn[mode] = (na, fws)
    core_norm = lambda: abi.run_chunk_fwd_out_norm(cn[False][0])
    core_norm_in_scan = lambda: abi.run_chunk_fwd_out_norm(cn[True][0])

    def block_fused():
        abi.run_frontend(fe)
        core_norm()
    fms, fkern = _timed(torch, abi, block_fused, steps, warmup)
    cn_ms, cn_kern = _timed(torch, abi, core_norm, steps, warmup)
    cs_ms, cs_kern = _timed(torch, abi, core_norm_in_scan, steps, warmup)
    give_ups = abi.wait_give_ups()
    return {"workload": "Gated DeltaNet block forward after in_proj at the config-2 shape: "
                        "dn_frontend_chunk_fwd (front-end q/k in the load stage) + "
                        "dn_out_norm, bf16",
            "ms_per_step": round(ms, 4), "tokens_per_s": round(B * S / (ms / 1e3), 1),
            "kernels": kern,
            "frontend_chunk_fwd_ms": round(fe_core_ms, 4),
            "frontend_plus_core_ms": round(parts["frontend"] + parts["core"], 4),
            "three_calls": {"calls": "dn_frontend + dn_chunk_fwd + dn_out_norm",
                            "ms_per_step": round(ms3, 4), "kernels": kern3},
            "separate_ms": parts, "sum_of_separate_ms": round(sum(parts.values()), 4),
            "one_call_core": {"calls": "dn_frontend + dn_chunk_fwd_out_norm",
                           "ms_per_step": round(fms, 4),
                           "tokens_per_s": round(B * S / (fms / 1e3), 1), "kernels": fkern,
                           "core_with_norm_ms": round(cn_ms, 4),
                           "core_plus_out_norm_ms": round(parts["core"] + parts["out_norm"], 4),
                           "core_with_norm_in_scan_ms": round(cs_ms, 4),
                           "in_scan_kernels": cs_kern,
                           "wait_give_ups": give_ups}}


def _host_cpu():
    """nproc and the CPU model name of this host."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu": model}


def cpu_baseline(torch):
    """The oracle on the whole config-2 workload (B=8, H=16, T=4096: 32768
    tokens), fp32, on all available host threads (OMP_NUM_THREADS), repeated
    until 10 s have passed; beside it, one thread on one sequence (B=1), and
    the host's nproc and CPU model."""
    import numpy as np
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O
    B, T, H, K, V, L = 8, 4096, 16, 128, 256, 64
    rng = np.random.default_rng(20260828)
    l2 = lambda x: x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)
    q = l2(rng.standard_normal((B, T, H, K), dtype=np.float32))
    k = l2(rng.standard_normal((B, T, H, K), dtype=np.float32))
    v = rng.standard_normal((B, T, H, V), dtype=np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, H, 1))))).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal((B, T, H, 1)))) * 0.05).astype(np.float32)
    s0 = np.zeros((B, H, K, V), np.float32)
    threads = O.max_threads()
    O.chunk_fwd(q[:, :64], k[:, :64], v[:, :64], beta[:, :64], beta[:, :64], g[:, :64], s0,
                chunk_len=L, dtype=np.float32)
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < 10.0:
        O.chunk_fwd(q, k, v, beta, beta, g, s0, chunk_len=L, dtype=np.float32)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    # One thread, one sequence of the same workload (B=1: 4096 tokens).
    O.set_threads(1)
    try:
        t1 = time.perf_counter()
        O.chunk_fwd(q[:1], k[:1], v[:1], beta[:1], beta[:1], g[:1], s0[:1], chunk_len=L,
                    dtype=np.float32)
        d1 = time.perf_counter() - t1
    finally:
        O.set_threads(threads)
    return dict(value=B * T / dt, unit="tokens/s", cores=threads, kind="port",
                sample=f"full config 2 (B=8 H=16 T=4096 dk=128 dv=256, 32768 tokens), "
                       f"fp32, {threads} OpenMP threads, {reps} runs of {dt:.2f} s",
                single_thread={"value": round(T / d1, 1), "unit": "tokens/s", "cores": 1,
                               "sample": f"one sequence of config 2 (B=1, 4096 tokens), "
                                         f"fp32, 1 thread, {d1:.2f} s"},
                host=_host_cpu())


def mfma_from_profiles(kernel):
    """MFMA work the matrix cores executed per launch, from the committed
    rocprofv3 --pmc summary (MfmaFlopsBF16, MfmaFlopsF32, MfmaUtil), if any."""
    path = ROOT / "profiles" / "mfma.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(kernel)
    except (ValueError, OSError):
        return None


def traffic_from_profiles(kernel):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
        return data.get(kernel, {}).get("bytes_per_launch")
    except (ValueError, OSError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=100,
                    help="untimed steps right before the timed ones (after a "
                         f"{SETTLE_S} s run-in that lets the clocks ramp up)")
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--algo", choices=["auto", "generic", "mfma", "fused"], default="auto")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the config 4 and config 5 measurements")
    ap.add_argument("--extra-steps", type=int, default=MIN_STEPS,
                    help="timed calls for configs 4 and 5, the front-end and the output norm "
                         f"(at least {MIN_STEPS}, after at least {MIN_WARMUP} warm-ups)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="short run for rocprofv3 --pmc: a 1 GiB copy (calibration), then 2 "
                         "forward, 2 decode, 2 DeltaProduct-decode, 2 front-end and 2 "
                         "output-norm calls, one config-5 forward + backward, one config-4 "
                         "forward, one config-2-shape backward at head_k_dim 128 and one at "
                         "256, block decode and inverse calls; prints no JSON")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the delta-rule core shards over (batch, "
              "head) with no communication, and this build runs no "
              "multi-GPU path. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    pkg = load_package()
    algo = {"auto": 0, "generic": 1, "mfma": 2, "fused": 3}[args.algo]
    if args.profile_pass:
        _EXACT["on"] = True
        # Calibration: a plain device copy of exactly 1 GiB read + 1 GiB written.
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        bench_chunk_fwd(torch, pkg, 2, 0, 2)  # the two-kernel MFMA forward
        bench_chunk_fwd(torch, pkg, 2, 0, 3)  # the fused MFMA forward
        bench_decode(torch, pkg, 2, 0)
        bench_product_decode(torch, pkg, 2, 0)
        bench_frontend(torch, pkg, 2, 0)
        bench_out_norm(torch, pkg, 2, 0)
        bench_config5(torch, pkg, 1, 0)
        bench_config4(torch, pkg, 1, 0)
        bench_config2_bwd(torch, pkg, 1, 0)
        bench_config2_bwd(torch, pkg, 1, 0, K=256)
        bench_block_decode(torch, pkg, 2, 0)
        bench_unit_lower_inverse(torch, pkg, 2, 0)
        torch.cuda.synchronize()
        print("[bench] profile pass done", file=sys.stderr, flush=True)
        return
    print(f"[bench] chunk forward: config 2, {args.warmup} warmup + {args.steps} steps",
          file=sys.stderr, flush=True)
    fw = bench_chunk_fwd(torch, pkg, args.steps, args.warmup, algo)
    tok_s = fw["tokens"] / (fw["ms"] / 1e3)
    prof = fw["prof"]
    dom = max(prof, key=lambda n: prof[n][0]) if prof else None
    roof = None
    if dom:
        # The dominant kernel's launch duration: with one kernel per step the
        # timed region's per-step time (HIP events on the launch stream,
        # launch gaps included); otherwise that kernel's average from the
        # separate profile pass (HIP events around each launch on its stream).
        one_kernel = len(prof) == 1 and prof[dom][1] > 0
        prof_s = prof[dom][0] / prof[dom][1] / 1e3
        avg_s = fw["ms"] / 1e3 if one_kernel else prof_s
        # Algorithmic bytes per launch: the path's (every tensor crossing the
        # C ABI once), however many intermediates the kernel itself moves.
        nbytes = fw["path_bytes"]
        ach = nbytes / avg_s / 1e9
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                "traffic": traffic_from_profiles(dom),
                "avg_launch_us": round(avg_s * 1e6, 2),
                "avg_launch_source": "timed region" if one_kernel else "profile pass",
                "profile_pass_avg_us": round(prof_s * 1e6, 2),
                "algorithmic_bytes": nbytes,
                "algorithmic_bytes_per_chunk_head": nbytes // fw["chunk_heads"],
                "design_bytes": fw["kernel_bytes"].get(dom)}
        # What the matrix cores executed (rocprofv3 MfmaFlopsBF16/F32, bf16 hi/lo
        # splits included) over each forward kernel's profile-pass duration.
        mfma = {}
        for name, (tot_ms, n) in prof.items():
            mf = mfma_from_profiles(name)
            if mf and n:
                sec = tot_ms / n / 1e3
                mfma[name] = mf | {
                    "avg_launch_us": round(sec * 1e6, 2),
                    "executed_bf16_TFLOPs": round(mf["bf16_flop_per_launch"] / sec / 1e12, 1),
                    "executed_frac_of_bf16_peak": round(
                        mf["bf16_flop_per_launch"] / sec / 1e12 / BF16_PEAK_TFLOPS, 4)}
        if mfma:
            roof["mfma"] = mfma
    per_kernel = {n: {"avg_us": round(v[0] / v[1] * 1e3, 2), "launches": v[1]}
                  for n, v in prof.items()}
    print(f"[bench] forward {fw['ms']:.3f} ms/step, {tok_s:.3e} tokens/s, kernels "
          f"{per_kernel}", file=sys.stderr, flush=True)

    decode = None
    if not args.no_decode:
        print(f"[bench] decode: config 3, {args.decode_steps} steps", file=sys.stderr,
              flush=True)
        dc = bench_decode(torch, pkg, args.decode_steps, 10)
        # One dn_step_row launch per step, back to back: the timed region's
        # time per step is the kernel's average launch duration (rocprofv3's
        # average agrees); kernel_us is the profile pass's per-launch events.
        gbs = dc["bytes"] / (dc["us"] * 1e-6) / 1e9
        decode = {"us_per_step": round(dc["us"], 2), "kernel_us": round(dc["kernel_us"], 2),
                  "steps": args.decode_steps, "bytes_per_step": dc["bytes"],
                  "roofline": {"bound": "hbm", "kernel": dc["kernel"],
                               "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": round(gbs / HBM_PEAK_GBS, 4),
                               "avg_launch_source": "timed region, one kernel a step",
                               "traffic": traffic_from_profiles(dc["kernel"])}}
        print(f"[bench] decode {decode}", file=sys.stderr, flush=True)
        pd = bench_product_decode(torch, pkg, max(args.decode_steps // 5, 1), 5)
        pd["u_dn_step_kernel_us"] = round(2 * dc["kernel_us"], 2)  # the same token as 2 ticks
        decode["product_u2"] = pd
        print(f"[bench] DeltaProduct decode {pd}", file=sys.stderr, flush=True)

    extra = {}
    other = {2: 3, 3: 2}.get(fw["algo"])
    if not args.no_extra and other:
        # The same workload through the other MFMA forward: the two-kernel
        # path (tiles through HBM) or the fused kernel (tiles in LDS).
        print(f"[bench] config 2 forward, {ALGO_NAMES[other]}", file=sys.stderr, flush=True)
        ff = bench_chunk_fwd(torch, pkg, args.extra_steps, MIN_WARMUP, other)
        ff_gbs = ff["path_bytes"] / (ff["ms"] / 1e3) / 1e9
        extra["other_mfma_forward"] = {
            "algo": ALGO_NAMES[other],
            "ms_per_step": round(ff["ms"], 4),
            "tokens_per_s": round(ff["tokens"] / (ff["ms"] / 1e3), 1),
            "kernels": {n: round(v[0] / v[1] * 1e3, 2) for n, v in ff["prof"].items()},
            "path_frac_of_hbm": round(ff_gbs / HBM_PEAK_GBS, 4),
            "traffic": {n: traffic_from_profiles(n) for n in ff["prof"]}}
        print(f"[bench] other MFMA forward {extra['other_mfma_forward']}", file=sys.stderr,
              flush=True)
        torch.cuda.empty_cache()
    if not args.no_extra:
        print("[bench] config 4 (DeltaProduct fold)", file=sys.stderr, flush=True)
        extra["config4"] = bench_config4(torch, pkg, args.extra_steps, MIN_WARMUP)
        print(f"[bench] config4 {extra['config4']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        print("[bench] config 5 (GDN-2 forward + backward)", file=sys.stderr, flush=True)
        extra["config5"] = bench_config5(torch, pkg, args.extra_steps, MIN_WARMUP)
        print(f"[bench] config5 {extra['config5']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        print("[bench] config-2 shape backward", file=sys.stderr, flush=True)
        extra["config2_backward"] = bench_config2_bwd(torch, pkg, args.extra_steps, MIN_WARMUP)
        # head_v_dim 192: a pass of 128 value columns and one of 64.
        b192 = bench_config2_bwd(torch, pkg, args.extra_steps, MIN_WARMUP, V=192)
        extra["config2_backward"]["head_v_dim_192"] = {
            k: b192[k] for k in ("algo", "ms_per_call", "tokens_per_s", "kernels")}
        # head_k_dim 256: each value pass of the chunk-local kernel as two
        # launches over the key halves (103 ms on the generic kernels).
        b256 = bench_config2_bwd(torch, pkg, args.extra_steps, MIN_WARMUP, K=256)
        extra["config2_backward"]["head_k_dim_256"] = {
            k: b256[k] for k in ("algo", "ms_per_call", "tokens_per_s", "roofline", "kernels")}
        print(f"[bench] config2_backward {extra['config2_backward']}", file=sys.stderr,
              flush=True)
        torch.cuda.empty_cache()
        print("[bench] block forward (front-end + core + out norm)", file=sys.stderr, flush=True)
        extra["block_forward"] = bench_block_forward(torch, pkg, args.extra_steps, MIN_WARMUP)
        print(f"[bench] block_forward {extra['block_forward']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        print("[bench] chunk lengths", file=sys.stderr, flush=True)
        extra["chunk_lengths"] = bench_chunk_lengths(torch, pkg, MIN_STEPS, MIN_WARMUP)
        print(f"[bench] chunk_lengths {extra['chunk_lengths']}", file=sys.stderr,
              flush=True)
        torch.cuda.empty_cache()
        print("[bench] projection front-end (dn_frontend)", file=sys.stderr, flush=True)
        extra["frontend"] = bench_frontend(torch, pkg, args.extra_steps, MIN_WARMUP)
        print(f"[bench] frontend {extra['frontend']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        print("[bench] output norm (dn_out_norm)", file=sys.stderr, flush=True)
        extra["out_norm"] = bench_out_norm(torch, pkg, args.extra_steps, MIN_WARMUP)
        print(f"[bench] out_norm {extra['out_norm']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        print("[bench] block decode (dn_block_step)", file=sys.stderr, flush=True)
        extra["block_decode"] = bench_block_decode(torch, pkg, args.extra_steps, MIN_WARMUP)
        print(f"[bench] block_decode {extra['block_decode']}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
        print("[bench] unit_lower_inverse", file=sys.stderr, flush=True)
        extra["unit_lower_inverse"] = bench_unit_lower_inverse(torch, pkg, MIN_STEPS, MIN_WARMUP)
        print(f"[bench] unit_lower_inverse {extra['unit_lower_inverse']}", file=sys.stderr,
              flush=True)
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline (oracle)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(torch)
        cpu["value"] = round(cpu["value"], 1)

    path_gbs = fw["path_bytes"] / (fw["ms"] / 1e3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": SETTLE_S,
        "ms_per_step": round(fw["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config 2: Gated DeltaNet chunkwise prefill (core forward)",
                   "batch": 8, "seq_len": 4096, "nheads": 16, "head_k_dim": 128,
                   "head_v_dim": 256, "chunk_len": 64, "qkv": "bf16", "state": "fp32",
                   "y": "bf16",
                   "algo": ALGO_NAMES.get(fw["algo"], fw["algo"])},
        "roofline": roof,
        "path_roofline": {"bound": "hbm", "achieved": round(path_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(path_gbs / HBM_PEAK_GBS, 4),
                          "algorithmic_bytes": fw["path_bytes"],
                          "mfma_TFLOPs": round(fw["path_flops"] / (fw["ms"] / 1e3) / 1e12, 2)},
        "kernels": per_kernel,
        "decode": decode,
        **extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
