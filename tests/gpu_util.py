"""Helpers shared by the GPU parity tests: seeded inputs moved to the GPU,
and the bf16 rounding the oracle is fed when the GPU path reads bf16."""

from __future__ import annotations

import sys

import numpy as np
import torch

from conftest import load_package, random_raw, rel_err  # noqa: F401

pkg = load_package()
DEV = torch.device("cuda:0")


def announce(what: str) -> None:
    print(f"[gpu] {what}", flush=True)
    sys.stdout.flush()


def to_gpu(args, qkv_dtype=torch.float32):
    """numpy (q, k, v, erase, write, g, state) → GPU tensors; q/k/v in qkv_dtype."""
    out = []
    for i, a in enumerate(args):
        if a is None:
            out.append(None)
            continue
        dt = qkv_dtype if i < 3 else torch.float32
        out.append(torch.tensor(np.ascontiguousarray(a), dtype=torch.float32, device=DEV).to(dt))
    return out


def as_oracle_inputs(gpu_args):
    """What the GPU path actually reads, in float64 for the oracle."""
    return [None if t is None else t.float().cpu().numpy().astype(np.float64) for t in gpu_args]


def np_of(t):
    return t.float().cpu().numpy()
