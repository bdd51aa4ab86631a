"""The oracle's hand-written backward (combined_backward.rs:72-538) against two
independent derivatives of the recurrence:

* central finite differences of the float64 recurrent oracle, and
* torch float64 autograd of a recurrence written here, token by token.

The loss is the reference's (src/delta/tests.rs:194-218): Σ y⊙Y + Σ S⊙Ŝ with
two random heads. The reference itself pins gradients only relative to its own
Recurrent path, so these checks are what pins gradient parity.
"""

import numpy as np
import pytest
import torch

from conftest import random_raw
from oracle import oracle as O

NAMES = ["q", "k", "v", "erase", "write", "g", "state"]


def loss_fn(args, y_head, s_head, chunk_len=None):
    if chunk_len is None:
        y, s = O.recurrent(*args)
    else:
        y, s = O.chunk_fwd(*args, chunk_len=chunk_len)
    return float((y * y_head).sum() + (s * s_head).sum())


def finite_difference(args, y_head, s_head, eps=1e-6):
    grads = []
    for idx, a in enumerate(args):
        if a is None:
            grads.append(None)
            continue
        gr = np.zeros_like(a)
        flat = a.reshape(-1)
        for i in range(flat.size):
            old = flat[i]
            flat[i] = old + eps
            up = loss_fn(args, y_head, s_head)
            flat[i] = old - eps
            dn = loss_fn(args, y_head, s_head)
            flat[i] = old
            gr.reshape(-1)[i] = (up - dn) / (2 * eps)
        grads.append(gr)
    return grads


def torch_recurrence_grads(args, y_head, s_head):
    """delta_step semantics (recurrent.rs:41-99), written independently."""
    ts = [None if a is None else torch.tensor(a, dtype=torch.float64, requires_grad=True)
          for a in args]
    q, k, v, e, w, g, s = ts
    B, S, H, K = q.shape
    scale = 1.0 / K ** 0.5
    ys = []
    for t in range(S):
        if g is not None:
            s = s * torch.exp(g[:, t]).unsqueeze(-1)          # [B,H,1|K,1]
        erased = torch.einsum("bhk,bhkv->bhv", k[:, t] * e[:, t], s)
        u = v[:, t] * w[:, t] - erased
        s = s + k[:, t].unsqueeze(-1) * u.unsqueeze(-2)
        ys.append(torch.einsum("bhk,bhkv->bhv", q[:, t] * scale, s))
    y = torch.stack(ys, 1)
    loss = (y * torch.tensor(y_head)).sum() + (s * torch.tensor(s_head)).sum()
    loss.backward()
    return [None if x is None else x.grad.numpy() for x in ts]


CASES = [
    # B, S, H, K, V, chunk_len, beta_max, gated, channel
    (1, 5, 1, 3, 4, 2, 0.95, False, False),
    (1, 7, 2, 4, 3, 3, 0.95, True, False),
    (1, 6, 1, 4, 5, 4, 1.95, True, False),
    (1, 9, 1, 4, 6, 4, 0.95, True, True),
    (1, 11, 1, 3, 2, 8, 1.95, True, True),
    (2, 5, 1, 4, 4, 8, 0.95, True, True),
]


@pytest.mark.parametrize("case", CASES)
def test_backward_matches_finite_differences(rng, case):
    B, S, H, K, V, L, beta_max, gated, channel = case
    args = random_raw(rng, B, S, H, K, V, beta_max, gated, True, channel)
    y_head = rng.standard_normal((B, S, H, V))
    s_head = rng.standard_normal((B, H, K, V))
    fd = finite_difference(args, y_head, s_head)
    got = O.chunk_bwd(y_head, s_head, *args, chunk_len=L)
    for name, a, b in zip(NAMES, got, fd):
        if b is None:
            assert a is None
            continue
        err = np.abs(a - b).max()
        assert err < 1e-6 * max(1.0, np.abs(b).max()), (name, err)


CASES_LARGE = [
    (2, 24, 2, 8, 8, 8, 0.95, True, False),
    (2, 37, 2, 4, 6, 16, 0.95, True, True),
    (2, 40, 2, 8, 8, 32, 0.95, True, True),
    (1, 13, 2, 8, 16, 5, 1.95, False, False),
    (2, 24, 2, 8, 8, 1, 0.95, True, True),
]


@pytest.mark.parametrize("case", CASES_LARGE)
def test_backward_matches_torch_autograd(rng, case):
    B, S, H, K, V, L, beta_max, gated, channel = case
    args = random_raw(rng, B, S, H, K, V, beta_max, gated, True, channel)
    y_head = rng.standard_normal((B, S, H, V))
    s_head = rng.standard_normal((B, H, K, V))
    want = torch_recurrence_grads(args, y_head, s_head)
    got = O.chunk_bwd(y_head, s_head, *args, chunk_len=L)
    for name, a, b in zip(NAMES, got, want):
        if b is None:
            assert a is None
            continue
        assert np.abs(a - b).max() < 1e-9 * max(1.0, np.abs(b).max()), name
    # float32 oracle within the reference's own custom-vs-taped tolerance
    got32 = O.chunk_bwd(y_head, s_head, *args, chunk_len=L, dtype=np.float32)
    for name, a, b in zip(NAMES, got32, want):
        if b is None:
            continue
        assert np.abs(a - b).max() < 2e-3 * max(1.0, np.abs(b).max()), name


def test_backward_detects_a_sign_error(rng):
    """Planting a sign error in the upstream state cotangent must move d_state."""
    args = random_raw(rng, 1, 9, 1, 4, 6, 0.95, True, True, True)
    y_head = rng.standard_normal((1, 9, 1, 6))
    s_head = rng.standard_normal((1, 1, 4, 6))
    good = O.chunk_bwd(y_head, s_head, *args, chunk_len=4)
    bad = O.chunk_bwd(y_head, -s_head, *args, chunk_len=4)
    assert np.abs(good[6] - bad[6]).max() > 1e-2
