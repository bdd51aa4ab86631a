"""Invariants and closed forms of the delta rule, checked on the oracle.

Mirrors src/delta/tests.rs (path equivalence :257-337, chunk_len invariance
:341-363, constant input :373-460, split stream :465-494, g=0 ≡ None
:573-602, broadcast ≡ channel :711-756) and the closed-form semantics of
gated_deltanet_2/tests.rs:461-526.
"""

import numpy as np
import pytest

from conftest import clamp_regime_case, closed_form_err, l2, random_raw
from oracle import oracle as O


@pytest.mark.parametrize("case", [
    (2, 16, 3, 8, 8, 8, 0.95, False, False, False),
    (2, 16, 3, 8, 8, 8, 0.95, True, False, False),
    (2, 12, 2, 8, 16, 4, 0.95, True, True, False),
    (2, 12, 2, 8, 8, 6, 1.95, True, True, False),
    (2, 13, 2, 8, 8, 8, 0.95, True, True, False),
    (1, 5, 1, 4, 4, 8, 0.95, False, False, False),
    (2, 16, 3, 8, 8, 8, 0.95, True, False, True),
    (2, 40, 2, 8, 8, 32, 0.95, True, True, True),
    (1, 37, 1, 4, 6, 16, 1.95, True, True, True),
])
@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-10), (np.float32, 1e-4)])
def test_chunk_matches_recurrent(rng, case, dtype, tol):
    B, S, H, K, V, L, beta_max, gated, random_state, channel = case
    args = random_raw(rng, B, S, H, K, V, beta_max, gated, random_state, channel)
    y0, s0 = O.recurrent(*args)
    y, s = O.chunk_fwd(*args, chunk_len=L, dtype=dtype)
    assert np.abs(y - y0).max() < tol
    assert np.abs(s - s0).max() < tol


@pytest.mark.parametrize("channel", [False, True])
def test_chunk_len_does_not_change_the_answer(rng, channel):
    args = random_raw(rng, 2, 24, 2, 8, 8, 0.95, True, True, channel)
    y0, s0 = O.chunk_fwd(*args, chunk_len=4)
    for L in [1, 3, 6, 8, 12, 16, 24, 32]:
        y, s = O.chunk_fwd(*args, chunk_len=L)
        assert np.abs(y - y0).max() < 1e-10 and np.abs(s - s0).max() < 1e-10


def constant_raw(rng, B, S, H, K, V, beta, gated):
    """src/delta/tests.rs:373-420: one direction per (b, h) held for S tokens."""
    hold = lambda a: np.broadcast_to(a, (B, S, H, a.shape[-1])).copy()
    q = hold(l2(rng.standard_normal((B, 1, H, K))))
    k = hold(l2(rng.standard_normal((B, 1, H, K))))
    v = hold(rng.standard_normal((B, 1, H, V)))
    erase = np.full((B, S, H, 1), beta)
    g = np.full((B, S, H, 1), -0.05) if gated else None
    return [q, k, v, erase, erase.copy(), g, np.zeros((B, H, K, V))]


@pytest.mark.parametrize("beta,gated", [(0.9, False), (0.9, True), (1.8, True)])
def test_constant_input_survives_every_chunk_length(rng, beta, gated):
    args = constant_raw(rng, 2, 128, 2, 8, 8, beta, gated)
    y0, s0 = O.recurrent(*args)
    for L in [16, 32, 48, 64, 128]:
        y, s = O.chunk_fwd(*args, chunk_len=L, dtype=np.float32)
        assert np.isfinite(y).all()
        assert np.abs(y - y0).max() < 1e-3 and np.abs(s - s0).max() < 1e-3


def test_split_calls_match_a_single_call(rng):
    q, k, v, e, w, g, s = random_raw(rng, 2, 20, 2, 8, 8, 0.95, True, False)
    y_all, s_all = O.chunk_fwd(q, k, v, e, w, g, s, chunk_len=4)
    cut = lambda a, sl: a[:, sl]
    y1, s_mid = O.chunk_fwd(*(cut(a, slice(0, 7)) for a in (q, k, v, e, w, g)), s, chunk_len=4)
    y2, s_end = O.chunk_fwd(*(cut(a, slice(7, 20)) for a in (q, k, v, e, w, g)), s_mid,
                            chunk_len=4)
    assert np.abs(np.concatenate([y1, y2], 1) - y_all).max() < 1e-10
    assert np.abs(s_end - s_all).max() < 1e-10


def test_zero_gate_is_the_ungated_rule(rng):
    q, k, v, e, w, _, s = random_raw(rng, 2, 12, 2, 8, 8, 0.95, False, True)
    zeros = np.zeros((2, 12, 2, 1))
    for run in (O.recurrent, lambda *a: O.chunk_fwd(*a, chunk_len=5)):
        y0, s0 = run(q, k, v, e, w, None, s)
        y1, s1 = run(q, k, v, e, w, zeros, s)
        assert np.abs(y0 - y1).max() < 1e-12 and np.abs(s0 - s1).max() < 1e-12


def test_broadcast_channel_gates_are_the_scalar_rule(rng):
    q, k, v, e, w, g, s = random_raw(rng, 2, 20, 2, 8, 12, 0.95, True, True)
    widen = lambda a, n: np.broadcast_to(a, a.shape[:-1] + (n,)).copy()
    for run in (O.recurrent, lambda *a: O.chunk_fwd(*a, chunk_len=8)):
        y0, s0 = run(q, k, v, e, w, g, s)
        y1, s1 = run(q, k, v, widen(e, 8), widen(w, 12), widen(g, 8), s)
        assert np.abs(y0 - y1).max() < 1e-10 and np.abs(s0 - s1).max() < 1e-10


def test_closed_form_write_accumulate_and_fixed_point(rng):
    """gated_deltanet_2/tests.rs:461-526: b=w=1 stores v; b=0,w=1 adds v again;
    a shared β leaves a stored v where it is."""
    K, V = 4, 3
    k = l2(rng.standard_normal((1, 1, K)))
    v = rng.standard_normal((1, 1, V))
    one = np.ones((1, 1, 1))
    zero = np.zeros((1, 1, 1))
    stored, state = O.delta_step(k, k, v, one, one, None, np.zeros((1, 1, K, V)), scale=1.0)
    assert np.abs(stored - v).max() < 1e-5
    doubled, _ = O.delta_step(k, k, v, zero, one, None, state, scale=1.0)
    assert np.abs(doubled - 2 * v).max() < 1e-5
    for beta in [0.25, 0.5, 1.0, 2.0]:
        kept, _ = O.delta_step(k, k, v, one * beta, one * beta, None, state, scale=1.0)
        assert np.abs(kept - v).max() < 1e-5


def test_deltaproduct_fold_with_one_householder_is_gdn1(rng):
    """delta_product/tests.rs:192-225 on the core: with u = 1 the fold of
    delta_product.rs:178-205 is the identity, and with u = 2 and the second
    micro-step's key/erase zero the folded run equals the unfolded one."""
    q, k, v, e, w, g, s = random_raw(rng, 1, 9, 2, 4, 6, 1.95, True, True)
    y0, s0 = O.chunk_fwd(q, k, v, e, w, g, s, chunk_len=4)

    def fold(first, last):  # [B,S,H,·] x2 → [B,2S,H,·] interleaved
        out = np.stack([first, last], 2)
        return out.reshape(out.shape[0], -1, *out.shape[3:])

    zq = np.zeros_like(q)
    y, s1 = O.chunk_fwd(fold(zq, q), fold(k, np.zeros_like(k)), fold(v, np.zeros_like(v)),
                        fold(e, np.zeros_like(e)), fold(w, np.zeros_like(w)),
                        fold(g, np.zeros_like(g)), s, chunk_len=4)
    assert np.abs(y[:, 1::2] - y0).max() < 1e-10
    assert np.abs(s1 - s0).max() < 1e-10


@pytest.mark.parametrize("chunk_len", [16, 64])
def test_block_decay_clamp_closed_form(chunk_len):
    """The per-channel decay where its clamp binds (decay.rs:41-49), forward
    and backward, against the closed forms of conftest.clamp_regime_case."""
    args, dy, want = clamp_regime_case()
    y, s = O.chunk_fwd(*args, chunk_len=chunk_len)
    rel, rest = closed_form_err(y, want["y"])
    assert rel < 1e-12 and rest < 1e-12
    assert np.abs(s).max() < 1e-200
    grads = O.chunk_bwd(dy, np.zeros_like(args[6]), *args, chunk_len=chunk_len)
    for name, got in zip(["d_q", "d_k", "d_v", "d_erase", "d_write", "d_g"], grads):
        rel, rest = closed_form_err(got, want[name])
        assert rel < 1e-12 and rest < 1e-12, (name, rel, rest)
