"""The oracle against the reference's FLA float64 fixture.

Mirrors matches_the_reference_delta_rule / _gated_delta_rule / _gdn2
(src/delta/tests.rs:533-568, 760-812): Recurrent and chunk_len 3/4/16 must
reproduce flash-linear-attention's naive recurrences on DIMS = [2, 9, 2, 4, 6].
The reference asserts 1e-4 absolute; FLA's naive code computes in float32, so
the float64 oracle is held to 1e-6 and the float32 oracle to 1e-5.
"""

import numpy as np
import pytest

from conftest import fla_fixture
from oracle import oracle as O

CASES = ["ungated", "gated", "gdn2"]


def inputs(case):
    _, a = fla_fixture()
    beta = a["IN_BETA"][..., None]
    if case == "ungated":
        return (a["IN_Q"], a["IN_K"], a["IN_V"], beta, beta, None, a["IN_STATE"]), \
            a["UNGATED_Y"], a["UNGATED_STATE"]
    if case == "gated":
        return (a["IN_Q"], a["IN_K"], a["IN_V"], beta, beta, a["IN_G"][..., None],
                a["IN_STATE"]), a["GATED_Y"], a["GATED_STATE"]
    return (a["IN_Q"], a["IN_K"], a["IN_V"], a["IN_B"], a["IN_W"], a["IN_GK"], a["IN_STATE"]), \
        a["GDN2_Y"], a["GDN2_STATE"]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-6), (np.float32, 1e-5)])
def test_recurrent_matches_fla(case, dtype, tol):
    args, want_y, want_s = inputs(case)
    y, s = O.recurrent(*args, dtype=dtype)
    assert np.abs(y - want_y).max() < tol
    assert np.abs(s - want_s).max() < tol


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("chunk_len", [1, 3, 4, 16, 64])
@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-6), (np.float32, 1e-5)])
def test_chunk_matches_fla(case, chunk_len, dtype, tol):
    args, want_y, want_s = inputs(case)
    y, s = O.chunk_fwd(*args, chunk_len=chunk_len, dtype=dtype)
    assert np.abs(y - want_y).max() < tol
    assert np.abs(s - want_s).max() < tol


def test_fixture_detects_a_dropped_decay():
    """A plausible bug planted in the oracle's inputs (the forget gate dropped)
    must fail the fixture by far more than the tolerance."""
    args, want_y, _ = inputs("gated")
    bad = list(args)
    bad[5] = None
    y, _ = O.recurrent(*bad)
    assert np.abs(y - want_y).max() > 1e-3


def test_step_is_one_recurrent_tick():
    """delta_step on [B,H,·] equals the first token of delta_recurrent."""
    args, _, _ = inputs("gdn2")
    one = [a[:, :1] if a is not None and a.ndim == 4 and a.shape[1] == 9 else a for a in args]
    y_seq, s_seq = O.recurrent(*one)
    step_args = [a[:, 0] if a is not None and a.ndim == 4 and a.shape[1] == 1 else a
                 for a in one]
    step_args[6] = args[6]
    y, s = O.delta_step(*step_args)
    np.testing.assert_allclose(y, y_seq[:, 0], atol=1e-12)
    np.testing.assert_allclose(s, s_seq, atol=1e-12)
