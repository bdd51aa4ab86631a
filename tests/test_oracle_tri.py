"""The oracle's blocked ladder (src/delta/tri/prim.rs:28-51) against what the
mathematics fixes. Mirrors src/delta/tri/tests.rs."""

import numpy as np
import pytest

from oracle import oracle as O


def strict_lower(rng, batch, size, scale):
    return np.tril(rng.normal(0.0, scale, (batch, size, size)), -1)


@pytest.mark.parametrize("size", [1, 2, 3, 4, 5, 7, 8, 16, 32, 64, 128])
def test_blocked_inverts(rng, size):
    """(I − N) T = I (tri/tests.rs:21-48), and T equals numpy's inverse."""
    n = strict_lower(rng, 3, size, 0.3)
    t = O.unit_lower_inverse(n)
    eye = np.eye(size)
    assert np.abs((eye - n) @ t - eye).max() < 1e-10
    assert np.abs(t - np.linalg.inv(eye - n)).max() < 1e-8 * max(1.0, np.abs(t).max())
    t32 = O.unit_lower_inverse(n, dtype=np.float32)
    assert np.abs((eye - n) @ t32 - eye).max() < 1e-3


def test_inverse_is_unit_lower_triangular(rng):
    """tri/tests.rs:84-98."""
    t = O.unit_lower_inverse(strict_lower(rng, 2, 8, 0.5))
    assert np.abs(np.triu(t, 1)).max() == 0.0
    assert np.abs(np.diagonal(t, axis1=1, axis2=2) - 1.0).max() < 1e-12


@pytest.mark.parametrize("size", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("beta", [0.9, 1.0, 1.9])
def test_constant_key_chunk_stays_bounded(size, beta):
    """tri/tests.rs:106-128: N = −β on the strict lower triangle; T is a
    differencing matrix bounded by max(1, β), in float32 too."""
    n = np.tril(np.full((size, size), -beta), -1)
    for dtype, tol in [(np.float64, 1e-10), (np.float32, 1e-4)]:
        t = O.unit_lower_inverse(n, dtype=dtype)
        eye = np.eye(size)
        assert np.abs((eye - n) @ t - eye).max() < tol
        assert np.abs(t).max() <= max(beta, 1.0) + 1e-4
    # Closed form: T[i][j] = −β(1 − β)^{i−j−1} below the diagonal.
    t = O.unit_lower_inverse(n)
    i, j = 5, 2
    assert abs(t[i, j] - (-beta * (1 - beta) ** (i - j - 1))) < 1e-12


@pytest.mark.parametrize("size", [1, 2, 3, 4, 5, 7, 8, 16, 32])
def test_neumann_equals_the_ladder_on_strict_lower_input(rng, size):
    """tri/tests.rs:40-46 and :50-82: where the series is conditioned both
    solves are the same function; in float64 they agree to rounding."""
    n = strict_lower(rng, 3, size, 0.3)
    t = O.neumann_inverse(n)
    assert np.abs(t - O.unit_lower_inverse(n)).max() < 1e-12
    t32 = O.neumann_inverse(n, dtype=np.float32)
    eye = np.eye(size)
    assert np.abs((eye - n) @ t32 - eye).max() < 1e-3


def test_neumann_multiplies_the_whole_matrix(rng):
    """tri.rs:99-107 multiplies N as given (tri/tests.rs:55-58: the two solves
    disagree about entries on and above the diagonal). On a full matrix the
    result is the truncated series Σ_{j<size} Nʲ, formed here from numpy's
    matrix powers; the ladder ignores those entries."""
    size = 6
    n = rng.normal(0.0, 0.2, (size, size))
    want = sum(np.linalg.matrix_power(n, j) for j in range(size))
    assert np.abs(O.neumann_inverse(n) - want).max() < 1e-12
    assert np.abs(O.unit_lower_inverse(n) - O.unit_lower_inverse(np.tril(n, -1))).max() == 0.0


def test_neumann_closed_form_on_a_constant_key_chunk():
    """N = −β on the strict lower triangle, at a size where the series is still
    conditioned in float64: T[i][j] = −β(1 − β)^{i−j−1} below the diagonal."""
    size, beta = 8, 0.5
    n = np.tril(np.full((size, size), -beta), -1)
    t = O.neumann_inverse(n)
    i, j = np.tril_indices(size, -1)
    assert np.abs(t[i, j] - (-beta * (1 - beta) ** (i - j - 1))).max() < 1e-12
    assert np.abs(np.diagonal(t) - 1.0).max() == 0.0
