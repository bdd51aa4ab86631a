"""dn_unit_lower_inverse, the standalone unit_lower_inverse
(src/delta/tri.rs:66-114), on the GPU through its Python mirror.

Checks: the reference's own tests (src/delta/tri/tests.rs: (I − N)·T = I,
Blocked ≡ Neumann where the series is conditioned, unit lower structure, the
constant-key chunk's bound), and the oracle in float64 on the same float32
inputs: the ladder of tri/prim.rs:28-51 for Blocked and the term-by-term
series of tri.rs:99-107 for Neumann (both pinned in tests/test_oracle_tri.py).
Sizes cover the four kernels: the blocked substitution (size ≤ 64), its
doubling to two 64-blocks (65…128), the panel substitution with its columns
in LDS (129…256) and read back from T (above 256), and the series (up to
140). Bar: float32 arithmetic, normwise
relative 2e-5 against the float64 oracle for Blocked; the reference's 1e-3
and 1e-4 for its own checks."""

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, pkg
from oracle import oracle as O

pytestmark = pytest.mark.gpu

abi = pkg.abi
BLOCKED, NEUMANN = pkg.TriSolve.BLOCKED, pkg.TriSolve.NEUMANN


def strict_lower(rng, batch, size, scale):
    return np.tril(rng.normal(0.0, scale, (batch, size, size)), -1).astype(np.float32)


def inv(n, solve=BLOCKED):
    t = pkg.unit_lower_inverse(torch.tensor(n, dtype=torch.float32, device=DEV), solve)
    torch.cuda.synchronize()
    return t.cpu().numpy().astype(np.float64)


def rel(a, b):
    return np.abs(a - b).max() / max(np.abs(b).max(), 1.0)


@pytest.mark.parametrize("size", [1, 2, 3, 4, 5, 7, 8, 16, 32, 64, 65, 100, 127, 128, 129, 200, 257, 300])
def test_blocked_inverts(rng, size):
    """tri/tests.rs:21-48 (sizes 1…128, entries of scale 0.3) and the oracle's
    ladder. Past 128 the entries are of scale 0.1: at 0.3, T's entries grow to
    ~10⁴ by size 257, and even T rounded once to float32 then leaves a
    residual above 1e-3."""
    announce(f"unit_lower_inverse blocked size {size}")
    n = strict_lower(rng, 3, size, 0.3 if size <= 128 else 0.1)
    t = inv(n)
    eye = np.eye(size)
    assert np.abs((eye - n) @ t - eye).max() < 1e-3
    e = rel(t, O.unit_lower_inverse(n.astype(np.float64)))
    print(f"  vs float64 ladder: {e:.2e}", flush=True)
    assert e < 2e-5


@pytest.mark.parametrize("size", [1, 2, 3, 4, 5, 7, 8, 16, 32])
def test_neumann_inverts(rng, size):
    """tri/tests.rs:43-48 and the oracle's series."""
    announce(f"unit_lower_inverse neumann size {size}")
    n = strict_lower(rng, 3, size, 0.3)
    t = inv(n, NEUMANN)
    eye = np.eye(size)
    assert np.abs((eye - n) @ t - eye).max() < 1e-3
    assert rel(t, O.neumann_inverse(n.astype(np.float64))) < 2e-5


def test_neumann_at_its_largest_size(rng):
    size = abi.TRI_NEUMANN_MAX_SIZE
    announce(f"unit_lower_inverse neumann size {size}")
    n = strict_lower(rng, 2, size, 0.02)
    t = inv(n, NEUMANN)
    assert rel(t, O.unit_lower_inverse(n.astype(np.float64))) < 2e-5
    assert rel(t, inv(n)) < 2e-5


def test_blocked_matches_neumann(rng):
    """tri/tests.rs:50-82 (values): size 16, where the series is conditioned."""
    announce("unit_lower_inverse blocked vs neumann")
    n = strict_lower(rng, 2, 16, 0.3)
    assert np.abs(inv(n) - inv(n, NEUMANN)).max() < 1e-4


def test_neumann_multiplies_the_whole_matrix_and_blocked_reads_the_strict_lower(rng):
    """tri/tests.rs:55-58: the solves disagree about entries on and above the
    diagonal. The series multiplies them in (the oracle's truncated series of
    the full matrix); the blocked solve ignores them."""
    announce("unit_lower_inverse on a full matrix")
    for size in (6, 40, 90):
        n = rng.normal(0.0, 0.2 / np.sqrt(size), (2, size, size)).astype(np.float32)
        if size <= abi.TRI_NEUMANN_MAX_SIZE:
            assert rel(inv(n, NEUMANN), O.neumann_inverse(n.astype(np.float64))) < 2e-5
        assert np.array_equal(inv(n), inv(np.tril(n, -1)))


@pytest.mark.parametrize("size", [8, 100])
def test_inverse_is_unit_lower_triangular(rng, size):
    """tri/tests.rs:84-98, exactly: nothing is written above the diagonal and
    the diagonal is 1."""
    announce(f"unit_lower_inverse structure size {size}")
    t = inv(strict_lower(rng, 2, size, 0.5))
    assert np.abs(np.triu(t, 1)).max() == 0.0
    assert np.array_equal(np.diagonal(t, axis1=1, axis2=2), np.ones((2, size)))


@pytest.mark.parametrize("size", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("beta", [0.9, 1.0, 1.9])
def test_blocked_inverts_a_constant_key_chunk(size, beta):
    """tri/tests.rs:100-128: N = −β on the strict lower triangle. (I − N)·T = I
    at 1e-4 and no entry above max(1, β); the closed form
    T[i][j] = −β(1 − β)^{i−j−1} below the diagonal, at 1e-5 up to size 64.
    Past 64 the last doubling, T₂₁ = −T₂₂·(A₂₁·T₁₁), sums 64 float32
    products of entries up to β² of alternating sign: 4e-5 there."""
    announce(f"unit_lower_inverse constant keys size {size} beta {beta}")
    n = np.tril(np.full((size, size), -beta, dtype=np.float32), -1)
    t = inv(n)
    eye = np.eye(size)
    assert np.abs((eye - n) @ t - eye).max() < 1e-4
    assert np.abs(t).max() <= max(beta, 1.0) + 1e-4
    i, j = np.tril_indices(size, -1)
    tol = 1e-5 if size <= 64 else 4e-5
    assert np.abs(t[i, j] - (-beta * (1 - beta) ** (i - j - 1))).max() < tol


def test_leading_axes_and_dtype(rng):
    """[..., size, size] of any leading axes; the result keeps N's dtype."""
    announce("unit_lower_inverse leading axes, bf16")
    n = strict_lower(rng, 6, 24, 0.3).reshape(2, 3, 24, 24)
    nb = torch.tensor(n, device=DEV).to(torch.bfloat16)
    t = pkg.unit_lower_inverse(nb)
    assert t.dtype == torch.bfloat16 and tuple(t.shape) == (2, 3, 24, 24)
    want = pkg.unit_lower_inverse(nb.float()).to(torch.bfloat16)
    assert torch.equal(t, want)


def test_many_chunk_sized_blocks(rng):
    """A chunk path's batch: 4096 blocks of 64 (the blocked-substitution kernel
    at scale), a sample checked against the ladder."""
    announce("unit_lower_inverse 4096 x 64")
    n = strict_lower(rng, 4096, 64, 0.15)
    t = inv(n)
    pick = rng.choice(4096, 16, replace=False)
    assert rel(t[pick], O.unit_lower_inverse(n[pick].astype(np.float64))) < 2e-5


def test_check_finite_refuses_nan():
    announce("unit_lower_inverse check_finite")
    n = torch.zeros(2, 8, 8, device=DEV)
    n[1, 5, 2] = float("nan")
    with pytest.raises(pkg.DeltaError, match="NaN or Inf"):
        pkg.unit_lower_inverse(n, check_finite=True)
