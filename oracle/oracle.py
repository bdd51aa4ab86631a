"""ctypes front of the CPU oracle (oracle.cpp) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker / the timed CPU baseline. Every function
takes numpy arrays in the reference's layouts (src/delta/path.rs:120-141):

    q, k   [B, S, H, K]        v      [B, S, H, V]
    erase  [B, S, H, 1|K]      write  [B, S, H, 1|V]
    g      [B, S, H, 1|K] or None      state  [B, H, K, V]

and a dtype of float32 or float64 (all arrays are converted to that dtype).
`scale=None` resolves to 1/sqrt(K) (src/delta/path.rs:161-165).
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None


def build() -> None:
    """Compile liboracle.so in place (gcc/g++ only)."""
    import subprocess

    subprocess.run(["make", "-C", str(_HERE), "-B", "liboracle.so"], check=True,
                   stdout=subprocess.DEVNULL)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            build()
        _LIB = ctypes.CDLL(str(path))
        _LIB.or_max_threads.restype = ctypes.c_int
    return _LIB


_P = ctypes.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def _prep(dtype, *arrays):
    out = []
    for a in arrays:
        out.append(None if a is None else np.ascontiguousarray(a, dtype=dtype))
    return out


def _suffix(dtype):
    dtype = np.dtype(dtype)
    if dtype == np.float32:
        return "f32", ctypes.c_float
    if dtype == np.float64:
        return "f64", ctypes.c_double
    raise TypeError(f"oracle supports float32/float64, got {dtype}")


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def max_threads() -> int:
    return int(lib().or_max_threads())


def _dims(q, v, erase, write, g):
    B, S, H, K = q.shape
    V = v.shape[3]
    return B, S, H, K, V, erase.shape[3], write.shape[3], (0 if g is None else g.shape[3])


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (code {rc})")


def recurrent(q, k, v, erase, write, g, state, scale=None, dtype=np.float64):
    """DeltaInput::delta_recurrent (src/delta/recurrent.rs:107-142)."""
    q, k, v, erase, write, g, state = _prep(dtype, q, k, v, erase, write, g, state)
    B, S, H, K, V, ew, ww, dw = _dims(q, v, erase, write, g)
    scale = 1.0 / math.sqrt(K) if scale is None else scale
    suf, cty = _suffix(dtype)
    y = np.zeros((B, S, H, V), dtype)
    s_out = np.zeros((B, H, K, V), dtype)
    fn = getattr(lib(), f"or_recurrent_{suf}")
    rc = fn(*(ctypes.c_long(x) for x in (B, S, H, K, V, ew, ww, dw)),
            *(_ptr(a) for a in (q, k, v, erase, write, g, state)), cty(scale),
            _ptr(y), _ptr(s_out))
    _check(rc, "recurrent")
    return y, s_out


def delta_step(q, k, v, erase, write, g, state, scale=None, dtype=np.float64):
    """delta_step (src/delta/recurrent.rs:41-99) on [B, H, ·] inputs."""
    add_s = lambda a: None if a is None else np.asarray(a)[:, None]
    y, s = recurrent(add_s(q), add_s(k), add_s(v), add_s(erase), add_s(write), add_s(g),
                     state, scale=scale, dtype=dtype)
    return y[:, 0], s


def chunk_fwd(q, k, v, erase, write, g, state, chunk_len=64, scale=None, dtype=np.float64):
    """DeltaChunkBackendExt::delta_chunk_recalculated's default body
    (src/delta/chunk_recalculated/chunk_recalculated.rs:115-177)."""
    q, k, v, erase, write, g, state = _prep(dtype, q, k, v, erase, write, g, state)
    B, S, H, K, V, ew, ww, dw = _dims(q, v, erase, write, g)
    scale = 1.0 / math.sqrt(K) if scale is None else scale
    suf, cty = _suffix(dtype)
    y = np.zeros((B, S, H, V), dtype)
    s_out = np.zeros((B, H, K, V), dtype)
    fn = getattr(lib(), f"or_chunk_fwd_{suf}")
    rc = fn(*(ctypes.c_long(x) for x in (B, S, H, K, V, ew, ww, dw, chunk_len)),
            *(_ptr(a) for a in (q, k, v, erase, write, g, state)), cty(scale),
            _ptr(y), _ptr(s_out))
    _check(rc, "chunk_fwd")
    return y, s_out


def chunk_bwd(dy, dstate, q, k, v, erase, write, g, state, chunk_len=64, scale=None,
              dtype=np.float64):
    """combined_backward (src/delta/chunk_recalculated/combined_backward.rs:72-189).

    Returns (dq, dk, dv, d_erase, d_write, d_g or None, d_state)."""
    dy, dstate, q, k, v, erase, write, g, state = _prep(
        dtype, dy, dstate, q, k, v, erase, write, g, state)
    B, S, H, K, V, ew, ww, dw = _dims(q, v, erase, write, g)
    scale = 1.0 / math.sqrt(K) if scale is None else scale
    suf, cty = _suffix(dtype)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    de = np.zeros_like(erase)
    dwr = np.zeros_like(write)
    dg = None if g is None else np.zeros_like(g)
    ds = np.zeros_like(state)
    fn = getattr(lib(), f"or_chunk_bwd_{suf}")
    rc = fn(*(ctypes.c_long(x) for x in (B, S, H, K, V, ew, ww, dw, chunk_len)),
            _ptr(dy), _ptr(dstate), *(_ptr(a) for a in (q, k, v, erase, write, g, state)),
            cty(scale), *(_ptr(a) for a in (dq, dk, dv, de, dwr, dg, ds)))
    _check(rc, "chunk_bwd")
    return dq, dk, dv, de, dwr, dg, ds


def _tri(fn, n, dtype):
    (n,) = _prep(dtype, n)
    squeeze = n.ndim == 2
    if squeeze:
        n = n[None]
    flat, size, _ = n.shape
    t = np.zeros_like(n)
    suf, _ = _suffix(dtype)
    rc = getattr(lib(), f"{fn}_{suf}")(ctypes.c_long(flat), ctypes.c_long(size), _ptr(n), _ptr(t))
    _check(rc, fn)
    return t[0] if squeeze else t


def unit_lower_inverse(n, dtype=np.float64):
    """The Blocked ladder (src/delta/tri/prim.rs:28-51) on [flat, size, size]."""
    return _tri("or_unit_lower_inverse", n, dtype)


def neumann_inverse(n, dtype=np.float64):
    """TriSolve::Neumann (src/delta/tri.rs:99-107): I + N + … + N^{size−1},
    term by term over the whole matrix, on [flat, size, size]."""
    return _tri("or_neumann_inverse", n, dtype)


def l2_normalize(x, eps=1e-6):
    """src/common/norm.rs:83-90: x / sqrt(sum(x^2) + 1e-6) over the last axis."""
    x = np.asarray(x)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)
