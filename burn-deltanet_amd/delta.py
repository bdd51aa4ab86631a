"""Host-side mirror of burn-deltanet's delta-rule core interface.

Same names, argument meaning and error behaviour as the reference's
src/delta (path.rs, recurrent.rs, chunk_recalculated/*.rs), over torch
tensors on the GPU; every computation is a call into libdeltanet_core.so
through the C ABI (abi.py). Where the reference panics on an assert, this
raises DeltaError with the same message.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from enum import Enum
from typing import Optional, Tuple

import torch

from . import abi
from .abi import DeltaError

Tensor = torch.Tensor


class TriSolve(Enum):
    """src/delta/tri.rs:53-64. Inside the chunk paths both variants evaluate
    the same exact inverse (the reference's Neumann series is a test baseline
    there); unit_lower_inverse honours the variant."""

    BLOCKED = "blocked"
    NEUMANN = "neumann"


@dataclass(frozen=True)
class DeltaPath:
    """src/delta/path.rs:21-99: which evaluation of the delta rule runs."""

    kind: str  # "recurrent" | "chunk" | "chunk_recalculated"
    chunk_len: Optional[int] = None
    solve: TriSolve = TriSolve.BLOCKED

    DEFAULT_CHUNK_LEN = 64

    @staticmethod
    def recurrent() -> "DeltaPath":
        return DeltaPath("recurrent")

    @staticmethod
    def chunk() -> "DeltaPath":
        return DeltaPath("chunk_recalculated")

    @staticmethod
    def default() -> "DeltaPath":
        return DeltaPath.chunk()

    @staticmethod
    def with_chunk_len(chunk_len: int) -> "DeltaPath":
        return DeltaPath("chunk_recalculated", chunk_len)

    @staticmethod
    def chunk_len_on_tape(chunk_len: int) -> "DeltaPath":
        return DeltaPath("chunk", chunk_len, TriSolve.BLOCKED)

    def resolved_chunk_len(self) -> int:
        if self.kind == "recurrent":
            return 1
        return self.DEFAULT_CHUNK_LEN if self.chunk_len is None else self.chunk_len


def beta_gates(beta: Tensor) -> Tuple[Tensor, Tensor]:
    """path.rs:147-150: a per-head β as (erase, write), each [..., 1]."""
    gate = beta.unsqueeze(-1)
    return gate, gate


@dataclass
class DeltaInput:
    """path.rs:120-141. q/k arrive L2-normalised and unscaled; gates squashed."""

    q_bshk: Tensor
    k_bshk: Tensor
    v_bshv: Tensor
    erase_bshK: Tensor
    write_bshV: Tensor
    g_bshK: Optional[Tensor]
    state_bhkv: Tensor
    scale: Optional[float] = None

    def dims(self):
        batch, sequence, nheads, head_k_dim = self.q_bshk.shape
        return batch, sequence, nheads, head_k_dim, self.v_bshv.shape[3]

    def resolved_scale(self) -> float:
        return 1.0 / math.sqrt(self.dims()[3]) if self.scale is None else float(self.scale)

    def has_channel_decay(self) -> bool:
        return self.g_bshK is not None and self.g_bshK.shape[3] > 1

    def sanity(self) -> None:
        """path.rs:177-208 (shape and gate-width checks)."""
        _check_shapes(self.q_bshk, self.k_bshk, self.v_bshv, self.erase_bshK, self.write_bshV,
                      self.g_bshK, self.state_bhkv)

    def run(self, path: DeltaPath = DeltaPath.default(), check_finite: bool = False):
        """path.rs:215-231. Returns (y_bshv, final_state_bhkv)."""
        self.sanity()
        if path.kind == "recurrent":
            return self.delta_recurrent(check_finite)
        chunk_len = path.resolved_chunk_len()
        if chunk_len <= 0:
            raise DeltaError(-4, "chunk_len must be at least 1")
        return self.delta_chunk_recalculated(chunk_len, check_finite)

    def delta_recurrent(self, check_finite: bool = False):
        """recurrent.rs:107-142: delta_step unrolled over the sequence — one
        dn_recurrent call (the state stays on chip across the tokens), or
        dn_step per token for head_k_dim above dn_recurrent's limit."""
        self.sanity()
        batch, sequence, nheads, head_k_dim, head_v_dim = self.dims()
        scale = self.resolved_scale()
        if head_k_dim <= abi.RECURRENT_MAX_K:
            # The same dtype and device rules as the chunk and step paths: one
            # q/k/v dtype, every tensor on the GPU, gates and state as fp32.
            dt = _qkv_dtype(self.q_bshk, self.k_bshk, self.v_bshv)
            q, k, v = _dev(self.q_bshk), _dev(self.k_bshk), _dev(self.v_bshv)
            e = _dev(self.erase_bshK, torch.float32)
            w = _dev(self.write_bshV, torch.float32)
            g = _dev(self.g_bshK, torch.float32)
            state = _dev(self.state_bhkv, torch.float32)
            y = torch.empty((batch, sequence, nheads, head_v_dim), dtype=dt, device=q.device)
            s_out = torch.empty_like(state)
            abi.run_recurrent(abi.recurrent_args(q, k, v, e, w, g, state, y, s_out, scale,
                                                 check_finite))
            return y, s_out
        state = self.state_bhkv.float().contiguous().clone()
        ys = []
        at = lambda x, t: None if x is None else x[:, t].contiguous()
        for t in range(sequence):
            y, state = delta_step(at(self.q_bshk, t), at(self.k_bshk, t), at(self.v_bshv, t),
                                  at(self.erase_bshK, t), at(self.write_bshV, t),
                                  at(self.g_bshK, t), state, scale, check_finite=check_finite,
                                  in_place=True)
            ys.append(y.unsqueeze(1))
        return torch.cat(ys, 1), state

    def delta_chunk_recalculated(self, chunk_len: int, check_finite: bool = False):
        """chunk_recalculated.rs:36-83 → DeltaChunkBackendExt (one autograd node)."""
        return DeltaChunkFunction.apply(
            self.q_bshk, self.k_bshk, self.v_bshv, self.erase_bshK, self.write_bshV,
            self.g_bshK, self.state_bhkv, chunk_len, self.resolved_scale(), check_finite)


def _expect(t: Tensor, shape, what):
    if tuple(t.shape) != tuple(shape):
        raise DeltaError(-2, f"{what}: expected shape {list(shape)}, got {list(t.shape)}")


def _gate_axis(t: Tensor, lead, full, what):
    n = len(lead)
    if t.dim() != n + 1 or tuple(t.shape[:n]) != tuple(lead):
        raise DeltaError(-2, f"{what}: expected leading dims {list(lead)}, got {list(t.shape)}")
    if t.shape[n] not in (1, full):
        raise DeltaError(-3, f"{what}: last axis must be 1 or {full}, got {t.shape[n]}")


def _check_shapes(q, k, v, erase, write, g, state, sequence_axis: bool = True):
    """path.rs:177-208's shape and gate-width checks (recurrent.rs:51-54 for a
    step, sequence_axis=False), run by every entry that hands buffers to the C
    ABI: the library sees plain pointers and sizes taken from q and v, so a
    tensor that disagrees with them would be read out of bounds."""
    nd = 4 if sequence_axis else 3
    what = "[batch, sequence, nheads, ·]" if sequence_axis else "[batch, nheads, ·]"
    for t, name in ((q, "q"), (v, "v")):
        if t.dim() != nd:
            raise DeltaError(-2, f"{name}: expected {what}, got {list(t.shape)}")
    lead, head_k_dim, head_v_dim = tuple(q.shape[:-1]), q.shape[-1], v.shape[-1]
    if sequence_axis and lead[1] <= 0:
        raise DeltaError(-1, "sequence length must be at least 1")
    batch, nheads = lead[0], lead[-1]
    _expect(k, lead + (head_k_dim,), "k")
    _expect(v, lead + (head_v_dim,), "v")
    _expect(state, (batch, nheads, head_k_dim, head_v_dim), "state")
    _gate_axis(erase, lead, head_k_dim, "erase gate")
    _gate_axis(write, lead, head_v_dim, "write gate")
    if g is not None:
        _gate_axis(g, lead, head_k_dim, "forget gate")


def _dev(t: Optional[Tensor], dtype=None) -> Optional[Tensor]:
    if t is None:
        return None
    if not t.is_cuda:
        raise DeltaError(-6, "tensors must live on the GPU (no CPU fallback)")
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _qkv_dtype(*ts):
    dt = ts[0].dtype
    if any(t.dtype != dt for t in ts):
        raise DeltaError(-7, "q, k and v must share one dtype")
    return dt


def unit_lower_inverse(n_strict: Tensor, solve: TriSolve = TriSolve.BLOCKED,
                       check_finite: bool = False) -> Tensor:
    """src/delta/tri.rs:66-114: T = (I − N)⁻¹ for a batched strictly lower
    triangular N of shape [..., size, size], computed in float32 by
    dn_unit_lower_inverse and returned in N's dtype. BLOCKED reads only N's
    strict lower triangle; NEUMANN sums I + N + … + N^{size−1} term by term over
    the whole matrix, up to size abi.TRI_NEUMANN_MAX_SIZE. As in the reference,
    the caller owes the strict lower property."""
    if n_strict.dim() < 2 or n_strict.shape[-2] != n_strict.shape[-1]:
        raise DeltaError(-2, "unit_lower_inverse expects a square trailing block")
    n = _dev(n_strict, torch.float32)
    t = torch.empty_like(n)
    code = abi.DN_TRI_NEUMANN if solve == TriSolve.NEUMANN else abi.DN_TRI_BLOCKED
    abi.run_unit_lower_inverse(abi.tri_args(n, t, code, check_finite))
    return t if n_strict.dtype == torch.float32 else t.to(n_strict.dtype)


def delta_chunk_recalculated(q_bshk, k_bshk, v_bshv, erase_bshK, write_bshV, g_bshK,
                             state_bhkv, has_gate: bool, chunk_len: int, scale: float,
                             algo: int = abi.DN_ALGO_AUTO, check_finite: bool = False,
                             y_dtype=None):
    """DeltaChunkBackendExt::delta_chunk_recalculated (chunk_recalculated.rs:110-151):
    `g_bshK` is read only when `has_gate`."""
    _check_shapes(q_bshk, k_bshk, v_bshv, erase_bshK, write_bshV,
                  g_bshK if has_gate else None, state_bhkv)
    dt = _qkv_dtype(q_bshk, k_bshk, v_bshv)
    q, k, v = _dev(q_bshk), _dev(k_bshk), _dev(v_bshv)
    e, w = _dev(erase_bshK, torch.float32), _dev(write_bshV, torch.float32)
    g = _dev(g_bshK, torch.float32) if has_gate else None
    s = _dev(state_bhkv, torch.float32)
    B, S, H, K = q.shape
    V = v.shape[3]
    y = torch.empty((B, S, H, V), dtype=y_dtype or dt, device=q.device)
    s_out = torch.empty((B, H, K, V), dtype=torch.float32, device=q.device)
    args = abi.chunk_fwd_args(q, k, v, e, w, g, s, y, s_out, chunk_len, scale, algo=algo,
                              check_finite=check_finite)
    _own_workspace(args, abi.lib().dn_chunk_fwd_workspace_bytes(args), q.device)
    abi.run_chunk_fwd(args)
    return y, s_out


def _own_workspace(args, nbytes: int, device) -> None:
    """Give the call a workspace from torch's caching allocator, so that the
    library never allocates (or synchronises the device) inside the call and
    concurrent calls on different streams never share scratch memory. The
    tensor lives as long as torch's stream-ordered allocator keeps it for the
    call's stream."""
    if nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
        args._workspace_tensor = ws  # keep it alive with the arguments


def delta_step(q_bhk, k_bhk, v_bhv, erase_bhK, write_bhV, g_bhK, state_bhkv, scale,
               check_finite: bool = False, in_place: bool = False, y_dtype=None):
    """recurrent.rs:41-99. Returns (y_bhv, next_state_bhkv). With
    `in_place=True` the state buffer itself is updated and returned."""
    _check_shapes(q_bhk, k_bhk, v_bhv, erase_bhK, write_bhV, g_bhK, state_bhkv,
                  sequence_axis=False)
    batch, nheads, head_k_dim = q_bhk.shape
    head_v_dim = v_bhv.shape[2]
    dt = _qkv_dtype(q_bhk, k_bhk, v_bhv)
    q, k, v = _dev(q_bhk), _dev(k_bhk), _dev(v_bhv)
    e, w = _dev(erase_bhK, torch.float32), _dev(write_bhV, torch.float32)
    g = _dev(g_bhK, torch.float32)
    s = _dev(state_bhkv, torch.float32)
    y = torch.empty((batch, nheads, head_v_dim), dtype=y_dtype or dt, device=q.device)
    s_out = s if in_place else torch.empty_like(s)
    abi.run_step(abi.step_args(q, k, v, e, w, g, s, y, s_out, scale, check_finite))
    return y, s_out


@dataclass
class DeltaChunkGrads:
    """combined_backward.rs:50-65."""

    d_q_bshk: Tensor
    d_k_bshk: Tensor
    d_v_bshv: Tensor
    d_erase_bshK: Tensor
    d_write_bshV: Tensor
    d_g_bshK: Optional[Tensor]
    d_state_bhkv: Tensor


def combined_backward(d_y_bshv, d_final_state_bhkv, q_bshk, k_bshk, v_bshv, erase_bshK,
                      write_bshV, g_bshK, state_bhkv, chunk_len: int, scale: float,
                      algo: int = abi.DN_ALGO_AUTO, check_finite: bool = False):
    """combined_backward.rs:72-189: recompute the chunk forward, then its
    closed-form gradient. Returns DeltaChunkGrads."""
    _check_shapes(q_bshk, k_bshk, v_bshv, erase_bshK, write_bshV, g_bshK, state_bhkv)
    _expect(d_y_bshv, tuple(q_bshk.shape[:3]) + (v_bshv.shape[3],), "d_y")
    if d_final_state_bhkv is not None:
        _expect(d_final_state_bhkv, tuple(state_bhkv.shape), "d_final_state")
    _qkv_dtype(q_bshk, k_bshk, v_bshv)
    q, k, v = _dev(q_bshk), _dev(k_bshk), _dev(v_bshv)
    e, w = _dev(erase_bshK, torch.float32), _dev(write_bshV, torch.float32)
    g = _dev(g_bshK, torch.float32)
    s = _dev(state_bhkv, torch.float32)
    gdt = d_y_bshv.dtype if d_y_bshv.dtype in (torch.float32, torch.bfloat16) else torch.float32
    dy = _dev(d_y_bshv, gdt)
    ds = _dev(d_final_state_bhkv, torch.float32)
    grads = (torch.empty(q.shape, dtype=gdt, device=q.device),
             torch.empty(k.shape, dtype=gdt, device=q.device),
             torch.empty(v.shape, dtype=gdt, device=q.device),
             torch.empty(e.shape, dtype=torch.float32, device=q.device),
             torch.empty(w.shape, dtype=torch.float32, device=q.device),
             None if g is None else torch.empty(g.shape, dtype=torch.float32, device=q.device),
             torch.empty(s.shape, dtype=torch.float32, device=q.device))
    args = abi.chunk_bwd_args(dy, ds, q, k, v, e, w, g, s, grads, chunk_len, scale, algo=algo,
                              check_finite=check_finite)
    _own_workspace(args, abi.lib().dn_chunk_bwd_workspace_bytes(args), q.device)
    abi.run_chunk_bwd(args)
    return DeltaChunkGrads(*grads)


class DeltaChunkFunction(torch.autograd.Function):
    """The custom autodiff node of chunk_recalculated/backward.rs:31-265: keeps
    only the seven leaves and runs combined_backward on the way back."""

    @staticmethod
    def forward(ctx, q, k, v, erase, write, g, state, chunk_len, scale, check_finite):
        y, s_out = delta_chunk_recalculated(q, k, v, erase, write, g, state, g is not None,
                                            chunk_len, scale, check_finite=check_finite)
        ctx.save_for_backward(q, k, v, erase, write, g, state)
        ctx.chunk_len, ctx.scale, ctx.check_finite = chunk_len, scale, check_finite
        return y, s_out

    @staticmethod
    def backward(ctx, d_y, d_state):
        q, k, v, erase, write, g, state = ctx.saved_tensors
        if d_y is None:
            d_y = torch.zeros(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device)
        gr = combined_backward(d_y, d_state, q, k, v, erase, write, g, state, ctx.chunk_len,
                               ctx.scale, check_finite=ctx.check_finite)
        cast = lambda t, ref: None if t is None else t.to(ref.dtype)
        return (cast(gr.d_q_bshk, q), cast(gr.d_k_bshk, k), cast(gr.d_v_bshv, v),
                cast(gr.d_erase_bshK, erase), cast(gr.d_write_bshV, write),
                None if g is None else cast(gr.d_g_bshK, g), cast(gr.d_state_bhkv, state),
                None, None, None)
