"""ctypes view of include/deltanet_core.h and thin launchers over torch tensors.

The structs below mirror the C header field for field. Torch supplies device
memory and the current HIP stream; every computation runs in
libdeltanet_core.so. There is no fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libdeltanet_core.so"

DN_F32, DN_BF16 = 0, 1
DN_ALGO_AUTO, DN_ALGO_GENERIC, DN_ALGO_MFMA, DN_ALGO_MFMA_FUSED = 0, 1, 2, 3
RECURRENT_MAX_K = 512  # dn_recurrent's head_k_dim limit (deltanet_core.h)
DN_ACT_IDENTITY, DN_ACT_SILU, DN_ACT_RELU, DN_ACT_ELU_PLUS_ONE = 0, 1, 2, 3
DN_QKNORM_NONE, DN_QKNORM_L2, DN_QKNORM_SUM = 0, 1, 2
DN_WRITE_FIXED, DN_WRITE_SCALAR, DN_WRITE_CHANNEL = 0, 1, 2
FRONTEND_MAX_HEAD_DIM, FRONTEND_MAX_KERNEL = 256, 8
OUT_NORM_MAX_HEAD_DIM = 1024
DN_TRI_BLOCKED, DN_TRI_NEUMANN = 0, 1
BLOCK_STEP_MAX_HEAD_DIM = 256  # DN_BLOCK_STEP_MAX_HEAD_DIM (deltanet_core.h)
TRI_NEUMANN_MAX_SIZE = 140  # DN_TRI_NEUMANN_MAX_SIZE (deltanet_core.h)

STATUS = {
    0: "DN_OK",
    -1: "DN_ERR_SEQUENCE",
    -2: "DN_ERR_SHAPE",
    -3: "DN_ERR_GATE_WIDTH",
    -4: "DN_ERR_CHUNK_LEN",
    -5: "DN_ERR_NONFINITE",
    -6: "DN_ERR_NULL",
    -7: "DN_ERR_DTYPE",
    -8: "DN_ERR_WORKSPACE",
    -9: "DN_ERR_UNSUPPORTED",
    -10: "DN_ERR_HIP",
}

EXPORTS = [
    "dn_chunk_fwd", "dn_chunk_bwd", "dn_step", "dn_recurrent", "dn_frontend", "dn_out_norm",
    "dn_chunk_fwd_workspace_bytes",
    "dn_chunk_bwd_workspace_bytes", "dn_chunk_fwd_algo", "dn_chunk_bwd_algo",
    "dn_last_error", "dn_version", "dn_profile_enable", "dn_profile_read",
    "dn_chunk_fwd_noalloc", "dn_unit_lower_inverse", "dn_block_step",
    "dn_chunk_fwd_out_norm", "dn_chunk_fwd_out_norm_workspace_bytes", "dn_wait_give_ups",
    "dn_frontend_chunk_fwd", "dn_frontend_chunk_fwd_workspace_bytes",
]
NOALLOC_SCRATCH_BYTES = 64 << 20  # DN_NOALLOC_SCRATCH_BYTES (deltanet_core.h)

_i64, _i32, _f64, _vp, _sz = (ctypes.c_int64, ctypes.c_int32, ctypes.c_double,
                              ctypes.c_void_p, ctypes.c_size_t)


class ChunkFwdArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("sequence", _i64), ("nheads", _i64), ("head_k_dim", _i64),
        ("head_v_dim", _i64), ("erase_width", _i64), ("write_width", _i64),
        ("decay_width", _i64), ("has_gate", _i32), ("chunk_len", _i32), ("scale", _f64),
        ("qkv_dtype", _i32), ("y_dtype", _i32), ("algo", _i32), ("check_finite", _i32),
        ("q", _vp), ("k", _vp), ("v", _vp), ("erase", _vp), ("write", _vp), ("g", _vp),
        ("state_in", _vp), ("y", _vp), ("state_out", _vp), ("workspace", _vp),
        ("workspace_bytes", _sz),
    ]


class ChunkBwdArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("sequence", _i64), ("nheads", _i64), ("head_k_dim", _i64),
        ("head_v_dim", _i64), ("erase_width", _i64), ("write_width", _i64),
        ("decay_width", _i64), ("has_gate", _i32), ("chunk_len", _i32), ("scale", _f64),
        ("qkv_dtype", _i32), ("grad_dtype", _i32), ("algo", _i32), ("check_finite", _i32),
        ("d_y", _vp), ("d_state_final", _vp), ("q", _vp), ("k", _vp), ("v", _vp),
        ("erase", _vp), ("write", _vp), ("g", _vp), ("state_in", _vp), ("d_q", _vp),
        ("d_k", _vp), ("d_v", _vp), ("d_erase", _vp), ("d_write", _vp), ("d_g", _vp),
        ("d_state", _vp), ("workspace", _vp), ("workspace_bytes", _sz),
    ]


class StepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("nheads", _i64), ("head_k_dim", _i64), ("head_v_dim", _i64),
        ("erase_width", _i64), ("write_width", _i64), ("decay_width", _i64),
        ("has_gate", _i32), ("scale", _f64), ("qkv_dtype", _i32), ("y_dtype", _i32),
        ("check_finite", _i32),
        ("q", _vp), ("k", _vp), ("v", _vp), ("erase", _vp), ("write", _vp), ("g", _vp),
        ("state_in", _vp), ("y", _vp), ("state_out", _vp),
    ]


class RecurrentArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("sequence", _i64), ("nheads", _i64), ("head_k_dim", _i64),
        ("head_v_dim", _i64), ("erase_width", _i64), ("write_width", _i64),
        ("decay_width", _i64), ("has_gate", _i32), ("scale", _f64), ("qkv_dtype", _i32),
        ("y_dtype", _i32), ("check_finite", _i32),
        ("q", _vp), ("k", _vp), ("v", _vp), ("erase", _vp), ("write", _vp), ("g", _vp),
        ("state_in", _vp), ("y", _vp), ("state_out", _vp),
    ]


class FrontendArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("sequence", _i64), ("nheads", _i64), ("head_k_dim", _i64),
        ("head_v_dim", _i64), ("n_householder", _i64), ("conv_kernel", _i64),
        ("proj_stride", _i64), ("conv_activation", _i32), ("qk_activation", _i32),
        ("qk_norm", _i32), ("write_gate", _i32), ("allow_neg_eigval", _i32),
        ("in_dtype", _i32), ("out_dtype", _i32),
        ("projected", _vp), ("conv_weight", _vp), ("conv_bias", _vp), ("window_in", _vp),
        ("window_out", _vp), ("q", _vp), ("k", _vp), ("v", _vp), ("erase", _vp),
        ("write", _vp),
    ]


class OutNormArgs(ctypes.Structure):
    _fields_ = [
        ("tokens", _i64), ("nheads", _i64), ("head_v_dim", _i64), ("gate_stride", _i64),
        ("eps", _f64), ("x_dtype", _i32), ("gate_dtype", _i32), ("out_dtype", _i32),
        ("x", _vp), ("gate", _vp), ("weight", _vp), ("out", _vp),
    ]


class FrontendChunkFwdArgs(ctypes.Structure):
    _fields_ = [("fe", FrontendArgs), ("fwd", ChunkFwdArgs)]


class ChunkFwdOutNormArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", ChunkFwdArgs), ("gate", _vp), ("gate_stride", _i64), ("gate_dtype", _i32),
        ("weight", _vp), ("eps", _f64), ("in_scan", _i32),
    ]


class BlockStepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("nheads", _i64), ("head_k_dim", _i64), ("head_v_dim", _i64),
        ("conv_kernel", _i64), ("proj_stride", _i64),
        ("conv_activation", _i32), ("qk_activation", _i32), ("qk_norm", _i32),
        ("write_gate", _i32), ("allow_neg_eigval", _i32), ("in_dtype", _i32),
        ("out_dtype", _i32), ("has_gate", _i32), ("decay_width", _i64), ("scale", _f64),
        ("eps", _f64), ("norm_gated", _i32), ("check_finite", _i32),
        ("projected", _vp), ("conv_weight", _vp), ("conv_bias", _vp), ("window_in", _vp),
        ("window_out", _vp), ("g", _vp), ("state_in", _vp), ("state_out", _vp),
        ("norm_weight", _vp), ("out", _vp), ("y", _vp),
    ]


class TriArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("size", _i64), ("solve", _i32), ("check_finite", _i32),
        ("n_strict", _vp), ("t", _vp),
    ]


_LIB = None


def lib() -> ctypes.CDLL:
    """Load libdeltanet_core.so (built by __graft_entry__.build())."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; "
                "g.build()'` — there is no CPU fallback for the delta-rule core")
        L = ctypes.CDLL(str(LIB_PATH))
        L.dn_chunk_fwd.argtypes = [ctypes.POINTER(ChunkFwdArgs), _vp]
        L.dn_chunk_fwd.restype = ctypes.c_int
        L.dn_chunk_fwd_noalloc.argtypes = [ctypes.POINTER(ChunkFwdArgs), _vp]
        L.dn_chunk_fwd_noalloc.restype = ctypes.c_int
        L.dn_chunk_bwd.argtypes = [ctypes.POINTER(ChunkBwdArgs), _vp]
        L.dn_chunk_bwd.restype = ctypes.c_int
        L.dn_step.argtypes = [ctypes.POINTER(StepArgs), _vp]
        L.dn_step.restype = ctypes.c_int
        L.dn_recurrent.argtypes = [ctypes.POINTER(RecurrentArgs), _vp]
        L.dn_recurrent.restype = ctypes.c_int
        L.dn_frontend.argtypes = [ctypes.POINTER(FrontendArgs), _vp]
        L.dn_frontend.restype = ctypes.c_int
        L.dn_out_norm.argtypes = [ctypes.POINTER(OutNormArgs), _vp]
        L.dn_out_norm.restype = ctypes.c_int
        L.dn_chunk_fwd_out_norm.argtypes = [ctypes.POINTER(ChunkFwdOutNormArgs), _vp]
        L.dn_chunk_fwd_out_norm.restype = ctypes.c_int
        L.dn_chunk_fwd_out_norm_workspace_bytes.argtypes = [ctypes.POINTER(ChunkFwdOutNormArgs)]
        L.dn_chunk_fwd_out_norm_workspace_bytes.restype = _sz
        L.dn_frontend_chunk_fwd.argtypes = [ctypes.POINTER(FrontendChunkFwdArgs), _vp]
        L.dn_frontend_chunk_fwd.restype = ctypes.c_int
        L.dn_frontend_chunk_fwd_workspace_bytes.argtypes = [ctypes.POINTER(FrontendChunkFwdArgs)]
        L.dn_frontend_chunk_fwd_workspace_bytes.restype = _sz
        L.dn_wait_give_ups.argtypes = []
        L.dn_wait_give_ups.restype = ctypes.c_int64
        L.dn_block_step.argtypes = [ctypes.POINTER(BlockStepArgs), _vp]
        L.dn_block_step.restype = ctypes.c_int
        L.dn_unit_lower_inverse.argtypes = [ctypes.POINTER(TriArgs), _vp]
        L.dn_unit_lower_inverse.restype = ctypes.c_int
        L.dn_chunk_fwd_workspace_bytes.argtypes = [ctypes.POINTER(ChunkFwdArgs)]
        L.dn_chunk_fwd_workspace_bytes.restype = _sz
        L.dn_chunk_bwd_workspace_bytes.argtypes = [ctypes.POINTER(ChunkBwdArgs)]
        L.dn_chunk_bwd_workspace_bytes.restype = _sz
        L.dn_chunk_fwd_algo.argtypes = [ctypes.POINTER(ChunkFwdArgs)]
        L.dn_chunk_fwd_algo.restype = ctypes.c_int
        L.dn_chunk_bwd_algo.argtypes = [ctypes.POINTER(ChunkBwdArgs)]
        L.dn_chunk_bwd_algo.restype = ctypes.c_int
        L.dn_profile_enable.argtypes = [ctypes.c_int]
        L.dn_profile_enable.restype = ctypes.c_int
        L.dn_profile_read.argtypes = [ctypes.c_int, ctypes.c_char_p, _sz,
                                      ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_int64)]
        L.dn_profile_read.restype = ctypes.c_int
        L.dn_last_error.restype = ctypes.c_char_p
        L.dn_version.restype = ctypes.c_char_p
        _LIB = L
    return _LIB


class DeltaError(ValueError):
    """A failed check of the core; carries the dn_status code."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code


def check(rc: int) -> None:
    if rc != 0:
        raise DeltaError(rc, lib().dn_last_error().decode())


def dtype_tag(t: torch.dtype) -> int:
    if t == torch.float32:
        return DN_F32
    if t == torch.bfloat16:
        return DN_BF16
    raise DeltaError(-7, f"unsupported dtype {t}; use float32 or bfloat16")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def nan_scale(scale):
    return float("nan") if scale is None else float(scale)


def chunk_fwd_args(q, k, v, erase, write, g, state, y, state_out, chunk_len, scale,
                   algo=DN_ALGO_AUTO, check_finite=False, workspace=None):
    B, S, H, K = q.shape
    V = v.shape[3]
    a = ChunkFwdArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = B, S, H, K, V
    a.erase_width, a.write_width = erase.shape[3], write.shape[3]
    a.decay_width = 0 if g is None else g.shape[3]
    a.has_gate = 0 if g is None else 1
    a.chunk_len = int(chunk_len)
    a.scale = nan_scale(scale)
    a.qkv_dtype = dtype_tag(q.dtype)
    a.y_dtype = dtype_tag(y.dtype)
    a.algo = int(algo)
    a.check_finite = int(bool(check_finite))
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.erase, a.write = erase.data_ptr(), write.data_ptr()
    a.g = None if g is None else g.data_ptr()
    a.state_in, a.y, a.state_out = state.data_ptr(), y.data_ptr(), state_out.data_ptr()
    if workspace is not None:
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    return a


def run_chunk_fwd(args: ChunkFwdArgs) -> None:
    check(lib().dn_chunk_fwd(ctypes.byref(args), stream_handle()))


def run_chunk_fwd_noalloc(args: ChunkFwdArgs) -> None:
    """dn_chunk_fwd_noalloc: the forward on the library's fixed scratch array
    (no allocation in the call; `workspace` is ignored)."""
    check(lib().dn_chunk_fwd_noalloc(ctypes.byref(args), stream_handle()))


def step_args(q, k, v, erase, write, g, state, y, state_out, scale, check_finite=False):
    B, H, K = q.shape
    V = v.shape[2]
    a = StepArgs()
    a.batch, a.nheads, a.head_k_dim, a.head_v_dim = B, H, K, V
    a.erase_width, a.write_width = erase.shape[2], write.shape[2]
    a.decay_width = 0 if g is None else g.shape[2]
    a.has_gate = 0 if g is None else 1
    a.scale = nan_scale(scale)
    a.qkv_dtype = dtype_tag(q.dtype)
    a.y_dtype = dtype_tag(y.dtype)
    a.check_finite = int(bool(check_finite))
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.erase, a.write = erase.data_ptr(), write.data_ptr()
    a.g = None if g is None else g.data_ptr()
    a.state_in, a.y, a.state_out = state.data_ptr(), y.data_ptr(), state_out.data_ptr()
    return a


def run_step(args: StepArgs) -> None:
    check(lib().dn_step(ctypes.byref(args), stream_handle()))


def recurrent_args(q, k, v, erase, write, g, state, y, state_out, scale, check_finite=False):
    """dn_recurrent over [batch, sequence, nheads, ·] inputs."""
    B, S, H, K = q.shape
    V = v.shape[3]
    a = RecurrentArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = B, S, H, K, V
    a.erase_width, a.write_width = erase.shape[3], write.shape[3]
    a.decay_width = 0 if g is None else g.shape[3]
    a.has_gate = 0 if g is None else 1
    a.scale = nan_scale(scale)
    a.qkv_dtype = dtype_tag(q.dtype)
    a.y_dtype = dtype_tag(y.dtype)
    a.check_finite = int(bool(check_finite))
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.erase, a.write = erase.data_ptr(), write.data_ptr()
    a.g = None if g is None else g.data_ptr()
    a.state_in, a.y, a.state_out = state.data_ptr(), y.data_ptr(), state_out.data_ptr()
    return a


def run_recurrent(args: RecurrentArgs) -> None:
    check(lib().dn_recurrent(ctypes.byref(args), stream_handle()))


def _ptr(t):
    """A tensor's address for the C ABI, whose kernels read it on the GPU: a
    host tensor is refused here rather than handed over as a host pointer."""
    if t is None:
        return None
    if not t.is_cuda:
        raise DeltaError(-6, "tensors must live on the GPU (no CPU fallback)")
    return t.data_ptr()


def frontend_args(projected, conv_weight, conv_bias, window_in, window_out, q, k, v, erase,
                  write, *, nheads, head_k_dim, head_v_dim, n_householder, conv_activation,
                  qk_activation, qk_norm, write_gate, allow_neg_eigval):
    """dn_frontend over `projected` [batch, sequence, proj_stride] (contiguous
    rows; the stride is its last axis)."""
    B, S, W = projected.shape
    a = FrontendArgs()
    a.batch, a.sequence, a.nheads = B, S, nheads
    a.head_k_dim, a.head_v_dim, a.n_householder = head_k_dim, head_v_dim, n_householder
    a.conv_kernel = 0 if conv_weight is None else conv_weight.shape[-1]
    a.proj_stride = W
    a.conv_activation, a.qk_activation = int(conv_activation), int(qk_activation)
    a.qk_norm, a.write_gate = int(qk_norm), int(write_gate)
    a.allow_neg_eigval = int(bool(allow_neg_eigval))
    a.in_dtype, a.out_dtype = dtype_tag(projected.dtype), dtype_tag(q.dtype)
    a.projected, a.conv_weight, a.conv_bias = (_ptr(projected), _ptr(conv_weight),
                                               _ptr(conv_bias))
    a.window_in, a.window_out = _ptr(window_in), _ptr(window_out)
    a.q, a.k, a.v, a.erase, a.write = (_ptr(q), _ptr(k), _ptr(v), _ptr(erase), _ptr(write))
    return a


def run_frontend(args: FrontendArgs) -> None:
    check(lib().dn_frontend(ctypes.byref(args), stream_handle()))


def out_norm_args(x, gate, weight, out, eps):
    """dn_out_norm over x [.., nheads, head_v_dim] (contiguous). `gate` has
    the same shape and may be a view whose heads are contiguous within a
    token and whose tokens are evenly strided (a column range of the
    projection)."""
    H, D = x.shape[-2], x.shape[-1]
    a = OutNormArgs()
    a.tokens, a.nheads, a.head_v_dim = x.numel() // (H * D), H, D
    if gate is not None:
        if tuple(gate.shape) != tuple(x.shape):
            raise DeltaError(-2, f"gate: expected shape {list(x.shape)}, got {list(gate.shape)}")
        if gate.stride(-1) != 1 or gate.stride(-2) != D:
            raise DeltaError(-2, "gate: heads must be contiguous within a token")
        lead, strides = gate.shape[:-2], gate.stride()[:-2]
        token_stride = strides[-1] if lead else H * D
        want = token_stride  # the leading axes must flatten to one token stride
        for n, st in zip(reversed(lead), reversed(strides)):
            if n > 1 and st != want:
                raise DeltaError(-2, "gate: tokens must be evenly strided")
            want *= n
        a.gate_stride = token_stride
        a.gate_dtype = dtype_tag(gate.dtype)
    a.eps = float(eps)
    a.x_dtype, a.out_dtype = dtype_tag(x.dtype), dtype_tag(out.dtype)
    a.x, a.gate, a.weight, a.out = _ptr(x), _ptr(gate), _ptr(weight), _ptr(out)
    return a


def run_out_norm(args: OutNormArgs) -> None:
    check(lib().dn_out_norm(ctypes.byref(args), stream_handle()))


def chunk_fwd_out_norm_args(fwd: ChunkFwdArgs, gate, weight, eps,
                            in_scan=False) -> ChunkFwdOutNormArgs:
    """dn_chunk_fwd_out_norm's arguments: `fwd` (whose y receives the norm's
    output) with the output norm's gate ([batch, sequence, nheads, head_v_dim]
    or a column view of the projection with evenly strided tokens; None for
    the plain norm), weight γ [head_v_dim] and eps; in_scan: the norm in the
    MFMA scan's y write rather than a pass of its own."""
    a = ChunkFwdOutNormArgs()
    a.fwd = fwd
    a.in_scan = int(bool(in_scan))
    H, D = fwd.nheads, fwd.head_v_dim
    if gate is not None:
        want = (fwd.batch, fwd.sequence, H, D)
        if tuple(gate.shape) != want:
            raise DeltaError(-2, f"gate: expected shape {list(want)}, got {list(gate.shape)}")
        if gate.stride(3) != 1 or gate.stride(2) != D or (
                fwd.sequence > 1 and fwd.batch > 1 and gate.stride(0) != gate.stride(1) * fwd.sequence):
            raise DeltaError(-2, "gate: heads contiguous within a token, tokens evenly strided")
        a.gate_stride = gate.stride(1) if fwd.sequence > 1 else gate.stride(0)
        a.gate_dtype = dtype_tag(gate.dtype)
    a.gate, a.weight, a.eps = _ptr(gate), _ptr(weight), float(eps)
    return a


def run_chunk_fwd_out_norm(args: ChunkFwdOutNormArgs) -> None:
    check(lib().dn_chunk_fwd_out_norm(ctypes.byref(args), stream_handle()))


def frontend_chunk_fwd_args(fe: FrontendArgs, fwd: ChunkFwdArgs) -> FrontendChunkFwdArgs:
    """dn_frontend_chunk_fwd's arguments: dn_frontend's `fe`, then the chunk
    forward `fwd` over fe's outputs (fwd.q, k, v, erase, write must be fe's)."""
    a = FrontendChunkFwdArgs()
    a.fe, a.fwd = fe, fwd
    return a


def run_frontend_chunk_fwd(args: FrontendChunkFwdArgs) -> None:
    check(lib().dn_frontend_chunk_fwd(ctypes.byref(args), stream_handle()))


def wait_give_ups() -> int:
    """dn_wait_give_ups: bounded cross-workgroup waits that gave up on this
    device so far (synchronises)."""
    return int(lib().dn_wait_give_ups())


def tri_args(n_strict, t, solve=DN_TRI_BLOCKED, check_finite=False) -> TriArgs:
    """dn_tri_args over [..., size, size] float32 tensors (any leading axes)."""
    size = n_strict.shape[-1]
    a = TriArgs()
    a.batch = n_strict.numel() // (size * size) if size else 0
    a.size = size
    a.solve = int(solve)
    a.check_finite = 1 if check_finite else 0
    a.n_strict, a.t = _ptr(n_strict), _ptr(t)
    return a


def run_block_step(args: BlockStepArgs) -> None:
    check(lib().dn_block_step(ctypes.byref(args), stream_handle()))


def run_unit_lower_inverse(args: TriArgs) -> None:
    check(lib().dn_unit_lower_inverse(ctypes.byref(args), stream_handle()))


def chunk_bwd_args(dy, dstate, q, k, v, erase, write, g, state, grads, chunk_len, scale,
                   algo=DN_ALGO_AUTO, check_finite=False, workspace=None):
    dq, dk, dv, de, dw, dg, ds = grads
    B, S, H, K = q.shape
    V = v.shape[3]
    a = ChunkBwdArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = B, S, H, K, V
    a.erase_width, a.write_width = erase.shape[3], write.shape[3]
    a.decay_width = 0 if g is None else g.shape[3]
    a.has_gate = 0 if g is None else 1
    a.chunk_len = int(chunk_len)
    a.scale = nan_scale(scale)
    a.qkv_dtype = dtype_tag(q.dtype)
    a.grad_dtype = dtype_tag(dy.dtype)
    a.algo = int(algo)
    a.check_finite = int(bool(check_finite))
    a.d_y = dy.data_ptr()
    a.d_state_final = None if dstate is None else dstate.data_ptr()
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.erase, a.write = erase.data_ptr(), write.data_ptr()
    a.g = None if g is None else g.data_ptr()
    a.state_in = state.data_ptr()
    a.d_q, a.d_k, a.d_v = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.d_erase, a.d_write = de.data_ptr(), dw.data_ptr()
    a.d_g = None if dg is None else dg.data_ptr()
    a.d_state = ds.data_ptr()
    if workspace is not None:
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    return a


def run_chunk_bwd(args: ChunkBwdArgs) -> None:
    check(lib().dn_chunk_bwd(ctypes.byref(args), stream_handle()))


def profile_enable(on: bool = True) -> None:
    """Start (clearing earlier records) or stop per-kernel HIP-event timing."""
    lib().dn_profile_enable(1 if on else 0)


def profile_read() -> dict:
    """{kernel name: (total_ms, launches)} for everything timed since enable."""
    L = lib()
    out = {}
    count = L.dn_profile_read(-1, None, 0, None, None)
    for i in range(count):
        name = ctypes.create_string_buffer(128)
        ms = ctypes.c_double()
        n = ctypes.c_int64()
        L.dn_profile_read(i, name, 128, ctypes.byref(ms), ctypes.byref(n))
        out[name.value.decode()] = (ms.value, n.value)
    return out
