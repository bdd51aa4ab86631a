"""Host-side mirror of the reference's projection front-end
(src/common/qkv.rs, conv.rs, norm.rs) over dn_frontend, and of its output
norm (OutNorm, norm.rs:106-144) over dn_out_norm.

`QkvProjection` keeps the reference's fields and methods (`key_dim`,
`value_dim`, `conv_dim`, `write_gate_width`, `d_in_proj`, `segments`,
`zero_conv_window`, `forward`, `step`). The in-projection is a plain library
GEMM (torch.matmul, i.e. hipBLASLt); everything after it, up to the delta
rule's inputs, is one dn_frontend call. Grouped values (n_value_heads ≠
nheads) and QkNorm.SUM are not offered: both depend on burn_stack code the
reference does not vendor.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum
from typing import List, Optional, Tuple

import torch
from torch import Tensor

from . import abi
from .abi import DeltaError


class QkActivation(IntEnum):
    """norm.rs:22-34."""
    IDENTITY = abi.DN_ACT_IDENTITY
    SILU = abi.DN_ACT_SILU
    RELU = abi.DN_ACT_RELU
    ELU_PLUS_ONE = abi.DN_ACT_ELU_PLUS_ONE


class ConvActivation(IntEnum):
    """conv.rs:29-35."""
    SILU = abi.DN_ACT_SILU
    IDENTITY = abi.DN_ACT_IDENTITY


class QkNorm(IntEnum):
    """norm.rs:56-65 (SUM is declared for completeness and refused)."""
    L2 = abi.DN_QKNORM_L2
    SUM = abi.DN_QKNORM_SUM
    NONE = abi.DN_QKNORM_NONE


class WriteGate(IntEnum):
    """qkv.rs:45-54."""
    FIXED = abi.DN_WRITE_FIXED
    SCALAR = abi.DN_WRITE_SCALAR
    CHANNEL = abi.DN_WRITE_CHANNEL


@dataclass
class ShortConv:
    """conv.rs:49-83: the depthwise weight [conv_dim, conv_kernel] (Conv1d's
    [conv_dim, 1, kernel] without its unit axis), an optional bias, and the
    fused activation."""

    weight: Tensor
    bias: Optional[Tensor] = None
    activation: ConvActivation = ConvActivation.SILU

    def conv_dim(self) -> int:
        return self.weight.shape[0]

    def conv_kernel(self) -> int:
        return self.weight.shape[-1]

    def zero_window(self, batch: int, device, dtype=torch.float32) -> Tensor:
        return torch.zeros((batch, self.conv_dim(), self.conv_kernel()), dtype=dtype,
                           device=device)


@dataclass
class Qkv:
    """qkv.rs:76-97 (k, v and the gates with the micro-steps folded into the
    sequence)."""

    q_bshk: Tensor
    k_bShk: Tensor
    v_bShv: Tensor
    erase_bShK: Tensor
    write_bShV: Tensor
    gate_bshv: Optional[Tensor]
    extra_bsx: Optional[Tensor]


@dataclass
class QkvStep:
    """qkv.rs:99-116."""

    q_bhk: Tensor
    k_buhk: Tensor
    v_buhv: Tensor
    erase_buhK: Tensor
    write_buhV: Tensor
    gate_bhv: Optional[Tensor]
    extra_bx: Optional[Tensor]


@dataclass
class QkvProjection:
    """qkv.rs:118-155, n_value_heads = nheads. `in_proj` is the weight
    [d_model, d_in_proj] (applied as x @ in_proj) or None when the caller
    supplies the projection itself (`forward_projected` / `step_projected`)."""

    nheads: int
    head_k_dim: int
    head_v_dim: int
    n_householder: int = 1
    conv: Optional[ShortConv] = None
    qk_activation: QkActivation = QkActivation.SILU
    qk_norm: QkNorm = QkNorm.L2
    write_gate: WriteGate = WriteGate.SCALAR
    has_gate: bool = False
    allow_neg_eigval: bool = False
    extra_channels: int = 0
    in_proj: Optional[Tensor] = None
    in_proj_bias: Optional[Tensor] = None  # QkvProjectionConfig::has_proj_bias

    def key_dim(self) -> int:
        return self.nheads * self.head_k_dim

    def value_dim(self) -> int:
        return self.nheads * self.head_v_dim

    def conv_dim(self) -> int:
        """qkv.rs:180-182."""
        return self.key_dim() + self.n_householder * (self.key_dim() + self.value_dim())

    def write_gate_width(self) -> int:
        """qkv.rs:189-197."""
        per = {WriteGate.FIXED: 0, WriteGate.SCALAR: self.nheads,
               WriteGate.CHANNEL: self.key_dim() + self.value_dim()}[self.write_gate]
        return self.n_householder * per

    def d_in_proj(self) -> int:
        """qkv.rs:199-205."""
        return (self.conv_dim() + self.write_gate_width()
                + (self.value_dim() if self.has_gate else 0) + self.extra_channels)

    def conv_kernel(self) -> int:
        return 0 if self.conv is None else self.conv.conv_kernel()

    def zero_conv_window(self, batch: int, device, dtype=torch.float32) -> Optional[Tensor]:
        return None if self.conv is None else self.conv.zero_window(batch, device, dtype)

    def segments(self) -> List[Tuple[str, int]]:
        """qkv.rs:237-262."""
        u = self.n_householder
        seg = [("q", self.key_dim()), ("k", u * self.key_dim()), ("v", u * self.value_dim())]
        if self.write_gate == WriteGate.SCALAR:
            seg.append(("beta", u * self.nheads))
        elif self.write_gate == WriteGate.CHANNEL:
            seg += [("erase", u * self.key_dim()), ("write", u * self.value_dim())]
        if self.has_gate:
            seg.append(("gate", self.value_dim()))
        if self.extra_channels > 0:
            seg.append(("extra", self.extra_channels))
        return seg

    # -- forward ---------------------------------------------------------------

    def forward(self, x_bsd: Tensor, conv_window_bwc: Optional[Tensor],
                out_dtype=None) -> Tuple[Qkv, Optional[Tensor]]:
        """qkv.rs:373-449: in_proj, then dn_frontend."""
        if self.in_proj is None:
            raise DeltaError(-6, "QkvProjection.forward needs in_proj; use forward_projected")
        return self.forward_projected(self._in_proj(x_bsd), conv_window_bwc, out_dtype)

    def step(self, x_bd: Tensor, conv_window_bwc: Optional[Tensor],
             out_dtype=None) -> Tuple[QkvStep, Optional[Tensor]]:
        """qkv.rs:454-516: the single-token form."""
        if self.in_proj is None:
            raise DeltaError(-6, "QkvProjection.step needs in_proj; use step_projected")
        return self.step_projected(self._in_proj(x_bd), conv_window_bwc, out_dtype)

    def forward_projected(self, projected_bsw: Tensor, conv_window_bwc: Optional[Tensor],
                          out_dtype=None) -> Tuple[Qkv, Optional[Tensor]]:
        B, S, W = projected_bsw.shape
        if W != self.d_in_proj():
            raise DeltaError(-2, f"projection width {W} != d_in_proj {self.d_in_proj()}")
        outs, window = self._run(projected_bsw, conv_window_bwc, out_dtype)
        gate, extra = self._tail_views(projected_bsw)
        return Qkv(*outs, gate_bshv=gate, extra_bsx=extra), window

    def step_projected(self, projected_bw: Tensor, conv_window_bwc: Optional[Tensor],
                       out_dtype=None) -> Tuple[QkvStep, Optional[Tensor]]:
        B, W = projected_bw.shape
        if W != self.d_in_proj():
            raise DeltaError(-2, f"projection width {W} != d_in_proj {self.d_in_proj()}")
        outs, window = self._run(projected_bw.reshape(B, 1, W), conv_window_bwc, out_dtype)
        q, k, v, e, w = outs
        gate, extra = self._tail_views(projected_bw.reshape(B, 1, W))
        return QkvStep(q[:, 0], k, v, e, w,
                       gate_bhv=None if gate is None else gate[:, 0],
                       extra_bx=None if extra is None else extra[:, 0]), window

    # -- internals ---------------------------------------------------------------

    def _in_proj(self, x: Tensor) -> Tensor:
        y = torch.matmul(x, self.in_proj)
        return y if self.in_proj_bias is None else y + self.in_proj_bias

    def _tail_views(self, p: Tensor):
        """The output gate and the extra channels: views of the projection,
        as the reference's split + reshape give (qkv.rs:267-300, 429)."""
        B, S, _ = p.shape
        c = self.conv_dim() + self.write_gate_width()
        gate = None
        if self.has_gate:
            gate = p[:, :, c:c + self.value_dim()].unflatten(2, (self.nheads, self.head_v_dim))
            c += self.value_dim()
        extra = p[:, :, c:c + self.extra_channels] if self.extra_channels > 0 else None
        return gate, extra

    def _run(self, p: Tensor, window: Optional[Tensor], out_dtype):
        if (self.conv is None) != (window is None):
            raise DeltaError(-2, "convolution window presence must match the block's "
                                 "convolution")  # qkv.rs:397-401
        B, S, _ = p.shape
        if window is not None and tuple(window.shape) != (B, self.conv_dim(), self.conv_kernel()):
            raise DeltaError(-2, f"conv window: expected {[B, self.conv_dim(), self.conv_kernel()]}"
                                 f", got {list(window.shape)}")
        if not p.is_cuda:
            raise DeltaError(-6, "tensors must live on the GPU (no CPU fallback)")
        p = p.contiguous()
        H, dk, dv, u = self.nheads, self.head_k_dim, self.head_v_dim, self.n_householder
        od = p.dtype if out_dtype is None else out_dtype
        dev = p.device
        q = torch.empty((B, S, H, dk), dtype=od, device=dev)
        k = torch.empty((B, S * u, H, dk), dtype=od, device=dev)
        v = torch.empty((B, S * u, H, dv), dtype=od, device=dev)
        if self.write_gate == WriteGate.CHANNEL:
            erase = torch.empty((B, S * u, H, dk), dtype=torch.float32, device=dev)
            write = torch.empty((B, S * u, H, dv), dtype=torch.float32, device=dev)
        else:
            # One tensor for both halves, as the reference's (beta.clone(), beta).
            erase = torch.empty((B, S * u, H, 1), dtype=torch.float32, device=dev)
            write = erase
        win_in = win_out = weight = bias = None
        act = ConvActivation.IDENTITY
        if self.conv is not None:
            weight = self.conv.weight.reshape(self.conv_dim(), -1).float().contiguous()
            bias = None if self.conv.bias is None else self.conv.bias.float().contiguous()
            act = self.conv.activation
            win_in = window.to(p.dtype).contiguous()
            win_out = torch.empty_like(win_in)
        abi.run_frontend(abi.frontend_args(
            p, weight, bias, win_in, win_out, q, k, v, erase, write, nheads=H, head_k_dim=dk,
            head_v_dim=dv, n_householder=u, conv_activation=act,
            qk_activation=self.qk_activation, qk_norm=self.qk_norm,
            write_gate=self.write_gate, allow_neg_eigval=self.allow_neg_eigval))
        return (q, k, v, erase, write), win_out


@dataclass
class OutNorm:
    """OutNorm (norm.rs:106-144): RMSNorm over head_v_dim, per head, with
    weight γ; gated, it multiplies by silu(gate) after the norm. `eps` is the
    RmsNorm epsilon of burn_stack, which the reference does not vendor;
    1e-5 (Burn's RmsNorm default) unless set."""

    weight: Tensor
    gated: bool = True
    eps: float = 1e-5

    @staticmethod
    def init(head_v_dim: int, has_gate: bool, device) -> "OutNorm":
        """norm.rs:137-143 (γ = 1)."""
        return OutNorm(torch.ones(head_v_dim, device=device), gated=has_gate)

    def forward(self, x: Tensor, gate: Optional[Tensor] = None, out_dtype=None) -> Tensor:
        """norm.rs:127-134, over x [.., nheads, head_v_dim]."""
        if self.gated and gate is None:
            raise DeltaError(-6, "OutNorm::Gated needs an output gate")
        if not self.gated and gate is not None:
            raise DeltaError(-2, "OutNorm::Plain takes no output gate")
        if self.weight.numel() != x.shape[-1]:
            raise DeltaError(-2, f"weight: expected {x.shape[-1]} values, got {self.weight.numel()}")
        if not x.is_cuda:
            raise DeltaError(-6, "tensors must live on the GPU (no CPU fallback)")
        x = x.contiguous()
        out = torch.empty(x.shape, dtype=x.dtype if out_dtype is None else out_dtype,
                          device=x.device)
        w = self.weight.float().contiguous()
        abi.run_out_norm(abi.out_norm_args(x, gate, w, out, self.eps))
        return out


def block_step_args(proj: QkvProjection, norm: OutNorm, projected_bw: Tensor,
                    conv_window_bwc: Optional[Tensor], g_bhK: Optional[Tensor],
                    state_bhkv: Tensor, scale: Optional[float] = None, out_dtype=None,
                    in_place: bool = False, return_y: bool = False, check_finite: bool = False):
    """dn_block_step's arguments for `block_step` and the tensors it writes:
    (args, out_bhv, next_window, next_state, y_bhv or None, kept) — `kept`
    holds the converted inputs the arguments point into."""
    from .delta import _dev, _expect, _gate_axis
    B, W = projected_bw.shape
    if W != proj.d_in_proj():
        raise DeltaError(-2, f"projection width {W} != d_in_proj {proj.d_in_proj()}")
    if proj.n_householder != 1:
        raise DeltaError(-9, "dn_block_step serves n_householder = 1 (dn_recurrent covers more)")
    if (proj.conv is None) != (conv_window_bwc is None):
        raise DeltaError(-2, "convolution window presence must match the block's convolution")
    if norm.gated and not proj.has_gate:
        raise DeltaError(-6, "OutNorm::Gated needs the projection's output gate")
    if proj.has_gate and not norm.gated:
        # norm.rs OutNorm::forward panics on a gate given to the plain norm
        raise DeltaError(-2, "OutNorm::Plain takes no output gate")
    H, dk, dv = proj.nheads, proj.head_k_dim, proj.head_v_dim
    # The library sizes every buffer from these dims: a tensor that disagrees
    # would be read out of bounds.
    _expect(state_bhkv, (B, H, dk, dv), "state")
    if g_bhK is not None:
        _gate_axis(g_bhK, (B, H), dk, "forget gate")
    if conv_window_bwc is not None:
        _expect(conv_window_bwc, (B, proj.conv_dim(), proj.conv_kernel()), "conv window")
    if norm.weight.numel() != dv:
        raise DeltaError(-2, f"norm weight: expected {dv} values, got {norm.weight.numel()}")
    p = _dev(projected_bw)
    state = _dev(state_bhkv, torch.float32)
    g = _dev(g_bhK, torch.float32)
    a = abi.BlockStepArgs()
    a.batch, a.nheads, a.head_k_dim, a.head_v_dim = B, H, dk, dv
    a.conv_kernel = proj.conv_kernel()
    a.proj_stride = W
    a.conv_activation = int(proj.conv.activation) if proj.conv is not None else 0
    a.qk_activation, a.qk_norm = int(proj.qk_activation), int(proj.qk_norm)
    a.write_gate, a.allow_neg_eigval = int(proj.write_gate), int(proj.allow_neg_eigval)
    a.in_dtype = abi.dtype_tag(p.dtype)
    od = p.dtype if out_dtype is None else out_dtype
    a.out_dtype = abi.dtype_tag(od)
    a.has_gate = 0 if g is None else 1
    a.decay_width = 0 if g is None else g.shape[-1]
    a.scale = abi.nan_scale(scale)  # NaN: 1/sqrt(head_k_dim)
    a.eps = float(norm.eps)
    a.norm_gated = int(norm.gated)
    a.check_finite = int(check_finite)
    kept = [p, state, g]
    win_out = None
    if proj.conv is not None:
        weight = proj.conv.weight.reshape(proj.conv_dim(), -1).float().contiguous()
        bias = None if proj.conv.bias is None else proj.conv.bias.float().contiguous()
        win_in = conv_window_bwc.to(p.dtype).contiguous()
        win_out = win_in if (in_place and win_in is conv_window_bwc) else torch.empty_like(win_in)
        a.conv_weight, a.conv_bias = abi._ptr(weight), abi._ptr(bias)
        a.window_in, a.window_out = abi._ptr(win_in), abi._ptr(win_out)
        kept += [weight, bias, win_in]
    s_out = state if (in_place and state is state_bhkv) else torch.empty_like(state)
    gamma = norm.weight.float().contiguous()
    out = torch.empty((B, H, dv), dtype=od, device=p.device)
    y = torch.empty((B, H, dv), dtype=torch.float32, device=p.device) if return_y else None
    a.projected, a.g = p.data_ptr(), None if g is None else g.data_ptr()
    a.state_in, a.state_out = state.data_ptr(), s_out.data_ptr()
    a.norm_weight, a.out = abi._ptr(gamma), out.data_ptr()
    a.y = None if y is None else y.data_ptr()
    kept.append(gamma)
    return a, out, win_out, s_out, y, kept


def block_step(proj: QkvProjection, norm: OutNorm, projected_bw: Tensor,
               conv_window_bwc: Optional[Tensor], g_bhK: Optional[Tensor], state_bhkv: Tensor,
               scale: Optional[float] = None, out_dtype=None, in_place: bool = False,
               return_y: bool = False, check_finite: bool = False):
    """One decode token of a delta-rule block between in_proj and out_proj in
    one launch (dn_block_step): `proj.step_projected`, `delta_step` and
    `norm.forward`, as gated_deltanet_1.rs:218-234 runs them, given the forget
    gate g = log α ([batch, nheads, 1 | head_k_dim], or None). q, k, v and y
    stay in fp32 between the stages. Returns (out_bhv, next_window,
    next_state[, y_bhv]); with in_place the state and the window are updated
    where they are."""
    a, out, win_out, s_out, y, kept = block_step_args(
        proj, norm, projected_bw, conv_window_bwc, g_bhK, state_bhkv, scale, out_dtype,
        in_place, return_y, check_finite)
    abi.run_block_step(a)
    del kept
    return (out, win_out, s_out, y) if return_y else (out, win_out, s_out)
