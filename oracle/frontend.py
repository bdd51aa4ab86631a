"""CPU oracle of the projection front-end — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker. It restates, in float64 numpy, what the
reference runs between the fused in-projection and the delta rule:

    QkvProjection::forward after in_proj   (src/common/qkv.rs:373-449)
    QkvProjection::step after in_proj      (src/common/qkv.rs:454-516)
    ShortConv::forward / ShortConv::step   (src/common/conv.rs:85-158)
    QkActivation / QkNorm / l2_normalize   (src/common/norm.rs:36-97)
    squash_write                           (src/common/qkv.rs:332-369)
    OutNorm::forward                       (src/common/norm.rs:106-144)

Layouts are the reference's: `projected` [B, S, ≥ conv_dim + gate width] with
the segments [q | k (u copies) | v (u copies) | β or (erase | write)]
(qkv.rs:237-262); the convolution window [B, conv_dim, kernel] with the
newest column last (conv.rs:14-20); the weight [conv_dim, kernel] (Conv1d's
[conv_dim, 1, kernel] without its unit axis).

Out of scope, as in the HIP front-end: grouped values (n_value_heads ≠
nheads) and QkNorm::Sum. Both depend on burn_stack code that is not vendored
in the reference (gqa_expand_to_heads, div_eps).
"""

from __future__ import annotations

import numpy as np

# Enumerations shared with include/deltanet_core.h.
ACT_IDENTITY, ACT_SILU, ACT_RELU, ACT_ELU_PLUS_ONE = 0, 1, 2, 3
QKNORM_NONE, QKNORM_L2 = 0, 1
WRITE_FIXED, WRITE_SCALAR, WRITE_CHANNEL = 0, 1, 2

L2_EPS = 1e-6  # norm.rs:83


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    """x·σ(x) (burn_stack Silu, as norm.rs:28 and conv.rs:30 describe it)."""
    return x * sigmoid(x)


def activation(x, kind):
    """QkActivation::apply (norm.rs:38-51); ConvActivation::apply (conv.rs:39-44)
    uses the first two."""
    if kind == ACT_IDENTITY:
        return x
    if kind == ACT_SILU:
        return silu(x)
    if kind == ACT_RELU:
        return np.maximum(x, 0.0)
    if kind == ACT_ELU_PLUS_ONE:
        return np.where(x < 0.0, np.exp(np.minimum(x, 0.0)), np.maximum(x, 0.0) + 1.0)
    raise ValueError(f"unknown activation {kind}")


def l2_normalize(x):
    """x / √(Σx² + ε) over the last axis (norm.rs:85-90)."""
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + L2_EPS)


def qk_norm(x, kind):
    """QkNorm::apply (norm.rs:69-75), L2 and None."""
    if kind == QKNORM_L2:
        return l2_normalize(x)
    if kind == QKNORM_NONE:
        return x
    raise ValueError(f"unsupported qk_norm {kind}")


def short_conv(x_bsw, window_bwc, weight_wk, bias_w, act):
    """ShortConv::forward (conv.rs:85-121): left-pad with the window's newest
    kernel−1 columns, depthwise cross-correlation with Valid padding, the
    activation; the next window is the padded input's last `kernel` columns."""
    B, S, W = x_bsw.shape
    K = weight_wk.shape[1]
    x_bws = np.transpose(x_bsw, (0, 2, 1))
    padded = np.concatenate([window_bwc[:, :, 1:], x_bws], axis=2) if K >= 2 else x_bws
    nxt = padded[:, :, S - 1:].copy()
    y = np.zeros((B, W, S))
    for j in range(K):
        y += weight_wk[None, :, j, None] * padded[:, :, j:j + S]
    if bias_w is not None:
        y += bias_w[None, :, None]
    return activation(np.transpose(y, (0, 2, 1)), act), nxt


def short_conv_step(x_bw, window_bwc, weight_wk, bias_w, act):
    """ShortConv::step (conv.rs:124-158): slide the window by one token, then
    the filter's dot product with it."""
    nxt = np.concatenate([window_bwc[:, :, 1:], x_bw[:, :, None]], axis=2)
    y = (nxt * weight_wk[None]).sum(2)
    if bias_w is not None:
        y = y + bias_w[None]
    return activation(y, act), nxt


def frontend(projected, *, nheads, head_k_dim, head_v_dim, n_householder=1, conv=None,
             qk_activation=ACT_SILU, qk_norm_kind=QKNORM_L2, write_gate=WRITE_SCALAR,
             allow_neg_eigval=False):
    """QkvProjection::forward from the projection output on (qkv.rs:373-449).

    `conv` is None or a dict(weight [conv_dim, K], bias [conv_dim] | None,
    window [B, conv_dim, K], activation). Returns dict(q, k, v, erase, write,
    window) with q [B, S, H, dk], k [B, S·u, H, dk], v [B, S·u, H, dv],
    erase [B, S·u, H, 1|dk], write [B, S·u, H, 1|dv]; window is None without
    a convolution."""
    p = np.asarray(projected, np.float64)
    B, S, _ = p.shape
    H, dk, dv, u = nheads, head_k_dim, head_v_dim, n_householder
    key_dim, value_dim = H * dk, H * dv
    conv_dim = key_dim + u * (key_dim + value_dim)
    x = p[:, :, :conv_dim]
    window = None
    if conv is not None:
        x, window = short_conv(x, np.asarray(conv["window"], np.float64),
                               np.asarray(conv["weight"], np.float64),
                               None if conv.get("bias") is None
                               else np.asarray(conv["bias"], np.float64),
                               conv["activation"])
    q = x[:, :, :key_dim].reshape(B, S, H, dk)
    k = x[:, :, key_dim:key_dim + u * key_dim].reshape(B, S * u, H, dk)
    v = x[:, :, key_dim + u * key_dim:conv_dim].reshape(B, S * u, H, dv)
    fused = (qk_activation == ACT_SILU and conv is not None
             and conv["activation"] == ACT_SILU)  # qkv.rs:223-229, 413-421
    if not fused:
        q, k, v = activation(q, qk_activation), activation(k, qk_activation), silu(v)
    q, k = qk_norm(q, qk_norm_kind), qk_norm(k, qk_norm_kind)
    # squash_write (qkv.rs:332-369)
    scale = 2.0 if allow_neg_eigval else 1.0
    g0 = conv_dim
    if write_gate == WRITE_FIXED:
        erase = np.full((B, S * u, H, 1), scale)
        write = erase.copy()
    elif write_gate == WRITE_SCALAR:
        erase = scale * sigmoid(p[:, :, g0:g0 + u * H]).reshape(B, S * u, H, 1)
        write = erase.copy()
    elif write_gate == WRITE_CHANNEL:
        erase = scale * sigmoid(p[:, :, g0:g0 + u * key_dim]).reshape(B, S * u, H, dk)
        write = sigmoid(p[:, :, g0 + u * key_dim:g0 + u * (key_dim + value_dim)]).reshape(
            B, S * u, H, dv)
    else:
        raise ValueError(f"unknown write gate {write_gate}")
    return dict(q=q, k=k, v=v, erase=erase, write=write, window=window)


def gate_width(nheads, head_k_dim, head_v_dim, n_householder, write_gate):
    """QkvProjection::write_gate_width (qkv.rs:189-197)."""
    per = {WRITE_FIXED: 0, WRITE_SCALAR: nheads,
           WRITE_CHANNEL: nheads * (head_k_dim + head_v_dim)}[write_gate]
    return n_householder * per


def conv_dim(nheads, head_k_dim, head_v_dim, n_householder):
    """QkvProjection::conv_dim (qkv.rs:180-182)."""
    return nheads * head_k_dim + n_householder * nheads * (head_k_dim + head_v_dim)


def out_norm(x, gate, weight, eps):
    """OutNorm::forward (norm.rs:106-144), per head over the last axis:
    x / √(mean(x²) + ε) · γ, times silu(gate) when gated. ε is burn_stack's
    RmsNorm(Gated) epsilon, which the reference does not vendor: parity in ε
    is unpinned, so it is an argument here."""
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(weight, np.float64)
    if gate is not None:
        y = y * silu(np.asarray(gate, np.float64))
    return y
