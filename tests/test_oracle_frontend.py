"""Pins of the front-end oracle (oracle/frontend.py) on the CPU.

Each check is chosen so that a plausible slip in the restatement fails it:
the convolution's tap orientation against torch's conv1d (a library routine
with Burn's cross-correlation convention), its impulse response, forward ≡
unrolled step and split stream ≡ whole (ShortConv's own contract,
conv.rs:1-20), the segment / micro-step mapping against channel-tagged inputs
(qkv.rs:237-262, 403-411), the L2 norm's invariants (norm.rs:77-90), and the
activations at special points (norm.rs:22-51)."""

import numpy as np
import pytest
import torch

from oracle import frontend as F


def rand_conv(rng, B, W, K):
    return dict(weight=rng.standard_normal((W, K)), bias=rng.standard_normal(W),
                window=rng.standard_normal((B, W, K)), activation=F.ACT_IDENTITY)


@pytest.mark.parametrize("K", [1, 2, 4, 6])
def test_conv_matches_torch_conv1d(rng, K):
    B, S, W = 2, 11, 5
    c = rand_conv(rng, B, W, K)
    x = rng.standard_normal((B, S, W))
    y, nxt = F.short_conv(x, c["window"], c["weight"], c["bias"], F.ACT_IDENTITY)
    padded = np.concatenate([c["window"][:, :, 1:], x.transpose(0, 2, 1)], 2)
    ref = torch.nn.functional.conv1d(torch.tensor(padded), torch.tensor(c["weight"][:, None]),
                                     torch.tensor(c["bias"]), groups=W).numpy()
    assert np.abs(y - ref.transpose(0, 2, 1)).max() < 1e-12
    assert np.array_equal(nxt, padded[:, :, -K:])


def test_conv_impulse_response_is_the_reversed_filter(rng):
    K, W, S = 4, 3, 9
    w = rng.standard_normal((W, K))
    x = np.zeros((1, S, W))
    x[0, 2] = 1.0
    y, _ = F.short_conv(x, np.zeros((1, W, K)), w, None, F.ACT_IDENTITY)
    for d in range(K):
        assert np.allclose(y[0, 2 + d], w[:, K - 1 - d])
    assert np.allclose(y[0, :2], 0) and np.allclose(y[0, 2 + K:], 0)


@pytest.mark.parametrize("act", [F.ACT_IDENTITY, F.ACT_SILU])
def test_conv_forward_equals_unrolled_step(rng, act):
    B, S, W, K = 2, 7, 6, 4
    c = rand_conv(rng, B, W, K)
    x = rng.standard_normal((B, S, W))
    y, nxt = F.short_conv(x, c["window"], c["weight"], c["bias"], act)
    win = c["window"]
    for t in range(S):
        yt, win = F.short_conv_step(x[:, t], win, c["weight"], c["bias"], act)
        assert np.abs(yt - y[:, t]).max() < 1e-12
    assert np.array_equal(win, nxt)


def test_conv_split_stream_equals_whole(rng):
    B, S, W, K = 1, 10, 4, 4
    c = rand_conv(rng, B, W, K)
    x = rng.standard_normal((B, S, W))
    y, nxt = F.short_conv(x, c["window"], c["weight"], c["bias"], F.ACT_SILU)
    for cut in [1, 2, 5]:
        y1, w1 = F.short_conv(x[:, :cut], c["window"], c["weight"], c["bias"], F.ACT_SILU)
        y2, w2 = F.short_conv(x[:, cut:], w1, c["weight"], c["bias"], F.ACT_SILU)
        assert np.abs(np.concatenate([y1, y2], 1) - y).max() < 1e-12
        assert np.array_equal(w2, nxt)


def test_segments_and_micro_steps_map_by_channel(rng):
    """No convolution, identity q/k activation and no norm: q and k are the
    raw segments, v their SiLU; k and v fold u copies into the sequence."""
    B, S, H, dk, dv, u = 2, 3, 2, 4, 5, 3
    cd = F.conv_dim(H, dk, dv, u)
    gw = F.gate_width(H, dk, dv, u, F.WRITE_CHANNEL)
    p = rng.standard_normal((B, S, cd + gw + 7))
    o = F.frontend(p, nheads=H, head_k_dim=dk, head_v_dim=dv, n_householder=u,
                   qk_activation=F.ACT_IDENTITY, qk_norm_kind=F.QKNORM_NONE,
                   write_gate=F.WRITE_CHANNEL, allow_neg_eigval=True)
    key_dim, value_dim = H * dk, H * dv
    for b in range(B):
        for s in range(S):
            for h in range(H):
                assert np.array_equal(o["q"][b, s, h], p[b, s, h * dk:(h + 1) * dk])
                for m in range(u):
                    kc = key_dim + m * key_dim + h * dk
                    vc = key_dim * (1 + u) + m * value_dim + h * dv
                    assert np.array_equal(o["k"][b, s * u + m, h], p[b, s, kc:kc + dk])
                    assert np.allclose(o["v"][b, s * u + m, h], F.silu(p[b, s, vc:vc + dv]))
                    ec = cd + m * key_dim + h * dk
                    wc = cd + u * key_dim + m * value_dim + h * dv
                    assert np.allclose(o["erase"][b, s * u + m, h],
                                       2 * F.sigmoid(p[b, s, ec:ec + dk]))
                    assert np.allclose(o["write"][b, s * u + m, h],
                                       F.sigmoid(p[b, s, wc:wc + dv]))


def test_scalar_and_fixed_gates(rng):
    B, S, H, dk, dv, u = 1, 4, 3, 2, 2, 2
    cd = F.conv_dim(H, dk, dv, u)
    p = rng.standard_normal((B, S, cd + u * H))
    for neg in [False, True]:
        o = F.frontend(p, nheads=H, head_k_dim=dk, head_v_dim=dv, n_householder=u,
                       write_gate=F.WRITE_SCALAR, allow_neg_eigval=neg)
        want = (2 if neg else 1) * F.sigmoid(p[:, :, cd:]).reshape(B, S * u, H, 1)
        assert np.allclose(o["erase"], want) and np.allclose(o["write"], want)
        o = F.frontend(p[:, :, :cd], nheads=H, head_k_dim=dk, head_v_dim=dv, n_householder=u,
                       write_gate=F.WRITE_FIXED, allow_neg_eigval=neg)
        assert np.all(o["erase"] == (2 if neg else 1)) and o["erase"].shape == (B, S * u, H, 1)


def test_activation_fusion_rule(rng):
    """SiLU runs once: in the convolution when both it and qk_activation are
    SiLU (qkv.rs:223-229), after it otherwise."""
    B, S, H, d = 1, 3, 1, 4
    cd = F.conv_dim(H, d, d, 1)
    p = rng.standard_normal((B, S, cd + H))
    ident = dict(weight=np.ones((cd, 1)), bias=None, window=np.zeros((B, cd, 1)))
    kw = dict(nheads=H, head_k_dim=d, head_v_dim=d, qk_norm_kind=F.QKNORM_NONE)
    fused = F.frontend(p, conv=dict(ident, activation=F.ACT_SILU), qk_activation=F.ACT_SILU,
                       **kw)
    split = F.frontend(p, conv=dict(ident, activation=F.ACT_IDENTITY),
                       qk_activation=F.ACT_SILU, **kw)
    for name in ["q", "k", "v"]:
        assert np.allclose(fused[name], split[name])
    assert np.allclose(fused["q"][0, :, 0], F.silu(p[0, :, :d]))


def test_l2_norm_invariants(rng):
    x = rng.standard_normal((5, 7, 16)) * 10
    n = F.l2_normalize(x)
    assert np.allclose(np.linalg.norm(n, axis=-1), 1.0, atol=1e-8)
    assert np.allclose(F.l2_normalize(3.7 * x), n, atol=1e-8)
    assert np.array_equal(F.l2_normalize(np.zeros((2, 8))), np.zeros((2, 8)))
    tiny = np.full((1, 4), 1e-4)  # Σx² = 4e-8, well below ε: scaled by 1/√(ε + 4e-8)
    assert np.allclose(F.l2_normalize(tiny), tiny / np.sqrt(1e-6 + 4e-8))


def test_activations_at_special_points():
    x = np.array([-50.0, -1.0, 0.0, 1.0, 50.0])
    assert np.allclose(F.activation(x, F.ACT_SILU), [-50 / (1 + np.exp(50)), -1 / (1 + np.e),
                                                     0.0, 1 / (1 + np.exp(-1)), 50.0])
    assert np.array_equal(F.activation(x, F.ACT_RELU), [0, 0, 0, 1, 50])
    e = F.activation(x, F.ACT_ELU_PLUS_ONE)
    assert np.allclose(e, [np.exp(-50), np.exp(-1), 1.0, 2.0, 51.0]) and np.all(e > 0)
    assert F.sigmoid(np.array(0.0)) == 0.5


def test_out_norm_is_torch_rms_norm_times_silu_gate(rng):
    """OutNorm's plain form against torch's rms_norm (a library routine:
    the mean of squares over the last axis, ε inside the root); the gated
    form multiplies by silu(gate) after the norm (norm.rs:106-113)."""
    x = rng.standard_normal((3, 5, 4, 16))
    w = rng.standard_normal(16)
    g = rng.standard_normal(x.shape)
    for eps in [1e-5, 1e-2]:
        ref = torch.nn.functional.rms_norm(torch.tensor(x), (16,), torch.tensor(w), eps).numpy()
        assert np.abs(F.out_norm(x, None, w, eps) - ref).max() < 1e-12
        assert np.abs(F.out_norm(x, g, w, eps) - ref * F.silu(g)).max() < 1e-12


def test_out_norm_closed_forms():
    c = np.full((1, 8), -3.0)
    assert np.allclose(F.out_norm(c, None, np.ones(8), 0.0), -1.0)       # a constant row → ±1
    assert np.allclose(F.out_norm(c, np.zeros((1, 8)), np.ones(8), 1e-5), 0.0)  # silu(0) = 0
    assert np.allclose(F.out_norm(np.zeros((1, 8)), None, np.ones(8), 1e-5), 0.0)
