"""The Python mirror's shape and device checks (CPU, no GPU needed).

The C ABI receives plain pointers and takes every size from q and v (or from
the block's dims), so a tensor that disagrees with them would be read out of
bounds on the GPU. Every entry that hands buffers to the library therefore
checks shapes first (path.rs:177-208, recurrent.rs:51-54) and refuses host
tensors. The tensors here live on the CPU: each case fails its check before
anything touches the device.
"""
import pytest
import torch

from conftest import load_package

pkg = load_package()
DeltaError = pkg.DeltaError


def chunk_inputs(B=1, S=8, H=2, K=4, V=6, ew=1, ww=1, dw=1):
    z = lambda *s: torch.zeros(s)
    return dict(q=z(B, S, H, K), k=z(B, S, H, K), v=z(B, S, H, V), e=z(B, S, H, ew),
                w=z(B, S, H, ww), g=z(B, S, H, dw), s=z(B, H, K, V))


def code_of(excinfo):
    return excinfo.value.code


@pytest.mark.parametrize("over,code,msg", [
    (dict(k=torch.zeros(1, 8, 2, 5)), -2, "k: expected shape [1, 8, 2, 4]"),
    (dict(v=torch.zeros(1, 7, 2, 6)), -2, "v: expected shape [1, 8, 2, 6]"),
    (dict(s=torch.zeros(1, 2, 4, 5)), -2, "state: expected shape [1, 2, 4, 6]"),
    (dict(e=torch.zeros(1, 8, 2, 3)), -3, "erase gate: last axis must be 1 or 4, got 3"),
    (dict(w=torch.zeros(1, 8, 3, 1)), -2, "write gate: expected leading dims [1, 8, 2]"),
    (dict(g=torch.zeros(1, 8, 2, 2)), -3, "forget gate: last axis must be 1 or 4, got 2"),
    (dict(q=torch.zeros(1, 8, 4)), -2, "q: expected [batch, sequence, nheads, ·]"),
])
def test_chunk_forward_checks_shapes_before_the_library(over, code, msg):
    t = chunk_inputs() | over
    with pytest.raises(DeltaError) as ex:
        pkg.delta_chunk_recalculated(t["q"], t["k"], t["v"], t["e"], t["w"], t["g"], t["s"],
                                     True, 64, float("nan"))
    assert code_of(ex) == code and msg in str(ex.value)


def test_ungated_chunk_forward_ignores_the_gate_tensor():
    """has_gate = False: the placeholder gate is never read, so its shape is
    not checked (chunk_recalculated.rs:50-56); the next check is the device."""
    t = chunk_inputs()
    with pytest.raises(DeltaError) as ex:
        pkg.delta_chunk_recalculated(t["q"], t["k"], t["v"], t["e"], t["w"],
                                     torch.zeros(1, 1, 1, 1), t["s"], False, 64, float("nan"))
    assert code_of(ex) == -6


def test_chunk_backward_checks_the_cotangent_shapes():
    t = chunk_inputs()
    args = (t["q"], t["k"], t["v"], t["e"], t["w"], t["g"], t["s"], 64, float("nan"))
    with pytest.raises(DeltaError) as ex:
        pkg.combined_backward(torch.zeros(1, 8, 2, 5), t["s"], *args)
    assert code_of(ex) == -2 and "d_y" in str(ex.value)
    with pytest.raises(DeltaError) as ex:
        pkg.combined_backward(torch.zeros(1, 8, 2, 6), torch.zeros(1, 2, 4, 4), *args)
    assert code_of(ex) == -2 and "d_final_state" in str(ex.value)
    with pytest.raises(DeltaError) as ex:
        pkg.combined_backward(torch.zeros(1, 8, 2, 6), None, t["q"], torch.zeros(1, 8, 2, 3),
                              *args[2:])
    assert code_of(ex) == -2 and "k:" in str(ex.value)


def test_recurrent_checks_shapes_when_called_directly():
    """DeltaInput.delta_recurrent (not only run) checks before the library."""
    t = chunk_inputs()
    di = pkg.DeltaInput(t["q"], t["k"], t["v"], torch.zeros(1, 8, 2, 3), t["w"], t["g"], t["s"])
    with pytest.raises(DeltaError) as ex:
        di.delta_recurrent()
    assert code_of(ex) == -3


@pytest.mark.parametrize("over,code,msg", [
    (dict(v=torch.zeros(1, 3, 6)), -2, "v: expected shape [1, 2, 6]"),
    (dict(e=torch.zeros(2, 2, 1)), -2, "erase gate: expected leading dims [1, 2]"),
    (dict(w=torch.zeros(1, 2, 5)), -3, "write gate: last axis must be 1 or 6, got 5"),
    (dict(g=torch.zeros(1, 2, 3)), -3, "forget gate: last axis must be 1 or 4, got 3"),
    (dict(s=torch.zeros(1, 2, 6, 4)), -2, "state: expected shape [1, 2, 4, 6]"),
])
def test_step_checks_shapes(over, code, msg):
    z = torch.zeros
    t = dict(q=z(1, 2, 4), k=z(1, 2, 4), v=z(1, 2, 6), e=z(1, 2, 1), w=z(1, 2, 1), g=z(1, 2, 1),
             s=z(1, 2, 4, 6)) | over
    with pytest.raises(DeltaError) as ex:
        pkg.delta_step(t["q"], t["k"], t["v"], t["e"], t["w"], t["g"], t["s"], 0.5)
    assert code_of(ex) == code and msg in str(ex.value)


def test_abi_pointer_helper_refuses_host_tensors():
    with pytest.raises(DeltaError) as ex:
        pkg.abi._ptr(torch.zeros(4))
    assert code_of(ex) == -6
    assert pkg.abi._ptr(None) is None


def test_out_norm_checks_the_weight_length():
    norm = pkg.OutNorm(torch.ones(5), gated=False)
    with pytest.raises(DeltaError) as ex:
        norm.forward(torch.zeros(3, 2, 6))
    assert code_of(ex) == -2 and "weight: expected 6 values, got 5" in str(ex.value)


def _block(H=2, dk=4, dv=6, conv_k=3):
    proj = pkg.QkvProjection(nheads=H, head_k_dim=dk, head_v_dim=dv, has_gate=True)
    proj.conv = pkg.ShortConv(torch.zeros(proj.conv_dim(), conv_k), None,
                              pkg.ConvActivation.SILU)
    return proj, pkg.OutNorm(torch.ones(dv), gated=True)


@pytest.mark.parametrize("what,msg", [
    ("state", "state: expected shape [2, 2, 4, 6]"),
    ("g", "forget gate: expected leading dims [2, 2]"),
    ("window", "conv window: expected shape"),
    ("weight", "norm weight: expected 6 values, got 7"),
])
def test_block_step_checks_shapes_before_the_library(what, msg):
    proj, norm = _block()
    B = 2
    p = torch.zeros(B, proj.d_in_proj())
    win = torch.zeros(B, proj.conv_dim(), 3)
    g, s = torch.zeros(B, 2, 1), torch.zeros(B, 2, 4, 6)
    if what == "state":
        s = torch.zeros(B, 2, 6, 4)
    elif what == "g":
        g = torch.zeros(B, 3, 1)
    elif what == "window":
        win = torch.zeros(B, proj.conv_dim(), 4)
    else:
        norm = pkg.OutNorm(torch.ones(7), gated=True)
    with pytest.raises(DeltaError) as ex:
        pkg.block_step(proj, norm, p, win, g, s)
    assert code_of(ex) == -2 and msg in str(ex.value)


def test_frontend_checks_the_window_shape():
    proj, _ = _block()
    p = torch.zeros(2, 5, proj.d_in_proj())
    with pytest.raises(DeltaError) as ex:
        proj.forward_projected(p, torch.zeros(2, proj.conv_dim(), 2))
    assert code_of(ex) == -2 and "conv window" in str(ex.value)


def test_block_step_refuses_a_gate_for_the_plain_norm():
    """A projection with an output gate and OutNorm::Plain: the reference's
    OutNorm::forward panics on the gate (norm.rs), and so does the mirror,
    before any library call."""
    proj, _ = _block()
    B = 2
    with pytest.raises(DeltaError) as ex:
        pkg.block_step(proj, pkg.OutNorm(torch.ones(6), gated=False),
                       torch.zeros(B, proj.d_in_proj()), torch.zeros(B, proj.conv_dim(), 3),
                       torch.zeros(B, 2, 1), torch.zeros(B, 2, 4, 6))
    assert code_of(ex) == -2 and "OutNorm::Plain takes no output gate" in str(ex.value)
