"""The C ABI without a GPU: the library loads, exports every symbol that
include/deltanet_core.h declares, and rejects invalid arguments with the
status codes that mirror the reference's assertions (path.rs:177-231,
recurrent.rs:51-54) before touching the device."""

import ctypes
import re

import pytest
import torch

from conftest import ROOT, load_package

pkg = load_package()
abi = pkg.abi

# The argument-check cases below pass a fake device address (0x1000) that a
# correct check never lets through. They run only where no GPU is visible, so
# that a regression in a check can never launch a kernel on that address.
fake_pointers = pytest.mark.skipif(
    torch.cuda.is_available(),
    reason="fake-pointer argument checks run on CPU-only hosts (no kernel can launch there)")


def header_symbols():
    text = (ROOT / "include" / "deltanet_core.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int64_t|int|size_t|const char \*)\s*(dn_\w+)\s*\(", text,
                                 re.M)))


def test_header_declares_the_three_entry_points():
    syms = header_symbols()
    for name in ["dn_chunk_fwd", "dn_chunk_bwd", "dn_step"]:
        assert name in syms
    assert sorted(abi.EXPORTS) == syms


def test_library_exports_every_declared_symbol():
    lib = abi.lib()
    for name in header_symbols():
        assert hasattr(lib, name), name
    assert b"gfx950" in lib.dn_version()


def fwd_args(**over):
    a = abi.ChunkFwdArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = 1, 8, 1, 4, 6
    a.erase_width, a.write_width, a.decay_width = 1, 1, 1
    a.has_gate, a.chunk_len, a.scale = 1, 64, float("nan")
    a.qkv_dtype = a.y_dtype = abi.DN_F32
    fake = 0x1000  # never dereferenced: every case below fails its checks first
    for f in ["q", "k", "v", "erase", "write", "g", "state_in", "y", "state_out"]:
        setattr(a, f, fake)
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,code,msg", [
    (dict(sequence=0), -1, "sequence length must be at least 1"),
    (dict(batch=0), -2, "at least 1"),
    (dict(erase_width=3), -3, "erase gate: last axis must be 1 or 4, got 3"),
    (dict(write_width=5), -3, "write gate: last axis must be 1 or 6, got 5"),
    (dict(decay_width=2), -3, "forget gate: last axis must be 1 or 4, got 2"),
    (dict(chunk_len=0), -4, "chunk_len must be at least 1"),
    # The generic kernels' 32-bit tile indexing: chunk_len² and chunk_len·dv.
    (dict(chunk_len=46341), -4, "chunk_len too large"),
    (dict(chunk_len=1 << 15, head_v_dim=1 << 16, write_width=1), -4, "chunk_len too large"),
    (dict(chunk_len=46340, q=None), -6, "NULL"),  # the largest accepted, then the next check
    # Extents past 32 bits, or a product that would overflow on the way,
    # are refused rather than narrowed.
    (dict(sequence=(1 << 31) + 1), -2, "tensor too large"),
    (dict(batch=1 << 30, sequence=1 << 30, nheads=1 << 30), -2, "tensor too large"),
    (dict(qkv_dtype=7), -7, "dtype"),
    (dict(q=None), -6, "NULL"),
])
@fake_pointers
def test_chunk_fwd_rejects_invalid_arguments(over, code, msg):
    lib = abi.lib()
    a = fwd_args(**over)
    rc = lib.dn_chunk_fwd(ctypes.byref(a), None)
    assert rc == code
    assert msg in lib.dn_last_error().decode()
    assert lib.dn_chunk_fwd_workspace_bytes(ctypes.byref(a)) == 0


@fake_pointers
def test_ungated_call_ignores_the_gate_width():
    """has_gate = 0 is the reference's placeholder gate (chunk_recalculated.rs:50-56):
    its width is never checked."""
    a = fwd_args(has_gate=0, decay_width=2, g=None, chunk_len=0)
    assert abi.lib().dn_chunk_fwd(ctypes.byref(a), None) == -4


@fake_pointers
def test_step_rejects_invalid_arguments():
    lib = abi.lib()
    a = abi.StepArgs()
    a.batch, a.nheads, a.head_k_dim, a.head_v_dim = 1, 1, 4, 6
    a.erase_width, a.write_width, a.decay_width, a.has_gate = 2, 1, 0, 0
    a.scale = 1.0
    assert lib.dn_step(ctypes.byref(a), None) == -3
    a.erase_width = 1
    assert lib.dn_step(ctypes.byref(a), None) == -6  # null pointers


@pytest.mark.parametrize("over,code,msg", [
    (dict(sequence=0), -1, "sequence length must be at least 1"),
    (dict(nheads=0), -2, "at least 1"),
    (dict(erase_width=3), -3, "erase gate: last axis must be 1 or 4, got 3"),
    (dict(write_width=5), -3, "write gate: last axis must be 1 or 6, got 5"),
    (dict(decay_width=2), -3, "forget gate: last axis must be 1 or 4, got 2"),
    (dict(y_dtype=3), -7, "dtype"),
    (dict(state_out=None), -6, "NULL"),
    (dict(head_k_dim=abi.RECURRENT_MAX_K + 1, erase_width=1, decay_width=1), -9,
     f"head_k_dim up to {abi.RECURRENT_MAX_K}"),
])
@fake_pointers
def test_recurrent_rejects_invalid_arguments(over, code, msg):
    """dn_recurrent takes dn_chunk_fwd's shape rules (no chunk_len) and
    refuses heads above its limit before touching any pointer."""
    lib = abi.lib()
    a = abi.RecurrentArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = 1, 8, 1, 4, 6
    a.erase_width, a.write_width, a.decay_width, a.has_gate = 1, 1, 1, 1
    a.scale = float("nan")
    a.qkv_dtype = a.y_dtype = abi.DN_F32
    for f in ["q", "k", "v", "erase", "write", "g", "state_in", "y", "state_out"]:
        setattr(a, f, 0x1000)  # never dereferenced: every case fails its checks first
    for k, v in over.items():
        setattr(a, k, v)
    assert lib.dn_recurrent(ctypes.byref(a), None) == code
    assert msg in lib.dn_last_error().decode()


@fake_pointers
def test_forward_algorithm_choice():
    """AUTO runs the two-kernel MFMA forward; DN_ALGO_MFMA_FUSED, on request
    only, the one-kernel forward, which needs only the sink row as workspace
    and serves per-head gates at head_k_dim 128 and head_v_dim a multiple of
    128."""
    lib = abi.lib()
    MFMA, FUSED = abi.DN_ALGO_MFMA, abi.DN_ALGO_MFMA_FUSED
    base = dict(batch=8, sequence=4096, nheads=16, head_k_dim=128, head_v_dim=256,
                qkv_dtype=abi.DN_BF16, y_dtype=abi.DN_BF16)
    ws = {}
    for algo, want in ((abi.DN_ALGO_AUTO, MFMA), (MFMA, MFMA), (FUSED, FUSED)):
        a = fwd_args(**base, algo=algo)
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == want
        ws[algo] = lib.dn_chunk_fwd_workspace_bytes(ctypes.byref(a))
    assert ws[FUSED] == 256 * 4  # one fp32-sized y row
    assert ws[abi.DN_ALGO_AUTO] == ws[MFMA] > 100 * 2**20
    for over in (dict(head_k_dim=64), dict(head_v_dim=192), dict(erase_width=128),
                 dict(qkv_dtype=abi.DN_F32)):
        a = fwd_args(**{**base, **over}, algo=FUSED)
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == -9, over
        assert lib.dn_chunk_fwd_workspace_bytes(ctypes.byref(a)) == 0


@fake_pointers
def test_mfma_paths_need_word_aligned_qkv():
    """The MFMA kernels read q and k in 16-byte words and v in 4-byte words:
    a view that starts off those boundaries runs the generic kernels under
    AUTO, and an explicit MFMA request is refused (no pointer is read)."""
    lib = abi.lib()
    base = dict(batch=8, sequence=4096, nheads=16, head_k_dim=128, head_v_dim=256,
                qkv_dtype=abi.DN_BF16, y_dtype=abi.DN_BF16)
    for over, auto in ((dict(), abi.DN_ALGO_MFMA), (dict(q=0x1008), abi.DN_ALGO_GENERIC),
                       (dict(k=0x1002), abi.DN_ALGO_GENERIC), (dict(v=0x1002), abi.DN_ALGO_GENERIC),
                       (dict(v=0x1004), abi.DN_ALGO_MFMA)):
        a = fwd_args(**base, **over, algo=abi.DN_ALGO_AUTO)
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == auto, over
        a = fwd_args(**base, **over, algo=abi.DN_ALGO_MFMA)
        want = abi.DN_ALGO_MFMA if auto == abi.DN_ALGO_MFMA else -9
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == want, over


def test_mfma_serves_any_chunk_len_for_per_head_gates():
    """The MFMA kernels' 64-token chunks serve every chunk_len when the
    forget gate is per head or absent (the chunk length changes only the
    order of roundings), with chunk 64's workspace; with a per-channel forget
    gate, whose block-decay clamp depends on where chunks start, only 64 is
    served there. No pointer is read."""
    lib = abi.lib()
    base = dict(batch=2, sequence=1000, nheads=4, head_k_dim=128, head_v_dim=128,
                qkv_dtype=abi.DN_BF16, y_dtype=abi.DN_BF16)
    ref = fwd_args(**base, chunk_len=64)
    ws64 = lib.dn_chunk_fwd_workspace_bytes(ctypes.byref(ref))
    for L in (1, 16, 32, 100, 128, 4096):
        for algo, want in ((abi.DN_ALGO_AUTO, abi.DN_ALGO_MFMA),
                           (abi.DN_ALGO_MFMA, abi.DN_ALGO_MFMA),
                           (abi.DN_ALGO_MFMA_FUSED, abi.DN_ALGO_MFMA_FUSED)):
            a = fwd_args(**base, chunk_len=L, algo=algo)
            assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == want, (L, algo)
        a = fwd_args(**base, chunk_len=L)
        assert lib.dn_chunk_fwd_workspace_bytes(ctypes.byref(a)) == ws64, L
        a = fwd_args(**base, chunk_len=L, has_gate=0)
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == abi.DN_ALGO_MFMA, L
        b = bwd_args(chunk_len=L)
        assert lib.dn_chunk_bwd_algo(ctypes.byref(b)) == abi.DN_ALGO_MFMA, L
        assert (lib.dn_chunk_bwd_workspace_bytes(ctypes.byref(b)) ==
                lib.dn_chunk_bwd_workspace_bytes(ctypes.byref(bwd_args(chunk_len=64)))), L
    pc = dict(base, erase_width=128, write_width=128, decay_width=128)
    assert lib.dn_chunk_fwd_algo(ctypes.byref(fwd_args(**pc, chunk_len=64))) == abi.DN_ALGO_MFMA
    for L in (32, 128):
        assert lib.dn_chunk_fwd_algo(ctypes.byref(fwd_args(**pc, chunk_len=L))) == \
            abi.DN_ALGO_GENERIC
        a = fwd_args(**pc, chunk_len=L, algo=abi.DN_ALGO_MFMA)
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == -9
        b = bwd_args(chunk_len=L, head_v_dim=128, erase_width=128, write_width=128,
                     decay_width=128)
        assert lib.dn_chunk_bwd_algo(ctypes.byref(b)) == abi.DN_ALGO_GENERIC


@pytest.mark.parametrize("over,code,msg", [
    (dict(weight=None), -6, "norm weight is NULL"),
    (dict(eps=-1.0), -2, "eps must be finite and non-negative"),
    (dict(eps=float("inf")), -2, "eps must be finite and non-negative"),
    (dict(gate_stride=5), -2, "gate_stride must cover nheads * head_v_dim"),
    (dict(gate_dtype=9), -7, "dtype"),
    (dict(fwd_over=dict(sequence=0)), -1, "sequence length must be at least 1"),
    (dict(fwd_over=dict(head_v_dim=2048, write_width=1)), -9, "head_v_dim up to 1024"),
])
@fake_pointers
def test_chunk_fwd_out_norm_rejects_invalid_arguments(over, code, msg):
    lib = abi.lib()
    a = abi.ChunkFwdOutNormArgs()
    a.fwd = fwd_args(**over.pop("fwd_over", {}))
    a.gate, a.gate_stride, a.gate_dtype = 0x1000, a.fwd.nheads * a.fwd.head_v_dim, abi.DN_F32
    a.weight, a.eps = 0x1000, 1e-5
    for k, v in over.items():
        setattr(a, k, v)
    assert lib.dn_chunk_fwd_out_norm(ctypes.byref(a), None) == code
    assert msg in lib.dn_last_error().decode()
    assert lib.dn_chunk_fwd_out_norm_workspace_bytes(ctypes.byref(a)) == 0


def test_chunk_fwd_out_norm_workspace_covers_the_forward():
    """The norm as its own pass needs the forward's workspace; in the scan's
    write, also the exchange words."""
    lib = abi.lib()
    f = fwd_args(batch=8, sequence=4096, nheads=16, head_k_dim=128, head_v_dim=256,
                 qkv_dtype=abi.DN_BF16, y_dtype=abi.DN_BF16)
    a = abi.ChunkFwdOutNormArgs()
    a.fwd, a.weight, a.eps = f, 0x1000, 1e-5
    fwd_ws = lib.dn_chunk_fwd_workspace_bytes(ctypes.byref(f))
    assert lib.dn_chunk_fwd_out_norm_workspace_bytes(ctypes.byref(a)) == fwd_ws
    a.in_scan = 1
    ws = lib.dn_chunk_fwd_out_norm_workspace_bytes(ctypes.byref(a))
    assert ws >= fwd_ws + 8 * 16 * (256 // 32) * 4 * 64 * 8


def test_channel_write_gates_with_a_head_decay_take_mfma_forward_generic_backward():
    """erase [.., dk] and/or write [.., dv] beside a per-head (or no) forget
    gate: the MFMA forward (per-channel kernels, head mask), the generic
    backward. No pointer is read."""
    lib = abi.lib()
    base = dict(batch=2, sequence=1000, nheads=4, head_k_dim=128, head_v_dim=128,
                qkv_dtype=abi.DN_BF16, y_dtype=abi.DN_BF16)
    for ew, ww, dw, gated in ((128, 128, 1, 1), (128, 1, 1, 1), (1, 128, 1, 1),
                              (128, 128, 0, 0)):
        over = dict(erase_width=ew, write_width=ww, decay_width=dw, has_gate=gated)
        a = fwd_args(**base, **over)
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == abi.DN_ALGO_MFMA, over
        b = bwd_args(head_v_dim=128, **over)
        assert lib.dn_chunk_bwd_algo(ctypes.byref(b)) == abi.DN_ALGO_GENERIC, over
        b.algo = abi.DN_ALGO_MFMA
        assert lib.dn_chunk_bwd_algo(ctypes.byref(b)) == -9, over


def test_mfma_paths_refuse_rows_past_32_bit_offsets():
    """The MFMA kernels address a chunk's 64 token rows with 32-bit byte
    offsets (4-byte y included): nheads·max(dk, dv) must stay below 2^23.
    Above it AUTO runs the generic kernels and an MFMA request is refused,
    rather than the offsets wrapping (no pointer is read)."""
    lib = abi.lib()
    base = dict(batch=1, sequence=64, head_k_dim=128, qkv_dtype=abi.DN_BF16,
                y_dtype=abi.DN_F32)
    for nheads, dv, auto in ((1 << 14, 256, abi.DN_ALGO_MFMA),
                             ((1 << 15) - 1, 256, abi.DN_ALGO_MFMA),
                             (1 << 15, 256, abi.DN_ALGO_GENERIC),
                             (1, 1 << 23, abi.DN_ALGO_GENERIC)):
        over = dict(nheads=nheads, head_v_dim=dv)
        for algo, want in ((abi.DN_ALGO_AUTO, auto),
                           (abi.DN_ALGO_MFMA, auto if auto == abi.DN_ALGO_MFMA else -9),
                           (abi.DN_ALGO_MFMA_FUSED,
                            abi.DN_ALGO_MFMA_FUSED if auto == abi.DN_ALGO_MFMA else -9)):
            a = fwd_args(**base, **over, algo=algo)
            assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == want, (over, algo)


def bwd_args(**over):
    a = abi.ChunkBwdArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = 8, 4096, 16, 128, 256
    a.erase_width = a.write_width = a.decay_width = 1
    a.has_gate, a.chunk_len, a.scale = 1, 64, float("nan")
    a.qkv_dtype = a.grad_dtype = abi.DN_BF16
    for f in ["d_y", "q", "k", "v", "erase", "write", "g", "state_in", "d_q", "d_k", "d_v",
              "d_erase", "d_write", "d_g", "d_state"]:
        setattr(a, f, 0x1000)
    for k, v in over.items():
        setattr(a, k, v)
    return a


@fake_pointers
def test_head_k_dim_256_forward_runs_mfma():
    """head_k_dim 256 with per-head (or no) gates and head_v_dim a multiple of
    128: the forward runs the MFMA kernels under AUTO (its scan in eight-wave
    workgroups of 128 value columns), and so does the backward with per-head
    gates; per-channel gates, other value widths and the one-kernel forward
    stay on the generic kernels there. No pointer is read."""
    lib = abi.lib()
    MFMA, GEN = abi.DN_ALGO_MFMA, abi.DN_ALGO_GENERIC
    base = dict(batch=2, sequence=1000, nheads=4, head_k_dim=256, head_v_dim=256,
                qkv_dtype=abi.DN_BF16, y_dtype=abi.DN_BF16)
    for over, auto in ((dict(), MFMA), (dict(head_v_dim=512), MFMA), (dict(has_gate=0), MFMA),
                       (dict(chunk_len=32), MFMA), (dict(head_v_dim=192), GEN),
                       (dict(head_v_dim=64), GEN), (dict(decay_width=256), GEN),
                       (dict(erase_width=256), GEN), (dict(qkv_dtype=abi.DN_F32), GEN)):
        a = fwd_args(**{**base, **over})
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == auto, over
        a = fwd_args(**{**base, **over}, algo=MFMA)
        assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == (MFMA if auto == MFMA else -9), over
    a = fwd_args(**base, algo=abi.DN_ALGO_MFMA_FUSED)
    assert lib.dn_chunk_fwd_algo(ctypes.byref(a)) == -9
    for over, auto in ((dict(), MFMA), (dict(has_gate=0), MFMA), (dict(head_v_dim=512), MFMA),
                       (dict(head_v_dim=192), GEN), (dict(erase_width=256), GEN),
                       (dict(decay_width=256), GEN)):
        b = bwd_args(**{**dict(head_k_dim=256, head_v_dim=256), **over})
        assert lib.dn_chunk_bwd_algo(ctypes.byref(b)) == auto, over
        b = bwd_args(**{**dict(head_k_dim=256, head_v_dim=256), **over}, algo=MFMA)
        assert lib.dn_chunk_bwd_algo(ctypes.byref(b)) == (MFMA if auto == MFMA else -9), over


def test_mfma_backward_needs_a_16_byte_aligned_d_y():
    """The backward's MFMA kernels read d_y in 16-byte words: an offset d_y
    view runs the generic kernels under AUTO, and an MFMA request is refused
    (no pointer is read)."""
    lib = abi.lib()
    for over, auto in ((dict(), abi.DN_ALGO_MFMA), (dict(d_y=0x1008), abi.DN_ALGO_GENERIC),
                       (dict(d_y=0x1002), abi.DN_ALGO_GENERIC), (dict(q=0x1008), abi.DN_ALGO_GENERIC)):
        assert lib.dn_chunk_bwd_algo(ctypes.byref(bwd_args(**over))) == auto, over
        a = bwd_args(**over, algo=abi.DN_ALGO_MFMA)
        want = abi.DN_ALGO_MFMA if auto == abi.DN_ALGO_MFMA else -9
        assert lib.dn_chunk_bwd_algo(ctypes.byref(a)) == want, over


@fake_pointers
def test_bwd_rejects_missing_d_g():
    lib = abi.lib()
    a = abi.ChunkBwdArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = 1, 4, 1, 4, 4
    a.erase_width = a.write_width = a.decay_width = 1
    a.has_gate, a.chunk_len, a.scale = 1, 4, float("nan")
    for f in ["d_y", "q", "k", "v", "erase", "write", "g", "state_in", "d_q", "d_k", "d_v",
              "d_erase", "d_write", "d_state"]:
        setattr(a, f, 0x1000)
    assert lib.dn_chunk_bwd(ctypes.byref(a), None) == -6
    a.algo = abi.DN_ALGO_MFMA
    a.d_g = 0x1000
    assert lib.dn_chunk_bwd_algo(ctypes.byref(a)) == -9


def test_host_mirror_sanity_mirrors_the_reference_asserts():
    """DeltaInput::sanity (path.rs:177-208) raises before any device work."""
    z = lambda *s: torch.zeros(*s)
    good = dict(q_bshk=z(1, 3, 2, 4), k_bshk=z(1, 3, 2, 4), v_bshv=z(1, 3, 2, 6),
                erase_bshK=z(1, 3, 2, 1), write_bshV=z(1, 3, 2, 1), g_bshK=None,
                state_bhkv=z(1, 2, 4, 6))
    pkg.DeltaInput(**good).sanity()
    with pytest.raises(pkg.DeltaError, match="erase gate: last axis must be 1 or 4, got 3"):
        pkg.DeltaInput(**{**good, "erase_bshK": z(1, 3, 2, 3)}).sanity()
    with pytest.raises(pkg.DeltaError, match="forget gate"):
        pkg.DeltaInput(**{**good, "g_bshK": z(1, 3, 2, 2)}).sanity()
    with pytest.raises(pkg.DeltaError, match="state"):
        pkg.DeltaInput(**{**good, "state_bhkv": z(1, 2, 6, 4)}).sanity()
    with pytest.raises(pkg.DeltaError, match="sequence length"):
        pkg.DeltaInput(**{**good, "q_bshk": z(1, 0, 2, 4)}).sanity()
    with pytest.raises(pkg.DeltaError, match="chunk_len must be at least 1"):
        pkg.DeltaInput(**good).run(pkg.DeltaPath.with_chunk_len(0))


def test_recurrent_path_applies_the_chunk_paths_dtype_and_device_rules():
    """DeltaPath::Recurrent (path.rs:215-231) through DeltaInput.delta_recurrent
    refuses what the chunk and step paths refuse, before any device work:
    tensors off the GPU (no CPU fallback) and q/k/v of different dtypes."""
    z = lambda *s, dt=torch.float32: torch.zeros(*s, dtype=dt)
    good = dict(q_bshk=z(1, 3, 2, 4), k_bshk=z(1, 3, 2, 4), v_bshv=z(1, 3, 2, 6),
                erase_bshK=z(1, 3, 2, 1), write_bshV=z(1, 3, 2, 1), g_bshK=z(1, 3, 2, 1),
                state_bhkv=z(1, 2, 4, 6))
    with pytest.raises(pkg.DeltaError, match="GPU"):
        pkg.DeltaInput(**good).run(pkg.DeltaPath.recurrent())
    mixed = {**good, "k_bshk": z(1, 3, 2, 4, dt=torch.bfloat16)}
    with pytest.raises(pkg.DeltaError, match="one dtype"):
        pkg.DeltaInput(**mixed).run(pkg.DeltaPath.recurrent())


def test_delta_path_mirrors_the_reference():
    P = pkg.DeltaPath
    assert P.default() == P.chunk() == P("chunk_recalculated")
    assert P.default().resolved_chunk_len() == 64
    assert P.recurrent().resolved_chunk_len() == 1
    assert P.with_chunk_len(16).resolved_chunk_len() == 16


def frontend_args(**over):
    a = abi.FrontendArgs()
    a.batch, a.sequence, a.nheads, a.head_k_dim, a.head_v_dim = 1, 8, 2, 4, 6
    a.n_householder, a.conv_kernel = 1, 4
    a.proj_stride = 2 * 4 + 2 * (4 + 6) + 2  # conv_dim + scalar β columns
    a.conv_activation, a.qk_activation = abi.DN_ACT_SILU, abi.DN_ACT_SILU
    a.qk_norm, a.write_gate = abi.DN_QKNORM_L2, abi.DN_WRITE_SCALAR
    a.in_dtype = a.out_dtype = abi.DN_F32
    for f in ["projected", "conv_weight", "window_in", "window_out", "q", "k", "v", "erase",
              "write"]:
        setattr(a, f, 0x1000)  # never dereferenced: every case fails its checks first
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,code,msg", [
    (dict(sequence=0), -1, "sequence length must be at least 1"),
    (dict(n_householder=0), -2, "at least 1"),
    (dict(window_in=None), -2, "convolution window presence must match"),
    (dict(conv_kernel=0), -2, "convolution window presence must match"),
    (dict(qk_norm=abi.DN_QKNORM_SUM), -9, "QkNorm::Sum"),
    (dict(head_k_dim=257, proj_stride=10 ** 5), -9, "head dims up to 256"),
    (dict(conv_kernel=9), -9, "conv_kernel up to 8"),
    (dict(proj_stride=29), -2, "narrower than the conv and write-gate columns (30)"),
    (dict(conv_activation=abi.DN_ACT_RELU), -2, "conv_activation"),
    (dict(out_dtype=5), -7, "dtype"),
    (dict(q=None), -6, "NULL"),
    (dict(write_gate=abi.DN_WRITE_CHANNEL, proj_stride=100), -2, "separate buffers"),
    # Extents past 32 bits, or products that would overflow int64, are refused.
    (dict(nheads=1 << 31, proj_stride=10 ** 5), -2, "tensor too large"),
    (dict(batch=1 << 40, sequence=1 << 40), -2, "tensor too large"),
])
@fake_pointers
def test_frontend_rejects_invalid_arguments(over, code, msg):
    """dn_frontend mirrors ShortConv's and QkvProjection's asserts
    (conv.rs:88-90, qkv.rs:397-401) and refuses what it does not offer."""
    lib = abi.lib()
    a = frontend_args(**over)
    assert lib.dn_frontend(ctypes.byref(a), None) == code
    assert msg in lib.dn_last_error().decode()


@pytest.mark.parametrize("over,code,msg", [
    (dict(tokens=0), -2, "at least 1"),
    (dict(head_v_dim=abi.OUT_NORM_MAX_HEAD_DIM + 1, gate_stride=10 ** 6), -9, "up to 1024"),
    (dict(gate_stride=15), -2, "gate_stride is narrower"),
    (dict(eps=-1.0), -2, "eps"),
    (dict(out_dtype=4), -7, "dtype"),
    (dict(weight=None), -6, "NULL"),
    (dict(nheads=1 << 31, gate_stride=1 << 40), -2, "tensor too large"),
])
@fake_pointers
def test_out_norm_rejects_invalid_arguments(over, code, msg):
    lib = abi.lib()
    a = abi.OutNormArgs()
    a.tokens, a.nheads, a.head_v_dim, a.gate_stride, a.eps = 4, 2, 8, 16, 1e-5
    a.x_dtype = a.gate_dtype = a.out_dtype = abi.DN_F32
    for f in ["x", "gate", "weight", "out"]:
        setattr(a, f, 0x1000)  # never dereferenced: every case fails its checks first
    for k, v in over.items():
        setattr(a, k, v)
    assert lib.dn_out_norm(ctypes.byref(a), None) == code
    assert msg in lib.dn_last_error().decode()


@pytest.mark.parametrize("over,code,msg", [
    (dict(size=-1), -2, "at least 0"),
    (dict(batch=-2), -2, "at least 0"),
    (dict(size=1 << 21), -2, "too large"),
    (dict(batch=1 << 62, size=64), -2, "too large"),  # the product would overflow int64
    (dict(solve=2), -9, "DN_TRI_BLOCKED or DN_TRI_NEUMANN"),
    (dict(solve=abi.DN_TRI_NEUMANN, size=abi.TRI_NEUMANN_MAX_SIZE + 1), -9, "up to 140"),
    (dict(), -6, "NULL"),
])
def test_unit_lower_inverse_rejects_invalid_arguments(over, code, msg):
    """dn_unit_lower_inverse's checks fire before any pointer is used (the
    pointers here are NULL); the square-block assert of tri.rs:74-79 is the
    mirrors' (tests/test_gpu_tri.py, tests/cpp/test_host.cpp)."""
    lib = abi.lib()
    a = abi.TriArgs()
    a.batch, a.size, a.solve = 3, 16, abi.DN_TRI_BLOCKED
    for k, v in over.items():
        setattr(a, k, v)
    assert lib.dn_unit_lower_inverse(ctypes.byref(a), None) == code
    assert msg in lib.dn_last_error().decode()


@pytest.mark.parametrize("batch,size", [(0, 16), (3, 0)])
def test_unit_lower_inverse_of_nothing_is_a_no_op(batch, size):
    a = abi.TriArgs()
    a.batch, a.size, a.solve = batch, size, abi.DN_TRI_BLOCKED
    assert abi.lib().dn_unit_lower_inverse(ctypes.byref(a), None) == 0


def test_unit_lower_inverse_mirror_checks_the_square_block():
    with pytest.raises(pkg.DeltaError, match="square trailing block"):
        pkg.unit_lower_inverse(torch.zeros(2, 3, 4))


def block_step_args(**over):
    a = abi.BlockStepArgs()
    a.batch, a.nheads, a.head_k_dim, a.head_v_dim = 2, 2, 16, 64
    a.conv_kernel, a.proj_stride = 0, 2 * 2 * 16 + 2 * 64 + 2 + 2 * 64
    a.conv_activation, a.qk_activation = abi.DN_ACT_SILU, abi.DN_ACT_SILU
    a.qk_norm, a.write_gate = abi.DN_QKNORM_L2, abi.DN_WRITE_SCALAR
    a.in_dtype = a.out_dtype = abi.DN_F32
    a.has_gate, a.decay_width, a.scale, a.eps, a.norm_gated = 1, 1, float("nan"), 1e-5, 1
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,code,msg", [
    (dict(batch=0), -2, "at least 1"),
    (dict(head_v_dim=300), -9, "up to 256"),
    (dict(head_v_dim=130), -9, "multiple of 4 above 128"),
    (dict(conv_kernel=9), -9, "conv_kernel up to 8"),
    (dict(in_dtype=3), -7, "dtype"),
    (dict(qk_norm=abi.DN_QKNORM_SUM), -9, "QkNorm::Sum"),
    (dict(write_gate=5), -2, "unknown write_gate"),
    (dict(decay_width=3), -3, "forget gate: last axis must be 1 or 16, got 3"),
    (dict(eps=-1.0), -2, "eps"),
    (dict(conv_kernel=4), -2, "window presence"),
    (dict(proj_stride=100), -2, "narrower than the conv, write-gate and norm-gate columns"),
    (dict(nheads=1 << 31), -2, "tensor too large"),
    (dict(), -6, "NULL"),
])
def test_block_step_rejects_invalid_arguments(over, code, msg):
    """dn_block_step's checks fire before any pointer is used (all NULL here):
    dn_frontend's, dn_step's and dn_out_norm's, and its own limits."""
    lib = abi.lib()
    a = block_step_args(**over)
    assert lib.dn_block_step(ctypes.byref(a), None) == code
    assert msg in lib.dn_last_error().decode()
