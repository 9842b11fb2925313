"""Host-side checks without a GPU: the C-ABI library loads and exports every
entry point include/gdn2_hip.h declares, its argument checks reject bad calls
before launching anything, and the Python API raises the reference's
exception types (reference gdn2/attention.py:44-61, :142-145;
gdn2/forward.py:740-745, :96-97, :291-295)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from gdt2_tilelang_amd import (GDN2Config, chunk_gdn2_bwd, gdn2_attention, gdn2_decode,
                               gdn2_prefill, resolve_backend)
from gdt2_tilelang_amd import _hip
from gdt2_tilelang_amd.inference import check_prefill_config
from oracle import make_inputs

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "gdn2_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(gdn2_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_hip.library_path())
    names = declared_symbols()
    assert len(names) >= 6
    for name in names:
        assert hasattr(lib, name), f"{name} declared in gdn2_hip.h but not exported"
        assert name in _hip.SIGNATURES, f"{name} has no ctypes signature"


def test_version_and_status_strings():
    lib = _hip.lib()
    assert lib.gdn2_hip_version() >= 4
    assert lib.gdn2_hip_status_string(0) == b"success"
    assert b"invalid argument" in lib.gdn2_hip_status_string(-1)
    assert b"unsupported shape" in lib.gdn2_hip_status_string(-2)


def test_workspace_size():
    lib = _hip.lib()
    # one record per (b, key head, 64-token chunk): 58112 bytes at DK=128 (factored
    # transition form: E 16 KiB, KA 16, QP 16, MOZ 8, gamma_last, scales), 41472 at DK=64
    assert lib.gdn2_hip_prefill_workspace_bytes(2, 16, 128, 4096) == 2 * 16 * 64 * 58112
    assert lib.gdn2_hip_prefill_workspace_bytes(1, 2, 128, 100) == 1 * 2 * 2 * 58112
    assert lib.gdn2_hip_prefill_workspace_bytes(2, 8, 128, 4096) == 2 * 8 * 64 * 58112
    assert lib.gdn2_hip_prefill_workspace_bytes(1, 2, 128, 2049) == 1 * 2 * 33 * 58112
    assert lib.gdn2_hip_prefill_workspace_bytes(8, 16, 128, 4096) == 8 * 16 * 64 * 58112
    assert lib.gdn2_hip_prefill_workspace_bytes(1, 2, 64, 100) == 1 * 2 * 2 * 41472
    assert lib.gdn2_hip_prefill_workspace_bytes(1, 2, 96, 64) == 0


def test_c_abi_rejects_bad_arguments_before_launch():
    """Null pointers / bad dtypes / shapes return GDN2_ERR_* without touching a device."""
    lib = _hip.lib()
    nul = None
    fake = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    assert lib.gdn2_hip_decode(nul, nul, nul, nul, nul, nul, 1, nul, nul, 1, 1, 1, 1, 128, 128, 1, 0, 1,
                               0.1, nul) == -1
    args = [fake] * 6
    assert lib.gdn2_hip_decode(*args, 7, fake, fake, 1, 1, 1, 1, 128, 128, 1, 0, 1, 0.1, nul) == -1
    assert lib.gdn2_hip_decode(*args, 1, fake, fake, 1, 1, 1, 1, 100, 128, 1, 0, 1, 0.1, nul) == -2
    assert lib.gdn2_hip_decode(*args, 1, fake, fake, 1, 1, 1, 1, 128, 100, 1, 0, 1, 0.1, nul) == -2
    assert lib.gdn2_hip_decode(*args, 1, fake, fake, 1, 1, 1, 1, 128, 128, 4, 2, 3, 0.1, nul) == -1
    # grouped heads: HK must divide H
    assert lib.gdn2_hip_decode(*args, 1, fake, fake, 1, 1, 6, 4, 128, 128, 1, 0, 1, 0.1, nul) == -1
    # a ragged token count is accepted (the last chunk is partly filled), but the
    # tokens must lie inside the allocation
    assert lib.gdn2_hip_chunk_local(fake, fake, fake, fake, 1, fake, 1, 1, 128, 100, 0, 101, 0.1,
                                    nul) == -1
    assert lib.gdn2_hip_chunk_local(fake, fake, fake, fake, 1, fake, 1, 1, 32, 64, 0, 64, 0.1,
                                    nul) == -2
    assert lib.gdn2_hip_prefill_scan(fake, fake, 1, fake, nul, fake, fake, 1, 1, 1, 1, 128, 24, 64, 0,
                                     64, nul) == -2
    assert lib.gdn2_hip_prefill_scan(fake, fake, 1, fake, nul, fake, fake, 1, 1, 4, 3, 128, 128, 64, 0,
                                     64, nul) == -1
    assert lib.gdn2_hip_prefill_chunks(*args, 1, nul, fake, fake, 1, nul, 1, 1, 1, 128, 128, 64, 0, 64,
                                       0.1, nul) == -1
    # packed sequences: offsets required, at least one sequence, the prefill shapes
    #                                   dt  cu    N  s_in s_out o  odt  ws   H  HK  DK   DV   T
    assert lib.gdn2_hip_prefill_varlen(*args, 1, nul, 2, nul, fake, fake, 1, fake, 2, 2, 128, 128, 100, 0.1,
                                       nul) == -1
    assert lib.gdn2_hip_prefill_varlen(*args, 1, fake, 0, nul, fake, fake, 1, fake, 2, 2, 128, 128, 100, 0.1,
                                       nul) == -1
    assert lib.gdn2_hip_prefill_varlen(*args, 1, fake, 2, nul, fake, fake, 1, fake, 2, 2, 32, 128, 100, 0.1,
                                       nul) == -2
    assert lib.gdn2_hip_prefill_varlen(*args, 1, fake, 2, nul, fake, fake, 1, fake, 2, 2, 128, 24, 100, 0.1,
                                       nul) == -2
    assert lib.gdn2_hip_prefill_varlen(*args, 1, fake, 2, nul, fake, fake, 1, fake, 6, 4, 128, 128, 100, 0.1,
                                       nul) == -1
    # ceil(T / 64) + nseq record slots per key head, 64-token chunk records
    assert lib.gdn2_hip_prefill_varlen_workspace_bytes(3, 2, 128, 100) == 2 * (2 + 3) * 58112
    assert lib.gdn2_hip_prefill_varlen_workspace_bytes(0, 2, 128, 100) == 0
    lds = [256] * 6
    #                                               x*6    ld*6  dt conv_w conv_b K cin  cout a_log dtb  es
    assert lib.gdn2_hip_layer_prologue_varlen(*args, *lds, 1, fake, nul, 4, nul, nul, fake, fake, 1.0,
                                              *args, nul, 2, 100, 2, 2, 64, 64, nul) == -1   # no offsets
    assert lib.gdn2_hip_layer_prologue_varlen(*args, *lds, 1, fake, nul, 4, nul, nul, fake, fake, 1.0,
                                              *args, fake, 0, 100, 2, 2, 64, 64, nul) == -1  # no sequence


def test_layer_decode_validates_every_stage_first():
    """gdn2_hip_layer_decode rejects what any of its five stages would reject
    (B*n > 8 GEMV rows, an unsupported DK, DV % 32, hidden % 8, a misaligned
    buffer) before its first launch, so a rejected call changes nothing. The
    pointers are never dereferenced: validation fails first."""
    lib = _hip.lib()
    nul = None
    f = ctypes.c_void_p(256)
    ws = ctypes.c_void_p(512)
    def call(B=1, n=1, hid=2048, H=16, HK=8, DK=128, DV=128, x=f):  # noqa: E306
        #                            x  wproj cw cb  K  cin  cout alog dtb  es   st  nw  eps  wo  out ws
        return lib.gdn2_hip_layer_decode(x, f, f, f, 4, f, ctypes.c_void_p(768), f, f, 1.0, f, f, 1e-5, f, f,
                                         ws, 1, B, n, hid, H, HK, DK, DV, 0.1, nul)
    assert call(B=3, n=3) == -2             # 9 rows > 8 (checked in long arithmetic)
    assert call(B=1 << 16, n=1 << 16) == -2
    assert call(DK=96) == -2
    assert call(DV=48) == -2
    assert call(hid=2044) == -2
    assert call(x=ctypes.c_void_p(258)) == -1


def test_backend_policy():
    assert resolve_backend("auto", on_cuda=False, needs_grad=False) == "torch"
    assert resolve_backend("auto", on_cuda=True, needs_grad=True) == "hip"
    assert resolve_backend("torch", on_cuda=True, needs_grad=False) == "torch"
    with pytest.raises(ValueError, match="requires a CUDA device"):
        resolve_backend("hip", on_cuda=False, needs_grad=False)
    # the reference's GPU backend name selects the hip kernels (gdn2/attention.py:41)
    assert resolve_backend("tilelang", on_cuda=True, needs_grad=False) == "hip"
    assert resolve_backend("tilelang", on_cuda=True, needs_grad=True) == "hip"
    with pytest.raises(ValueError, match="requires a CUDA device"):
        resolve_backend("tilelang", on_cuda=False, needs_grad=False)
    with pytest.raises(ValueError, match="unknown backend"):
        resolve_backend("triton", on_cuda=True, needs_grad=False)


def test_cpu_tensors_fail_loudly():
    ins = make_inputs(1, 64, 2, 64, 64)
    with pytest.raises(NotImplementedError, match="'hip' backend only"):
        gdn2_attention(*ins)                       # auto -> torch on CPU: not in this package
    with pytest.raises(ValueError, match="requires a CUDA device"):
        gdn2_attention(*ins, config=GDN2Config(backend="hip"))
    with pytest.raises(ValueError, match="requires a CUDA device"):
        gdn2_prefill(*ins)
    with pytest.raises(ValueError, match="requires a CUDA device"):
        gdn2_decode(*ins, torch.zeros(1, 2, 64, 64))


def test_varlen_host_validation():
    """Packed sequences: the torch backend and CPU tensors are refused as for a
    dense batch; the offsets are checked on the host before any launch."""
    from gdt2_tilelang_amd.forward import check_cu_seqlens
    ins = make_inputs(1, 128, 2, 16, 16)
    cu = torch.tensor([0, 64, 128])
    with pytest.raises(NotImplementedError, match="'hip' backend only"):
        gdn2_attention(*ins, config=GDN2Config(backend="torch"), cu_seqlens=cu)
    with pytest.raises(ValueError, match="requires a CUDA device"):
        gdn2_attention(*ins, config=GDN2Config(backend="hip"), cu_seqlens=cu)
    assert check_cu_seqlens(torch.tensor([0, 0, 5, 5, 9]), 9).tolist() == [0, 0, 5, 5, 9]
    assert check_cu_seqlens(torch.tensor([0, 7], dtype=torch.int32), 7).dtype == torch.int32
    with pytest.raises(ValueError, match="start at 0"):
        check_cu_seqlens(torch.tensor([1, 9]), 9)
    with pytest.raises(ValueError, match="end at the packed length"):
        check_cu_seqlens(torch.tensor([0, 8]), 9)
    with pytest.raises(ValueError, match="non-decreasing"):
        check_cu_seqlens(torch.tensor([0, 6, 4, 9]), 9)
    with pytest.raises(ValueError, match="1-D"):
        check_cu_seqlens(torch.tensor([0]), 0)
    with pytest.raises(TypeError, match="int32 or int64"):
        check_cu_seqlens(torch.tensor([0.0, 9.0]), 9)


def test_varlen_slot_map_is_injective():
    """The record-slot map the packed kernels use (sequence s's chunk c at
    s + floor(cu[s] / 64) + c) gives distinct slots below ceil(T / 64) + N,
    checked by brute force over random offsets (empty and ragged sequences)."""
    g = torch.Generator().manual_seed(7)
    for _ in range(200):
        N = int(torch.randint(1, 12, (1,), generator=g))
        lens = torch.randint(0, 200, (N,), generator=g) * (torch.rand(N, generator=g) > 0.2)
        cu = [0] + torch.cumsum(lens, 0).tolist()
        T = cu[-1]
        slots = [s + cu[s] // 64 + c for s in range(N) for c in range(-(-(cu[s + 1] - cu[s]) // 64))]
        assert len(set(slots)) == len(slots)
        assert all(0 <= x < -(-T // 64) + N for x in slots)
        # slot -> sequence: the last s with s + cu[s] // 64 <= slot
        for x in slots:
            s = max(i for i in range(N) if i + cu[i] // 64 <= x)
            c = x - s - cu[s] // 64
            assert 0 <= c * 64 < cu[s + 1] - cu[s]


def test_tiling_and_dtype_validation():
    with pytest.raises(ValueError, match="power of two"):
        check_prefill_config(GDN2Config(chunk_size=48))
    with pytest.raises(ValueError, match="divisible"):
        check_prefill_config(GDN2Config(chunk_size=64, sub_chunk_size=24))
    with pytest.raises(ValueError, match="at least 2 sub-chunks"):
        check_prefill_config(GDN2Config(chunk_size=64, sub_chunk_size=64))
    with pytest.raises(ValueError, match="chunk_size 64"):
        check_prefill_config(GDN2Config(chunk_size=128))
    with pytest.raises(TypeError, match="state dtype"):
        check_prefill_config(GDN2Config(state_dtype=torch.int32))
    check_prefill_config(GDN2Config(state_dtype=torch.bfloat16))
    check_prefill_config(GDN2Config(chunk_size=64, sub_chunk_size=32))
    with pytest.raises(TypeError, match="unsupported dtype"):
        _hip.dtype_code(torch.int32)


def test_backward_host_validation():
    """chunk_gdn2_bwd checks its device on the host; the C ABI rejects unsupported
    head dims, bad dtypes, null pointers and misaligned workspaces before any
    launch, and sizes no workspace for an unsupported shape."""
    lib = _hip.lib()
    with pytest.raises(ValueError, match="CUDA"):
        x = torch.zeros(1, 4, 2, 64)
        chunk_gdn2_bwd(x, x, x, x, x, x, None, None, x, None)
    assert lib.gdn2_hip_prefill_workspace_bytes(1, 2, 96, 64) == 0
    wsb = lib.gdn2_hip_backward_workspace_bytes
    assert wsb(1, 2, 2, 48, 64, 128) == 0          # DK not in (32, 64, 128)
    assert wsb(1, 2, 2, 64, 24, 128) == 0          # DV % 16
    assert wsb(1, 3, 2, 64, 64, 128) == 0          # HK must divide H
    # B=2 H=4 HK=2 DK=64 DV=32 S=100 (2 chunks): records of B*HK*NC chunks (A,
    # KA, QP, Ai, Aqk, gamma padded to 64, A^T, QP^T), two state checkpoints
    # B*H*NC*DK*DV floats each, four gradient shares B*S*H*DK
    rec = 2 * 2 * 2 * (64 * 64 + 64 * 64 + 64 * 64 + 4096 + 4096 + 64 + 64 * 64 + 64 * 64) * 4
    gs = 2 * 4 * 2 * (3 * 64 * 64 + 2 * 4096 + 64) * 4   # per (b, value head, chunk) sums of the gradient kernel
    ck = 2 * 4 * 2 * 64 * 32 * 4
    part = 4 * 2 * 100 * 4 * 64 * 4
    up = lambda x: (x + 255) // 256 * 256
    wide = up(2 * 100 * 4 * 32 * 4)   # an fp32 copy of do (a 16-bit do of another dtype than the inputs)
    assert wsb(2, 4, 2, 64, 32, 100) == up(rec) + 2 * up(ck) + up(part) + up(gs) + wide
    # one value head per key head: the pairwise pass writes the outputs, no gradient shares
    rec1 = 2 * 4 * 2 * (64 * 64 + 64 * 64 + 64 * 64 + 4096 + 4096 + 64 + 64 * 64 + 64 * 64) * 4
    assert wsb(2, 4, 4, 64, 32, 100) == up(rec1) + 2 * up(ck) + up(gs) + wide
    fake = ctypes.c_void_p(256)   # never dereferenced: validation fails first
    args = [fake] * 6
    tail = [fake] * 8
    call = lambda dt, dk, dv, ws=fake, ptrs=args: lib.gdn2_hip_backward(
        *ptrs, dt, 0.1, None, fake, 1, None, *tail[:3], fake, fake, fake, None, ws, 1, 64, 2, 2, dk, dv, None)
    assert call(7, 64, 64) == -1
    assert call(1, 48, 64) == -2
    assert call(1, 64, 24) == -2
    assert call(1, 64, 64, ws=ctypes.c_void_p(264)) == -1
    assert call(1, 64, 64, ptrs=[None] + args[1:]) == -1


def test_backward_varlen_host_validation():
    """gdn2_hip_backward_varlen: the workspace size is the dense formula with
    ceil(T/64) + nseq chunk slots, and bad arguments are refused before any
    launch (no GPU needed)."""
    lib = _hip.lib()
    wsv = lib.gdn2_hip_backward_varlen_workspace_bytes
    wsb = lib.gdn2_hip_backward_workspace_bytes
    up = lambda x: (x + 255) // 256 * 256
    assert wsv(0, 2, 2, 64, 64, 100) == 0            # nseq >= 1
    assert wsv(3, 2, 2, 48, 64, 100) == 0            # DK not in (32, 64, 128)
    assert wsv(3, 3, 2, 64, 64, 100) == 0            # HK must divide H
    # T = 100, 3 sequences: 2 + 3 = 5 slots per head, against 2 chunks for a dense row
    H, HK, DK, DV, T, N = 4, 2, 64, 32, 100, 3
    rec = HK * 5 * (64 * 64 + 64 * 64 + 64 * 64 + 4096 + 4096 + 64 + 64 * 64 + 64 * 64) * 4
    ck = H * 5 * DK * DV * 4
    part = 4 * T * H * DK * 4
    gs = H * 5 * (3 * 64 * DK + 2 * 4096 + DK) * 4
    wide = up(T * H * DV * 4)
    assert wsv(N, H, HK, DK, DV, T) == up(rec) + 2 * up(ck) + up(part) + up(gs) + wide
    assert wsv(N, H, HK, DK, DV, T) > wsb(1, H, HK, DK, DV, T)
    fake = ctypes.c_void_p(256)   # never dereferenced: validation fails first
    call = lambda dt, dk, cu=fake, ws=fake, nseq=N: lib.gdn2_hip_backward_varlen(
        *([fake] * 6), dt, 0.1, None, fake, 1, None, *([fake] * 6), None, ws, cu, nseq, T, H, HK, dk, DV, None)
    assert call(7, 64) == -1                  # dtype
    assert call(1, 48) == -2                  # DK
    assert call(1, 64, cu=None) == -1         # offsets missing
    assert call(1, 64, nseq=0) == -1
    assert call(1, 64, ws=ctypes.c_void_p(264)) == -1   # workspace alignment
