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
    assert lib.gdn2_hip_version() >= 2
    assert lib.gdn2_hip_status_string(0) == b"success"
    assert b"invalid argument" in lib.gdn2_hip_status_string(-1)
    assert b"unsupported shape" in lib.gdn2_hip_status_string(-2)


def test_workspace_size():
    lib = _hip.lib()
    # one record per (b, key head, 64-token chunk); 66304 bytes at DK=128, 41472 at DK=64
    assert lib.gdn2_hip_prefill_workspace_bytes(2, 16, 128, 4096) == 2 * 16 * 64 * 66304
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


def test_backend_policy():
    assert resolve_backend("auto", on_cuda=False, needs_grad=False) == "torch"
    assert resolve_backend("auto", on_cuda=True, needs_grad=True) == "hip"
    assert resolve_backend("torch", on_cuda=True, needs_grad=False) == "torch"
    with pytest.raises(ValueError, match="requires a CUDA device"):
        resolve_backend("hip", on_cuda=False, needs_grad=False)
    with pytest.raises(ValueError, match="unknown backend"):
        resolve_backend("tilelang", on_cuda=True, needs_grad=False)


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


def test_varlen_is_rejected():
    ins = make_inputs(1, 128, 2, 16, 16)
    with pytest.raises(NotImplementedError, match="variable-length"):
        gdn2_attention(*ins, config=GDN2Config(backend="torch"), cu_seqlens=torch.tensor([0, 64, 128]))


def test_tiling_and_dtype_validation():
    with pytest.raises(ValueError, match="power of two"):
        check_prefill_config(GDN2Config(chunk_size=48))
    with pytest.raises(ValueError, match="divisible"):
        check_prefill_config(GDN2Config(chunk_size=64, sub_chunk_size=24))
    with pytest.raises(ValueError, match="at least 2 sub-chunks"):
        check_prefill_config(GDN2Config(chunk_size=64, sub_chunk_size=64))
    with pytest.raises(ValueError, match="chunk_size 64"):
        check_prefill_config(GDN2Config(chunk_size=128))
    with pytest.raises(TypeError, match="fp32 state"):
        check_prefill_config(GDN2Config(state_dtype=torch.bfloat16))
    check_prefill_config(GDN2Config(chunk_size=64, sub_chunk_size=32))
    with pytest.raises(TypeError, match="unsupported dtype"):
        _hip.dtype_code(torch.int32)


def test_backward_is_not_provided():
    with pytest.raises(NotImplementedError, match="forward-only"):
        chunk_gdn2_bwd()
