"""gdn2_hip_prefill_chunks_noalloc (chunk records in the library's own
device scratch, no allocation) against gdn2_hip_prefill_chunks on a
caller-provided workspace: identical kernels on identical records, so o and
the final state must be bit-identical. Two calls in a row, the second smaller
(and at the other DK), then a call beyond the scratch, which must be rejected
before anything is launched."""

from __future__ import annotations

import pytest
import torch

from gdt2_tilelang_amd import _hip
from tests.helpers import device_inputs, seeded_state

pytestmark = pytest.mark.gpu

SCRATCH = 64 * 1024 * 1024
GDN2_ERR_SCRATCH = -3


def _run(noalloc, B, S, H, HK, DK, DV, s0, dev, out_dtype=torch.float32):
    lib = _hip.lib()
    q, k, v, g, b, w = dev
    o = torch.full((B, S, H, DV), float("nan"), dtype=out_dtype, device="cuda")
    st = torch.full((B, H, DK, DV), float("nan"), device="cuda")
    P = _hip.ptr
    common = (P(q), P(k), P(v), P(g), P(b), P(w), _hip.dtype_code(q.dtype), P(s0), P(st), P(o),
              _hip.dtype_code(out_dtype))
    shape = (B, H, HK, DK, DV, S, 0, S, DK ** -0.5, _hip.stream_of(q.device))
    if noalloc:
        rc = lib.gdn2_hip_prefill_chunks_noalloc(*common, *shape)
    else:
        ws = torch.empty(lib.gdn2_hip_prefill_workspace_bytes(B, HK, DK, S), dtype=torch.uint8, device="cuda")
        rc = lib.gdn2_hip_prefill_chunks(*common, P(ws), *shape)
    assert rc == 0, lib.gdn2_hip_status_string(rc)
    torch.cuda.synchronize()
    return o, st


def _inputs(B, S, H, HK, DK, DV, seed):
    _, dev = device_inputs(B, S, H, DK, DV, torch.bfloat16, seed=seed)
    q, k, v, g, b, w = dev
    q, k, g, b = (t[:, :, :HK].contiguous() for t in (q, k, g, b))     # grouped key heads
    return (q, k, v, g, b, w)


@pytest.mark.parametrize("B,S,H,HK,DK,DV,seed", [(2, 1000, 4, 2, 128, 128, 0), (1, 300, 3, 3, 64, 96, 1),
                                                (1, 2100, 4, 2, 128, 128, 2)])   # the last: 33 chunks of 2 key heads
def test_noalloc_prefill_equals_workspace_prefill(B, S, H, HK, DK, DV, seed):
    print(f"noalloc prefill B={B} S={S} H={H} HK={HK} DK={DK} DV={DV}", flush=True)
    dev = _inputs(B, S, H, HK, DK, DV, seed)
    s0 = seeded_state(B, H, DK, DV, seed=seed).cuda()
    o_ref, st_ref = _run(False, B, S, H, HK, DK, DV, s0, dev)
    o, st = _run(True, B, S, H, HK, DK, DV, s0, dev)
    assert torch.isfinite(o).all() and torch.isfinite(st).all()
    assert torch.equal(o, o_ref) and torch.equal(st, st_ref)


def test_noalloc_two_calls_second_smaller():
    """The scratch keeps the previous call's records; a smaller second call
    must still equal its workspace twin (it overwrites what it reads)."""
    print("noalloc two calls, second smaller", flush=True)
    big = _inputs(2, 1100, 4, 4, 128, 128, 5)
    small = _inputs(1, 130, 2, 1, 128, 64, 6)
    s_big = seeded_state(2, 4, 128, 128, seed=5).cuda()
    o1, st1 = _run(True, 2, 1100, 4, 4, 128, 128, s_big, big)
    o2, st2 = _run(True, 1, 130, 2, 1, 128, 64, None, small)
    r1, rs1 = _run(False, 2, 1100, 4, 4, 128, 128, s_big, big)
    r2, rs2 = _run(False, 1, 130, 2, 1, 128, 64, None, small)
    assert torch.equal(o1, r1) and torch.equal(st1, rs1)
    assert torch.equal(o2, r2) and torch.equal(st2, rs2)


def test_noalloc_rejects_calls_beyond_the_scratch():
    lib = _hip.lib()
    HK = 32                                  # past 16 key heads: one 64-token chunk record each
    per_chunk = lib.gdn2_hip_prefill_workspace_bytes(1, HK, 128, 64) // HK
    max_chunks = SCRATCH // per_chunk
    S_ok = (max_chunks // HK) * 64
    assert lib.gdn2_hip_prefill_workspace_bytes(1, HK, 128, S_ok) <= SCRATCH
    assert lib.gdn2_hip_prefill_workspace_bytes(1, HK, 128, S_ok + 64) > SCRATCH
    f = torch.zeros(1, device="cuda")
    P = _hip.ptr
    st = torch.full((1, HK, 128, 128), 7.0, device="cuda")
    rc = lib.gdn2_hip_prefill_chunks_noalloc(P(f), P(f), P(f), P(f), P(f), P(f), 1, None, P(st), P(f), 1,
                                            1, HK, HK, 128, 128, S_ok + 64, 0, S_ok + 64, 0.1,
                                            _hip.stream_of(f.device))
    assert rc == GDN2_ERR_SCRATCH
    assert b"scratch" in lib.gdn2_hip_status_string(rc)
    torch.cuda.synchronize()
    assert torch.all(st == 7.0)              # nothing was launched
