"""Decode kernel parity (GPU): gdn2_decode / gdn2_decode_step against the CPU
oracle's per-token loop (reference gdn2/inference.py:337-345), which is itself
pinned to the recurrence in tests/test_oracle.py.

The kernel keeps the whole recurrence in fp32, so the state is compared at
1e-5 and o at the rounding of its dtype (bf16: 2^-8 relative).
"""

from __future__ import annotations

import pytest
import torch

import oracle
from gdt2_tilelang_amd import gdn2_decode, gdn2_decode_step, gdn2_prefill
from gdt2_tilelang_amd.inference import _decode_into
from tests.helpers import device_inputs, seeded_state

pytestmark = pytest.mark.gpu
rel_err = oracle.rel_err


@pytest.mark.parametrize("n", [1, 3, 8, 16, 19])
@pytest.mark.parametrize("DK,DV", [(64, 64), (128, 128), (32, 96), (256, 64), (128, 32), (64, 160), (128, 256)])
def test_decode_matches_oracle(n, DK, DV):
    print(f"decode n={n} DK={DK} DV={DV}", flush=True)
    B, H = 2, 3
    cpu, dev = device_inputs(B, n, H, DK, DV, torch.bfloat16)
    s0 = seeded_state(B, H, DK, DV)
    st_ref = s0.clone()
    o_ref = oracle.decode_loop(*cpu, st_ref, None).float()
    st = s0.cuda()
    o = gdn2_decode(*dev, st)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and o.shape == (B, n, H, DV)
    assert rel_err(st.cpu(), st_ref) < 1e-5
    assert rel_err(o.float().cpu(), o_ref) < 4e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_decode_dtypes(dtype):
    B, n, H, DK, DV = 2, 5, 2, 64, 64
    cpu, dev = device_inputs(B, n, H, DK, DV, dtype)
    s0 = seeded_state(B, H, DK, DV)
    st_ref = s0.clone()
    o_ref = oracle.decode_loop(*cpu, st_ref, None).float()
    st = s0.cuda()
    o = gdn2_decode(*dev, st)
    torch.cuda.synchronize()
    assert o.dtype == dtype
    assert rel_err(st.cpu(), st_ref) < 1e-5
    assert rel_err(o.float().cpu(), o_ref) < (1e-5 if dtype == torch.float32 else 1e-3)


def test_decode_multi_equals_repeated_steps():
    """Holding the state on chip across n tokens == n one-token launches."""
    B, n, H, D = 2, 12, 3, 128
    _, dev = device_inputs(B, n, H, D, D, torch.bfloat16)
    s0 = seeded_state(B, H, D, D).cuda()
    st_multi = s0.clone()
    o_multi = gdn2_decode(*dev, st_multi)
    st_one = s0.clone()
    o_one = torch.cat([gdn2_decode(*(t[:, i:i + 1] for t in dev), st_one) for i in range(n)], 1)
    torch.cuda.synchronize()
    assert rel_err(st_multi, st_one) < 1e-6
    assert rel_err(o_multi.float(), o_one.float()) < 4e-3


def test_decode_step_layout():
    """gdn2_decode_step: [B, H, D] tensors, reference decode_step semantics."""
    B, H, D, T = 2, 4, 64, 8
    cpu, dev = device_inputs(B, T, H, D, D, torch.bfloat16)
    s0 = seeded_state(B, H, D, D)
    o_ref, s_ref = oracle.recurrent_gdn2(*cpu, None, s0, True)
    st = s0.cuda()
    outs = [gdn2_decode_step(*(x[:, t] for x in dev), st).float() for t in range(T)]
    torch.cuda.synchronize()
    assert rel_err(torch.stack(outs, 1).cpu(), o_ref) < 4e-3
    assert rel_err(st.cpu(), s_ref) < 1e-5


def test_decode_zero_tokens_is_noop():
    B, H, D = 2, 2, 64
    _, dev = device_inputs(B, 0, H, D, D, torch.bfloat16)
    s0 = seeded_state(B, H, D, D).cuda()
    st = s0.clone()
    o = gdn2_decode(*dev, st)
    torch.cuda.synchronize()
    assert o.shape == (B, 0, H, D)
    assert torch.equal(st, s0)


def _decode_f32_out(q, k, v, g, b, w, state):
    """gdn2_decode on bf16 tokens with an fp32 o (the C ABI's out_dtype), so the
    output is compared unrounded."""
    B, n, H, DV = v.shape
    o = torch.empty(B, n, H, DV, dtype=torch.float32, device=v.device)
    ts = [t.contiguous() for t in (q, k, v, g, b, w)]
    _decode_into(*ts, state, o, n, 0, n, q.shape[-1] ** -0.5)
    return o


@pytest.mark.parametrize("B,n,prompt", [(64, 1, 512), (32, 8, 1024)])
def test_decode_baseline_configs(B, n, prompt):
    """BASELINE configs 2 and 3 at full size: H=16, D=128, bf16 tokens, state
    from a seeded prefill; several calls in a row with fp32 o, each held to the
    2e-3 bar against the oracle loop, the state too, and (config 3) each call
    against n single-token calls."""
    print(f"decode config B={B} n={n} prompt={prompt}", flush=True)
    H, D = 16, 128
    _, pdev = device_inputs(B, prompt, H, D, D, torch.bfloat16, dist="cfg", seed=2)
    _, st = gdn2_prefill(*pdev)
    calls = 4 if n > 1 else 8
    cpu, dev = device_inputs(B, n * calls, H, D, D, torch.bfloat16, dist="cfg", seed=3)
    st_ref = st.cpu().clone()
    st_single = st.clone()
    worst = 0.0
    for c in range(calls):
        sl = slice(c * n, (c + 1) * n)
        o = _decode_f32_out(*(t[:, sl] for t in dev), st)
        o_ref = oracle.decode_loop(*(t[:, sl] for t in cpu), st_ref, None).float()
        torch.cuda.synchronize()
        e = rel_err(o.cpu(), o_ref)
        worst = max(worst, e)
        assert e < 2e-3, (c, e)
        if n > 1:
            o1 = torch.cat([_decode_f32_out(*(t[:, c * n + i:c * n + i + 1] for t in dev), st_single)
                            for i in range(n)], 1)
            assert rel_err(o, o1) < 2e-3
    torch.cuda.synchronize()
    es = rel_err(st.cpu(), st_ref)
    print(f"  worst o rel_err {worst:.2e}, state {es:.2e}", flush=True)
    assert es < 2e-3
    # the public entry (o in v.dtype) is the same result rounded to bf16
    st2 = st.clone()
    ob = gdn2_decode(*(t[:, :n] for t in dev), st2)
    o32 = _decode_f32_out(*(t[:, :n] for t in dev), st.clone())
    torch.cuda.synchronize()
    assert ob.dtype == torch.bfloat16 and torch.equal(ob, o32.to(torch.bfloat16))


@pytest.mark.parametrize("B,H,DK,DV,n", [
    (57, 13, 64, 96, 11), (40, 13, 128, 128, 8),
    (64, 8, 64, 64, 5), (128, 4, 32, 32, 3), (32, 8, 128, 256, 8), (48, 11, 128, 96, 2),
])
def test_decode_many_heads(B, H, DK, DV, n):
    """Multi-token decode over hundreds of heads (odd head counts), a partial
    column tile (DV = 96: three waves per workgroup), a second token block
    (n = 11), one-wave workgroups (DV = 32) and two column tiles per head."""
    print(f"decode many heads B={B} H={H} DK={DK} DV={DV} n={n}", flush=True)
    cpu, dev = device_inputs(B, n, H, DK, DV, torch.bfloat16)
    s0 = seeded_state(B, H, DK, DV)
    st_ref = s0.clone()
    o_ref = oracle.decode_loop(*cpu, st_ref, None).float()
    st = s0.cuda()
    o = gdn2_decode(*dev, st)
    torch.cuda.synchronize()
    assert rel_err(st.cpu(), st_ref) < 1e-5
    assert rel_err(o.float().cpu(), o_ref) < 4e-3
