"""Packed variable-length prefill (GPU): N sequences concatenated in one
``[1, T, H, D]`` row with ``cu_seqlens`` offsets, each its own recurrence.

The reference rejects packed batches (gdn2/attention.py:142-145); its
semantics here are those of the packed-batch convention it names: sequence i
equals a separate call on its own tokens from ``initial_state[i]``. So every
sequence is checked against the CPU oracle's prefill on its slice (same 2e-3
bar as the dense prefill), against a separate dense call, and, for thousands
of short sequences (all rounds of the kernels' slot -> sequence search),
against a zero-padded dense batch, whose padding is inert (g = 0, b = w = 0).
"""

from __future__ import annotations

import pytest
import torch

import oracle
from gdt2_tilelang_amd import GDN2Config, chunk_gdn2_fwd, gdn2_attention
from tests.helpers import device_inputs, seeded_state

pytestmark = pytest.mark.gpu
rel_err = oracle.rel_err
TOL = 2e-3
F32 = GDN2Config(output_dtype=torch.float32)


def _grouped(cpu, dev, HK):
    cpu = (cpu[0][:, :, :HK], cpu[1][:, :, :HK], cpu[2], cpu[3][:, :, :HK], cpu[4][:, :, :HK], cpu[5])
    dev = tuple(t.contiguous() for t in (dev[0][:, :, :HK], dev[1][:, :, :HK], dev[2], dev[3][:, :, :HK],
                                         dev[4][:, :, :HK], dev[5]))
    return cpu, dev


def _packed(lens, H, HK, DK, DV, dtype=torch.bfloat16, seed=0):
    T = sum(lens)
    cpu, dev = device_inputs(1, T, H, DK, DV, dtype, seed=seed)
    cpu, dev = _grouped(cpu, dev, HK)
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32)
    return cpu, dev, cu


@pytest.mark.parametrize("DK,H,HK", [(128, 4, 4), (64, 4, 2), (128, 6, 3)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_varlen_matches_oracle(DK, H, HK, dtype):
    lens = [0, 1, 63, 64, 65, 200, 0, 130, 7]
    DV = 128 if DK == 128 else 96
    print(f"varlen lens={lens} DK={DK} DV={DV} H={H} HK={HK} {dtype}", flush=True)
    cpu, dev, cu = _packed(lens, H, HK, DK, DV, dtype)
    N = len(lens)
    s0 = seeded_state(N, H, DK, DV)
    s0_dev = s0.cuda()
    o, st = gdn2_attention(*dev, initial_state=s0_dev, output_final_state=True, config=F32,
                           cu_seqlens=cu.cuda())
    torch.cuda.synchronize()
    assert o.shape == (1, sum(lens), H, DV) and st.shape == (N, H, DK, DV)
    assert torch.equal(s0_dev.cpu(), s0)               # initial_state is never modified
    rep = H // HK
    exp = lambda t: t.repeat_interleave(rep, dim=2)
    o_ref = torch.zeros(1, sum(lens), H, DV)
    s_ref = s0.clone()
    for i in range(N):
        a, e = int(cu[i]), int(cu[i + 1])
        if e == a:
            continue
        sl = [t[:, a:e] for t in cpu]
        oi, si = oracle.prefill(exp(sl[0]), exp(sl[1]), sl[2], exp(sl[3]), exp(sl[4]), sl[5], s0[i:i + 1].clone())
        o_ref[:, a:e] = oi
        s_ref[i] = si[0]
    eo, es = rel_err(o.cpu(), o_ref), rel_err(st.cpu(), s_ref)
    print(f"  rel_err o={eo:.2e} state={es:.2e}", flush=True)
    assert eo < TOL and es < TOL
    for i in (0, 6):                                   # empty sequences pass their state through
        assert torch.equal(st[i].cpu(), s0[i])


def test_varlen_equals_separate_calls():
    """Each packed sequence equals a dense call on its tokens alone, bit for
    bit: both sides run the same chunk-local and scan kernels on the same
    64-token chunk records, with each sequence's chunks starting at its own
    first token."""
    lens = [150, 3, 64, 0, 257, 40]
    H, HK, DK, DV = 4, 2, 128, 128
    print(f"varlen vs separate lens={lens}", flush=True)
    _, dev, cu = _packed(lens, H, HK, DK, DV, seed=5)
    N = len(lens)
    s0 = seeded_state(N, H, DK, DV, seed=3).cuda()
    o, st = gdn2_attention(*dev, initial_state=s0, output_final_state=True, config=F32, cu_seqlens=cu)
    for i in range(N):
        a, e = int(cu[i]), int(cu[i + 1])
        if e == a:
            assert torch.equal(st[i], s0[i])
            continue
        oi, si = gdn2_attention(*(t[:, a:e] for t in dev), initial_state=s0[i:i + 1],
                                output_final_state=True, config=F32)
        assert torch.equal(o[:, a:e], oi), i
        assert torch.equal(st[i:i + 1], si), i
    torch.cuda.synchronize()


def test_varlen_long_sequence():
    """A sequence of 33 chunks (a ragged last one) between two short ones,
    packed, against a dense call on its tokens (bit for bit) and against the
    oracle (2e-3)."""
    lens = [5, 2100, 70]
    H, HK, DK, DV = 4, 2, 128, 128
    print(f"varlen long sequence lens={lens}", flush=True)
    cpu, dev, cu = _packed(lens, H, HK, DK, DV, seed=8)
    s0 = seeded_state(len(lens), H, DK, DV, seed=4)
    o, st = gdn2_attention(*dev, initial_state=s0.cuda(), output_final_state=True, config=F32, cu_seqlens=cu)
    a, e = int(cu[1]), int(cu[2])
    oi, si = gdn2_attention(*(t[:, a:e] for t in dev), initial_state=s0[1:2].cuda(), output_final_state=True,
                            config=F32)
    torch.cuda.synchronize()
    assert torch.equal(o[:, a:e], oi) and torch.equal(st[1:2], si)
    rep = H // HK
    exp = lambda t: t.repeat_interleave(rep, dim=2)
    sl = [t[:, a:e] for t in cpu]
    o_ref, s_ref = oracle.prefill(exp(sl[0]), exp(sl[1]), sl[2], exp(sl[3]), exp(sl[4]), sl[5], s0[1:2].clone())
    assert rel_err(o[:, a:e].cpu(), o_ref) < TOL and rel_err(st[1:2].cpu(), s_ref) < TOL


def test_varlen_no_initial_state_and_no_final():
    lens = [70, 0, 33]
    H, DK, DV = 2, 64, 64
    cpu, dev, cu = _packed(lens, H, H, DK, DV, seed=9)
    o, st = gdn2_attention(*dev, config=F32, cu_seqlens=cu)
    assert st is None
    o2, st2 = gdn2_attention(*dev, output_final_state=True, config=F32, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    assert torch.count_nonzero(st2[1]) == 0            # empty sequence, no initial state: zeros
    o_ref, s_ref = oracle.prefill(*(t[:, 70:] for t in cpu), None)
    assert rel_err(o[:, 70:].cpu(), o_ref) < TOL and rel_err(st2[2:].cpu(), s_ref) < TOL


def test_varlen_all_empty():
    H, DK, DV = 2, 64, 64
    _, dev, cu = _packed([0, 0, 0], H, H, DK, DV)
    s0 = seeded_state(3, H, DK, DV).cuda()
    o, st = gdn2_attention(*dev, initial_state=s0, output_final_state=True, config=F32, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert o.shape == (1, 0, H, DV) and torch.equal(st, s0)


@pytest.mark.parametrize("N", [100, 5000])
def test_varlen_many_short_sequences(N):
    """Thousands of short sequences (N = 5000 takes three rounds of the
    64-way slot search) against a zero-padded dense batch, and the first
    sequences against the oracle."""
    gen = torch.Generator().manual_seed(N)
    lens = (torch.randint(1, 41, (N,), generator=gen) * (torch.rand(N, generator=gen) > 0.25)).tolist()
    H, DK, DV = 2, 64, 64
    Lmax = max(lens)
    print(f"varlen many N={N} T={sum(lens)} Lmax={Lmax}", flush=True)
    cpu, dev, cu = _packed(lens, H, H, DK, DV, seed=N)
    s0 = seeded_state(N, H, DK, DV, seed=2).cuda()
    o, st = gdn2_attention(*dev, initial_state=s0, output_final_state=True, config=F32, cu_seqlens=cu)
    # the same tokens as a padded [N, Lmax] batch
    idx_b = torch.repeat_interleave(torch.arange(N), torch.tensor(lens))
    idx_t = torch.cat([torch.arange(n) for n in lens])
    padded = []
    for t in dev:
        p = t.new_zeros(N, Lmax, *t.shape[2:])
        p[idx_b.cuda(), idx_t.cuda()] = t[0]
        padded.append(p)
    op, sp = chunk_gdn2_fwd(*padded, DK ** -0.5, s0, True, F32)
    torch.cuda.synchronize()
    assert rel_err(st, sp) < 1e-5
    assert rel_err(o[0], op[idx_b.cuda(), idx_t.cuda()]) < 1e-5
    for i in range(8):
        a, e = int(cu[i]), int(cu[i + 1])
        if e == a:
            assert torch.equal(st[i], s0[i])
            continue
        oi, si = oracle.prefill(*(t[:, a:e] for t in cpu), s0[i:i + 1].cpu().clone())
        assert rel_err(o[:, a:e].cpu(), oi) < TOL and rel_err(st[i:i + 1].cpu(), si) < TOL
