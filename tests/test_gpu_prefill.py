"""Prefill / chunkwise-forward parity (GPU) against the CPU oracle.

The bar: o and the final state within 2e-3 max-abs
error relative to the fp32 reference, `rel_err = max|a - ref| / max|ref|`
(reference tests/test_gdn2.py:38-39). o is compared in fp32
(`GDN2Config(output_dtype=torch.float32)`) because rounding o to bf16 alone
can cost up to 2^-8 relative; the bf16-output path is checked to be the fp32
result rounded. Inputs are rounded to the kernel dtype before the oracle sees
them, so input quantisation is not counted as error.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle
from gdt2_tilelang_amd import GDN2Config, chunk_gdn2_fwd, gdn2_attention, gdn2_decode, gdn2_prefill
from tests.golden.make_golden import config0_inputs
from tests.helpers import device_inputs, seeded_state

pytestmark = pytest.mark.gpu
rel_err = oracle.rel_err


TOL = 2e-3
F32 = GDN2Config(output_dtype=torch.float32)
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "config0.npz")


def _check(B, S, H, DK, DV, dtype=torch.bfloat16, decay_scale=4.0, dist="ref", with_state=True, seed=0):
    print(f"prefill B={B} S={S} H={H} DK={DK} DV={DV} {dtype} decay={decay_scale} {dist}", flush=True)
    cpu, dev = device_inputs(B, S, H, DK, DV, dtype, decay_scale=decay_scale, seed=seed, dist=dist)
    s0 = seeded_state(B, H, DK, DV) if with_state else None
    o_ref, s_ref = oracle.prefill(*cpu, None if s0 is None else s0.clone())
    o, st = gdn2_prefill(*dev, None if s0 is None else s0.cuda(), config=F32)
    torch.cuda.synchronize()
    assert o.shape == (B, S, H, DV) and o.dtype == torch.float32
    eo, es = rel_err(o.cpu(), o_ref), rel_err(st.cpu(), s_ref)
    print(f"  rel_err o={eo:.2e} state={es:.2e}", flush=True)
    assert eo < TOL and es < TOL
    return dev, o, st


@pytest.mark.parametrize("B,S,H,DK,DV", [
    (2, 512, 4, 64, 64), (1, 1024, 8, 128, 128), (2, 320, 2, 64, 128),
    (2, 1000, 4, 64, 64), (1, 100, 2, 128, 64), (1, 7, 2, 64, 64), (3, 192, 2, 128, 96),
])
def test_prefill_matches_oracle(B, S, H, DK, DV):
    _check(B, S, H, DK, DV)


@pytest.mark.parametrize("B,H,DK,DV,dtype", [
    (1, 66, 128, 128, torch.bfloat16), (1, 66, 128, 128, torch.float32), (1, 88, 128, 96, torch.bfloat16),
    (2, 34, 64, 128, torch.bfloat16), (1, 130, 64, 64, torch.bfloat16)])
def test_prefill_several_value_tiles_per_workgroup(B, H, DK, DV, dtype):
    """Many heads (B*H*DV/16 > 512 value tiles): at DK = 64 the scan gives
    each workgroup two 16-column tiles; at DK = 128 more tiles than the GPU
    holds at once, so workgroups run in several rounds. The bf16 output of the
    DK = 128 scan is its fp32 output rounded (the same arithmetic up to the
    store)."""
    assert B * H * DV // 16 > 512
    dev, o, st = _check(B, 192, H, DK, DV, dtype=dtype, seed=3)
    if DK == 128:
        ob, sb = gdn2_prefill(*dev, seeded_state(B, H, DK, DV).cuda(), config=GDN2Config(output_dtype=torch.bfloat16))
        torch.cuda.synchronize()
        assert ob.dtype == torch.bfloat16
        assert torch.equal(ob, o.to(torch.bfloat16)) and torch.equal(sb, st)


@pytest.mark.parametrize("decay_scale,DV,dtype", [
    (0.3, 128, torch.bfloat16), (4.0, 128, torch.bfloat16), (30.0, 128, torch.bfloat16),
    (4.0, 64, torch.float32), (1.0, 32, torch.float16)])
def test_prefill_long_ragged(decay_scale, DV, dtype):
    """A long call of few key heads: 33 chunks with a ragged last chunk of 52
    rows, across the decay regimes of the chunk-local stage and value widths
    of one to eight 16-column scan tiles."""
    _check(1, 2100, 2, 128, DV, dtype=dtype, decay_scale=decay_scale, seed=7)


@pytest.mark.parametrize("decay_scale", [0.0, 1.0, 8.0, 30.0])
def test_prefill_decay_scales(decay_scale):
    """Covers both block-rescaling paths: 8 and 30 force the exact path
    (a channel losing > 83 nats in 16 tokens) and must not overflow."""
    _, o, _ = _check(1, 256, 2, 128, 128, decay_scale=decay_scale)
    assert torch.isfinite(o).all()


@pytest.mark.parametrize("DK", [64, 128])
def test_prefill_long_memory(DK):
    """No decay at all (g = 0): the state is never forgotten, Un = U - W S is a
    small difference of large terms, and rounding errors accumulate over the
    whole prompt. The split-operand plan must still hold 2e-3 over 4096 tokens."""
    _check(1, 4096, 2, DK, 128, decay_scale=0.0, with_state=False)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("DK", [64, 128])
def test_prefill_input_dtypes(dtype, DK):
    _check(2, 256, 2, DK, 64, dtype=dtype)


def test_prefill_no_initial_state():
    _check(2, 384, 3, 128, 128, with_state=False)


def test_prefill_bf16_output_is_rounded_fp32():
    B, S, H, D = 2, 512, 4, 128
    _, dev = device_inputs(B, S, H, D, D, torch.bfloat16)
    o32, s32 = gdn2_prefill(*dev, config=F32)
    o16, s16 = gdn2_prefill(*dev)
    torch.cuda.synchronize()
    assert o16.dtype == torch.bfloat16
    assert torch.equal(s32, s16)
    assert ((o16.float() - o32).abs() <= o32.abs() * 2 ** -8 + 1e-30).all()


def test_segmented_prefill_equals_one_pass():
    """reference tests/test_inference.py:135-150, on the GPU kernels."""
    B, S, H, D = 2, 448, 3, 64
    _, dev = device_inputs(B, S, H, D, D, torch.bfloat16)
    o_all, s_all = gdn2_prefill(*dev, config=F32)
    outs, st = [], None
    for lo, hi in ((0, 64), (64, 160), (160, 197), (197, 448)):
        o, st = gdn2_prefill(*(t[:, lo:hi] for t in dev), st, config=F32)
        outs.append(o)
    torch.cuda.synchronize()
    assert rel_err(torch.cat(outs, 1), o_all) < TOL
    assert rel_err(st, s_all) < TOL


def test_prefill_baseline_config1():
    """B=2 S=4096 H=16 DK=DV=128, bf16 inputs, fp32 g,
    q,k L2-normalised, g = logsigmoid(N(0,1)), b,w = sigmoid(N(0,1))."""
    _check(2, 4096, 16, 128, 128, dist="cfg", with_state=False)


def test_gdn2_attention_and_chunk_fwd():
    """Functional op: zero-padding of a ragged length is inert; initial_state
    is read, not written; final state only on request."""
    B, S, H, D = 2, 200, 2, 64
    cpu, dev = device_inputs(B, S, H, D, D, torch.bfloat16)
    s0 = seeded_state(B, H, D, D)
    o_ref, s_ref = oracle.recurrent_gdn2(*cpu, None, s0, True)
    s0d = s0.cuda()
    o, st = gdn2_attention(*dev, initial_state=s0d, output_final_state=True, config=F32)
    o2, none = chunk_gdn2_fwd(*dev, D ** -0.5, s0d, False, F32)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(s0d.cpu(), s0)
    assert rel_err(o.cpu(), o_ref) < TOL and rel_err(st.cpu(), s_ref) < TOL
    assert torch.equal(o, o2)
    o16, _ = gdn2_attention(*dev)
    assert o16.dtype == torch.bfloat16 and o16.shape == (B, S, H, D)


@pytest.mark.parametrize("DK,H,HK", [(128, 8, 4), (64, 6, 2), (128, 4, 1), (128, 72, 8)])
def test_grouped_heads_equal_repeated(DK, H, HK):
    """q, k, b, g on HK key heads with v, w on H value heads must give exactly
    what the reference's repeat_interleave expansion gives (attention.py:
    295-297): prefill (whole chunks + ragged tail) and a following decode."""
    from gdt2_tilelang_amd import gdn2_decode

    print(f"grouped heads DK={DK} H={H} HK={HK}", flush=True)
    B, S, n = 2, 200, 5
    _, kd = device_inputs(B, S + n, HK, DK, DK, torch.bfloat16, decay_scale=1.0, seed=5)
    _, vd = device_inputs(B, S + n, H, DK, DK, torch.bfloat16, decay_scale=1.0, seed=6)
    q, k, _, g, b, _ = kd
    v, w = vd[2], vd[5]
    rep = H // HK
    qe, ke, ge, be = (t.repeat_interleave(rep, dim=2) for t in (q, k, g, b))
    s0 = seeded_state(B, H, DK, DK).cuda()
    o1, s1 = gdn2_prefill(q[:, :S], k[:, :S], v[:, :S], g[:, :S], b[:, :S], w[:, :S], s0.clone(), config=F32)
    o2, s2 = gdn2_prefill(qe[:, :S], ke[:, :S], v[:, :S], ge[:, :S], be[:, :S], w[:, :S], s0.clone(),
                          config=F32)
    d1 = gdn2_decode(q[:, S:], k[:, S:], v[:, S:], g[:, S:], b[:, S:], w[:, S:], s1)
    d2 = gdn2_decode(qe[:, S:], ke[:, S:], v[:, S:], ge[:, S:], be[:, S:], w[:, S:], s2)
    torch.cuda.synchronize()
    # the grouped form reads each key head's inputs and record in place of
    # their copies: the same kernels on the same values, bit for bit
    assert torch.equal(o1, o2) and torch.equal(s1, s2) and torch.equal(d1, d2)


@pytest.mark.parametrize("DK,DV,B,S_alloc,t0,n", [
    (64, 64, 2, 230, 10, 150), (128, 64, 2, 230, 10, 150), (128, 16, 2, 230, 10, 150), (64, 48, 2, 230, 10, 150),
    (128, 128, 1, 2200, 37, 2100)])   # the last 33 chunks of 2 key heads
def test_c_abi_ragged_window(DK, DV, B, S_alloc, t0, n):
    """The C ABI on a window [t0, t0 + n) of a larger allocation with n not a
    chunk multiple: the last chunk's missing rows are read as zeros, o rows
    outside the window are left alone, and the result equals the recurrence on
    the window alone. DV 16 and 48: value widths the C ABI takes (multiples of
    16) below the Python API's multiples of 32."""
    from gdt2_tilelang_amd import _hip

    H = 2
    print(f"ragged window DK={DK} DV={DV} t0={t0} n={n} s_alloc={S_alloc}", flush=True)
    cpu, dev = device_inputs(B, S_alloc, H, DK, DV, torch.bfloat16)
    s0 = seeded_state(B, H, DK, DV)
    win = tuple(t[:, t0:t0 + n] for t in cpu)
    o_ref, s_ref = oracle.recurrent_gdn2(*win, None, s0.clone(), True)
    q, k, v, g, b, w = dev
    lib = _hip.lib()
    ws = torch.empty(lib.gdn2_hip_prefill_workspace_bytes(B, H, DK, n), dtype=torch.uint8, device="cuda")
    o = torch.full((B, S_alloc, H, DV), 7.0, device="cuda")
    s_in, s_out = s0.cuda(), torch.empty(B, H, DK, DV, device="cuda")
    P = _hip.ptr
    _hip.check(lib.gdn2_hip_prefill_chunks(P(q), P(k), P(v), P(g), P(b), P(w), _hip.dtype_code(q.dtype),
                                           P(s_in), P(s_out), P(o), 0, P(ws), B, H, H, DK, DV, S_alloc,
                                           t0, n, DK ** -0.5, _hip.stream_of(q.device)), "prefill_chunks")
    torch.cuda.synchronize()
    oc = o.cpu()
    assert (oc[:, :t0] == 7.0).all() and (oc[:, t0 + n:] == 7.0).all()
    eo, es = rel_err(oc[:, t0:t0 + n], o_ref), rel_err(s_out.cpu(), s_ref)
    print(f"  rel_err o={eo:.2e} state={es:.2e}", flush=True)
    assert eo < TOL and es < TOL


def test_prefill_random_shapes():
    """Seeded random shapes against the oracle: ragged lengths (including under
    one chunk), grouped heads, DK 64 / 128, DV from 32 to 256, three input
    dtypes, with and without an initial state."""
    gen = torch.Generator().manual_seed(1234)

    def pick(xs):
        return xs[int(torch.randint(len(xs), (1,), generator=gen))]

    for case in range(14):
        B = pick([1, 2, 3])
        S = int(torch.randint(1, 700, (1,), generator=gen))
        HK = pick([1, 2, 3])
        H = HK * pick([1, 2])
        DK = pick([64, 128])
        DV = pick([32, 64, 96, 128, 160, 256])
        dtype = pick([torch.bfloat16, torch.float16, torch.float32])
        with_state = bool(torch.randint(2, (1,), generator=gen))
        print(f"case {case}: B={B} S={S} H={H} HK={HK} DK={DK} DV={DV} {dtype} state={with_state}", flush=True)
        cpu, dev = device_inputs(B, S, H, DK, DV, dtype, seed=case)
        # grouped heads: the key-side tensors keep the first HK heads
        cpu = (cpu[0][:, :, :HK], cpu[1][:, :, :HK], cpu[2], cpu[3][:, :, :HK], cpu[4][:, :, :HK], cpu[5])
        dev = tuple(t.contiguous() for t in (dev[0][:, :, :HK], dev[1][:, :, :HK], dev[2], dev[3][:, :, :HK],
                                             dev[4][:, :, :HK], dev[5]))
        rep = H // HK
        exp = lambda t: t.repeat_interleave(rep, dim=2)
        s0 = seeded_state(B, H, DK, DV, seed=case) if with_state else None
        o_ref, s_ref = oracle.prefill(exp(cpu[0]), exp(cpu[1]), cpu[2], exp(cpu[3]), exp(cpu[4]), cpu[5],
                                      None if s0 is None else s0.clone())
        o, st = gdn2_prefill(*dev, None if s0 is None else s0.cuda(), config=F32)
        torch.cuda.synchronize()
        eo, es = rel_err(o.cpu(), o_ref), rel_err(st.cpu(), s_ref)
        print(f"  rel_err o={eo:.2e} state={es:.2e}", flush=True)
        assert eo < TOL and es < TOL


def test_config0_golden_on_hip():
    """BASELINE config 0 (B=1 S=256 H=2 D=64, fp32 inputs, logsigmoid decay,
    seed 0) through the public op and prefill on the GPU, against the float64
    golden vectors of tests/golden/config0.npz (independent numpy recurrence)."""
    print("config 0 golden: gdn2_attention + gdn2_prefill, fp32", flush=True)
    ref = np.load(GOLDEN)
    o_ref, s_ref = torch.from_numpy(ref["o"]).float(), torch.from_numpy(ref["S"]).float()
    dev = [t.cuda() for t in config0_inputs()]
    assert all(t.dtype == torch.float32 for t in dev)
    o1, s1 = gdn2_attention(*dev, output_final_state=True)
    o2, s2 = gdn2_prefill(*dev)
    torch.cuda.synchronize()
    assert o1.dtype == torch.float32 and o2.dtype == torch.float32
    errs = [rel_err(o1.cpu(), o_ref), rel_err(s1.cpu(), s_ref), rel_err(o2.cpu(), o_ref), rel_err(s2.cpu(), s_ref)]
    print("  rel_err attention o/S, prefill o/S: " + " ".join(f"{e:.2e}" for e in errs), flush=True)
    assert max(errs) < TOL


@pytest.mark.parametrize("st_dt", [torch.bfloat16, torch.float16])
def test_state_dtype_is_honoured(st_dt):
    """config.state_dtype as in the reference (inference.py:523-526): the
    incoming state is cast to it, the returned state is in it (the kernels
    compute in fp32 and round once), and a prompt shorter than one chunk or a
    decode call updates a state already in that dtype in place."""
    print(f"state_dtype {st_dt}", flush=True)
    B, S, H, D = 2, 200, 2, 64
    cpu, dev = device_inputs(B, S + 5, H, D, D, torch.bfloat16)
    s0 = seeded_state(B, H, D, D).to(st_dt)
    cfg = GDN2Config(output_dtype=torch.float32, state_dtype=st_dt)
    o, st = gdn2_prefill(*(t[:, :S] for t in dev), s0.cuda(), config=cfg)
    o_ref, s_ref = oracle.prefill(*(t[:, :S] for t in cpu), s0.float().clone())
    torch.cuda.synchronize()
    assert st.dtype == st_dt
    assert rel_err(o.cpu(), o_ref) < TOL
    assert rel_err(st.float().cpu(), s_ref) < TOL + 2.0 ** -8
    # short prompt: the state in state_dtype is updated in place
    st_short = st.clone()
    o2, st2 = gdn2_prefill(*(t[:, S:S + 5] for t in dev), st_short, config=cfg)
    o2_ref = oracle.decode_loop(*(t[:, S:S + 5] for t in cpu), st.float().cpu().clone(), None).float()
    torch.cuda.synchronize()
    assert st2 is st_short and st2.dtype == st_dt
    assert rel_err(o2.cpu(), o2_ref) < TOL
    st3 = st.clone()
    gdn2_decode(*(t[:, S:S + 5] for t in dev), st3)
    torch.cuda.synchronize()
    assert st3.dtype == st_dt and torch.equal(st3, st2)
    _, fin = gdn2_attention(*(t[:, :S] for t in dev), initial_state=s0.cuda(), output_final_state=True,
                            config=cfg)
    torch.cuda.synchronize()
    assert fin.dtype == st_dt and rel_err(fin.float().cpu(), s_ref) < TOL + 2.0 ** -8
