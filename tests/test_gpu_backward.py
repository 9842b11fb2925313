"""Training backward (GPU) against autograd through the float64 recurrence.

The reference checks its staged backward against autograd through its own
forward (reference tests/test_backward.py:21-72: rel_err < 1e-4 for every
gradient, with and without state gradients, and under fast decay). Here the
hip backward (gdn2_hip_backward through chunk_gdn2_bwd / gdn2_attention) is
checked against torch autograd through oracle.recurrent_gdn2 in float64, the
pinned token recurrence, so no step of the chunkwise derivation is taken on
trust. Grouped heads are compared against autograd through the reference's
repeat_interleave of q, k, g, b (whose backward sums the value heads of a key
head). Inputs are rounded to the kernel dtype before the oracle sees them.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from gdt2_tilelang_amd import GDN2Config, GatedDeltaNet2, GatedDeltaNet2Config, chunk_gdn2_bwd, gdn2_attention

pytestmark = pytest.mark.gpu
rel_err = oracle.rel_err
NAMES = ["dq", "dk", "dv", "dg", "db", "dw", "dS0"]


def _inputs(B, S, H, HK, DK, DV, decay, seed):
    q, k, _, g, b, _ = oracle.make_inputs(B, S, HK, DK, DV, decay_scale=decay, seed=seed)
    _, _, v, _, _, w = oracle.make_inputs(B, S, H, DK, DV, decay_scale=decay, seed=seed + 1)
    return q, k, v, g, b, w


def _autograd(q, k, v, g, b, w, s0, do, dht, scale, rep):
    ts = [t.detach().double().cpu().requires_grad_(True) for t in (q, k, v, g, b, w)]
    s0t = None if s0 is None else s0.detach().double().cpu().requires_grad_(True)
    qq, kk, gg, bb = (t.repeat_interleave(rep, dim=2) for t in (ts[0], ts[1], ts[3], ts[4]))
    o, sf = oracle.recurrent_gdn2(qq, kk, ts[2], gg, bb, ts[5], scale, s0t, dht is not None, dtype=torch.float64)
    loss = (o * do.double().cpu()).sum()
    if dht is not None:
        loss = loss + (sf * dht.double().cpu()).sum()
    loss.backward()
    return [t.grad for t in ts] + [None if s0t is None else s0t.grad]


@pytest.mark.parametrize("B,S,H,HK,DK,DV,dtype,state,dht,decay", [
    (2, 128, 3, 3, 32, 32, torch.float32, True, True, 4.0),
    (2, 150, 4, 2, 64, 48, torch.float32, True, True, 4.0),
    (1, 200, 2, 2, 128, 128, torch.float32, False, False, 4.0),
    (1, 128, 2, 1, 64, 64, torch.float32, False, False, 25.0),
    (1, 70, 2, 2, 128, 64, torch.float32, True, False, 1.0),
    (2, 100, 2, 2, 64, 64, torch.bfloat16, True, True, 4.0),
    (1, 300, 4, 2, 128, 128, torch.float32, True, True, 2.0),
    (1, 64, 2, 2, 128, 32, torch.float16, False, True, 4.0),
])
def test_backward_matches_autograd(B, S, H, HK, DK, DV, dtype, state, dht, decay):
    print(f"backward B={B} S={S} H={H} HK={HK} DK={DK} DV={DV} {dtype} state={state} dht={dht} "
          f"decay={decay}", flush=True)
    torch.manual_seed(0)
    q, k, v, g, b, w = (t.to(dtype).float() if t is not None else None for t in _inputs(B, S, H, HK, DK, DV,
                                                                                         decay, 0))
    g = g.float()
    s0 = torch.randn(B, H, DK, DV) * 0.3 if state else None
    do = (torch.randn(B, S, H, DV)).to(dtype).float()
    dh = torch.randn(B, H, DK, DV) * 0.5 if dht else None
    scale = DK ** -0.5
    ref = _autograd(q, k, v, g, b, w, s0, do, dh, scale, H // HK)
    cu = lambda t, dt=dtype: None if t is None else t.to(dt).cuda()
    got = chunk_gdn2_bwd(cu(q), cu(k), cu(v), g.cuda(), cu(b), cu(w), scale, cu(s0, torch.float32), cu(do),
                         cu(dh, torch.float32))
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    for name, a, r in zip(NAMES, got, ref):
        if r is None:
            assert a is None, name
            continue
        assert a.dtype == (torch.float32 if name in ("dg", "dS0") else dtype), name
        assert torch.isfinite(a.float()).all(), f"{name} not finite"
        e = rel_err(a.float(), r)
        print(f"  {name} rel err {e:.2e}", flush=True)
        assert e < tol, f"{name}: {e:.2e}"


def test_autograd_through_gdn2_attention():
    """loss.backward() through gdn2_attention runs the hip backward and gives
    the same gradients as a direct chunk_gdn2_bwd call."""
    print("autograd through gdn2_attention", flush=True)
    B, S, H, HK, DK, DV = 1, 130, 4, 2, 64, 64
    q, k, v, g, b, w = (t.cuda() for t in _inputs(B, S, H, HK, DK, DV, 4.0, 3))
    s0 = (torch.randn(B, H, DK, DV) * 0.3).cuda()
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, g, b, w, s0)]
    o, sf = gdn2_attention(*leaves[:6], initial_state=leaves[6], output_final_state=True,
                           config=GDN2Config(output_dtype=torch.float32))
    do = torch.randn_like(o)
    dh = torch.randn_like(sf)
    ((o * do).sum() + (sf * dh).sum()).backward()
    direct = chunk_gdn2_bwd(q, k, v, g, b, w, DK ** -0.5, s0, do, dh)
    torch.cuda.synchronize()
    for name, leaf, d in zip(NAMES, leaves, direct):
        assert leaf.grad is not None, name
        assert torch.equal(leaf.grad, d), name
    ref = _autograd(q, k, v, g, b, w, s0, do, dh, DK ** -0.5, H // HK)
    for name, leaf, r in zip(NAMES, leaves, ref):
        assert rel_err(leaf.grad, r) < 1e-4, name


def test_backward_zero_tokens():
    """With no tokens the initial-state gradient is the final-state gradient."""
    print("backward S=0", flush=True)
    x = torch.zeros(1, 0, 2, 64, device="cuda")
    s0 = torch.randn(1, 2, 64, 64, device="cuda")
    dh = torch.randn(1, 2, 64, 64, device="cuda")
    dq, dk, dv, dg, db, dw, ds0 = chunk_gdn2_bwd(x, x, x, x, x, x, None, s0, x, dh)
    torch.cuda.synchronize()
    assert dq.shape == x.shape and dv.shape == x.shape
    assert torch.equal(ds0, dh)


def test_layer_trains_through_the_hip_backward():
    """GatedDeltaNet2.forward under autograd on the GPU takes the torch-op
    projections around gdn2_attention (hip forward and backward): the loss
    gradient of every parameter exists and is finite, and the gradient of the
    input matches a central finite difference along a random direction."""
    print("layer backward", flush=True)
    torch.manual_seed(0)
    cfg = GatedDeltaNet2Config(hidden_size=128, num_heads=4, num_kv_heads=2, head_dim_k=64, head_dim_v=32)
    layer = GatedDeltaNet2(cfg).cuda()
    x = torch.randn(2, 90, 128, device="cuda", requires_grad=True)
    out, _ = layer(x)
    wgt = torch.randn_like(out)
    (out * wgt).sum().backward()
    for n, p in layer.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n
    d = torch.randn_like(x)
    eps = 3e-2
    # the same (training) path for both evaluations: the parameters require grad
    lp = (layer(x.detach() + eps * d)[0] * wgt).double().sum().item()
    lm = (layer(x.detach() - eps * d)[0] * wgt).double().sum().item()
    fd = (lp - lm) / (2 * eps)
    an = (x.grad * d).double().sum().item()
    print(f"  directional derivative: autograd {an:.6f} finite difference {fd:.6f}", flush=True)
    assert abs(an - fd) <= 2e-2 * max(1.0, abs(fd))


def test_packed_sequences_backward():
    """Autograd through gdn2_attention(cu_seqlens=...): every packed sequence
    (including an empty one) gets the gradients of its own recurrence."""
    print("packed backward", flush=True)
    H, HK, DK, DV = 2, 2, 64, 64
    lens = [70, 0, 130, 5]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T = int(cu[-1])
    q, k, v, g, b, w = _inputs(1, T, H, HK, DK, DV, 4.0, 5)
    N = len(lens)
    s0 = torch.randn(N, H, DK, DV) * 0.3
    do = torch.randn(1, T, H, DV)
    dh = torch.randn(N, H, DK, DV) * 0.5
    leaves = [t.cuda().requires_grad_(True) for t in (q, k, v, g, b, w, s0)]
    o, sf = gdn2_attention(*leaves[:6], initial_state=leaves[6], output_final_state=True,
                           config=GDN2Config(output_dtype=torch.float32), cu_seqlens=cu.cuda())
    ((o * do.cuda()).sum() + (sf * dh.cuda()).sum()).backward()
    torch.cuda.synchronize()
    for i, n in enumerate(lens):
        a = int(cu[i])
        sl = lambda t: t[:, a:a + n]
        ref = _autograd(*(sl(t) for t in (q, k, v, g, b, w)), s0[i:i + 1], sl(do), dh[i:i + 1], DK ** -0.5, 1)
        for name, leaf, r in zip(NAMES[:6], leaves[:6], ref[:6]):
            if n:
                assert rel_err(sl(leaf.grad), r) < 1e-4, (i, name)
        assert rel_err(leaves[6].grad[i:i + 1], ref[6]) < 1e-4, (i, "dS0")


def test_backward_sixteen_chunks_full_head_dims():
    """DK = DV = 128 over 16 chunks (1000 tokens, a ragged last chunk) with an
    initial state and a final-state gradient: the scans' chains across many
    chunk steps, against float64 autograd."""
    print("backward S=1000 DK=DV=128", flush=True)
    B, S, H, HK, DK, DV = 1, 1000, 2, 2, 128, 128
    q, k, v, g, b, w = _inputs(B, S, H, HK, DK, DV, 1.0, 9)
    s0 = torch.randn(B, H, DK, DV) * 0.3
    do = torch.randn(B, S, H, DV)
    dh = torch.randn(B, H, DK, DV) * 0.5
    ref = _autograd(q, k, v, g, b, w, s0, do, dh, DK ** -0.5, 1)
    got = chunk_gdn2_bwd(*(t.cuda() for t in (q, k, v, g, b, w)), None, s0.cuda(), do.cuda(), dh.cuda())
    torch.cuda.synchronize()
    for name, a, r in zip(NAMES, got, ref):
        e = rel_err(a, r)
        print(f"  {name} rel err {e:.2e}", flush=True)
        assert e < 1e-4, name


@pytest.mark.parametrize("lens,H,HK,DK,DV,dtype,state,dht", [
    ([70, 0, 130, 5, 64, 1, 200], 4, 2, 64, 48, torch.float32, True, True),
    ([300, 17, 0, 0, 128, 65], 2, 2, 128, 128, torch.bfloat16, True, False),
    ([33] * 20 + [0, 190], 3, 3, 32, 32, torch.float32, False, True),
    ([0, 0], 2, 1, 64, 64, torch.float32, True, True),
])
def test_packed_backward_equals_per_sequence_calls(lens, H, HK, DK, DV, dtype, state, dht):
    """chunk_gdn2_varlen_bwd (one gdn2_hip_backward_varlen call) gives
    bit-identical gradients to chunk_gdn2_bwd run on each sequence alone:
    each record slot repeats the dense chunk's arithmetic and each scan
    workgroup walks one sequence's chunks in the same order."""
    from gdt2_tilelang_amd import chunk_gdn2_varlen_bwd
    print(f"packed backward lens={lens} H={H} HK={HK} DK={DK} DV={DV} {dtype} state={state} dht={dht}", flush=True)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T, N = int(cu[-1]), len(lens)
    q, k, v, g, b, w = (t.to(dtype).cuda() for t in _inputs(1, max(T, 1), H, HK, DK, DV, 4.0, 11))
    q, k, v, g, b, w = (t[:, :T] for t in (q, k, v, g, b, w))
    g = g.float()
    gen = torch.Generator().manual_seed(12)
    s0 = (torch.randn(N, H, DK, DV, generator=gen) * 0.3).cuda() if state else None
    do = torch.randn(1, T, H, DV, generator=gen).to(dtype).cuda()
    dh = (torch.randn(N, H, DK, DV, generator=gen) * 0.5).cuda() if dht else None
    got = chunk_gdn2_varlen_bwd(q, k, v, g, b, w, None, cu.cuda(), s0, do, dh)
    torch.cuda.synchronize()
    for i, n in enumerate(lens):
        a = int(cu[i])
        sl = lambda t: t[:, a:a + n]
        if n == 0:
            if state:
                want = dh[i] if dht else torch.zeros_like(s0[i])
                assert torch.equal(got[6][i], want), (i, "dS0 pass-through")
            continue
        ref = chunk_gdn2_bwd(*(sl(t) for t in (q, k, v, g, b, w)), None,
                             None if s0 is None else s0[i:i + 1], sl(do), None if dh is None else dh[i:i + 1])
        for name, full, r in zip(NAMES[:6], got[:6], ref[:6]):
            assert torch.equal(sl(full), r), (i, name)
        if state:
            assert torch.equal(got[6][i:i + 1], ref[6]), (i, "dS0")


@pytest.mark.parametrize("in_dtype,do_dtype", [(torch.bfloat16, torch.float16), (torch.float16, torch.bfloat16),
                                               (torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16)])
def test_backward_output_gradient_dtypes(in_dtype, do_dtype):
    """The inputs are read in their own dtype and do in the inputs' dtype or
    fp32 in place; a do of another 16-bit dtype is widened first. Every
    combination gives exactly the gradients of the same do values in fp32
    (16-bit values are exact in fp32)."""
    print(f"backward in={in_dtype} do={do_dtype}", flush=True)
    B, S, H, HK, DK, DV = 1, 150, 4, 2, 64, 32
    q, k, v, g, b, w = (t.cuda() for t in _inputs(B, S, H, HK, DK, DV, 4.0, 21))
    q, k, v, b, w = (t.to(in_dtype) for t in (q, k, v, b, w))
    do = torch.randn(B, S, H, DV, generator=torch.Generator().manual_seed(22)).to(do_dtype).cuda()
    s0 = (torch.randn(B, H, DK, DV, generator=torch.Generator().manual_seed(23)) * 0.3).cuda()
    got = chunk_gdn2_bwd(q, k, v, g, b, w, None, s0, do, None)
    ref = chunk_gdn2_bwd(q, k, v, g, b, w, None, s0, do.float(), None)
    torch.cuda.synchronize()
    for name, a, r in zip(NAMES, got, ref):
        assert torch.equal(a, r), name


def test_backward_state_argument_shapes():
    """A wrong-shaped initial state or final-state gradient is refused before
    any launch (the kernels would read past it)."""
    from gdt2_tilelang_amd import chunk_gdn2_varlen_bwd
    q, k, v, g, b, w = (t.cuda() for t in _inputs(1, 100, 2, 2, 64, 64, 4.0, 31))
    do = torch.randn(1, 100, 2, 64, device="cuda")
    good = torch.zeros(1, 2, 64, 64, device="cuda")
    bad = torch.zeros(2, 2, 64, 64, device="cuda")
    with pytest.raises(ValueError, match="dht"):
        chunk_gdn2_bwd(q, k, v, g, b, w, None, good, do, bad)
    with pytest.raises(ValueError, match="initial_state"):
        chunk_gdn2_bwd(q, k, v, g, b, w, None, bad, do, None)
    cu = torch.tensor([0, 40, 100], dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="dht"):
        chunk_gdn2_varlen_bwd(q, k, v, g, b, w, None, cu, None, do, good)
    chunk_gdn2_varlen_bwd(q, k, v, g, b, w, None, cu, None, do, bad)   # two sequences: [2, H, DK, DV]
    torch.cuda.synchronize()
