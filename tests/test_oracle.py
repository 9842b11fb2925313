"""Pinning the CPU oracle (no GPU).

Each oracle function is checked against something other than its own formula:
* golden vectors of BASELINE config 0 written by an independent float64 numpy
  recurrence (tests/golden/make_golden.py);
* closed forms: zero gates give S0 * exp(sum g); tied gates give the KDA loop;
* brute force: the strictly-lower pairwise products against a float64 triple sum;
* the reference's invariants (reference tests/test_gdn2.py:47-121,
  tests/test_inference.py:21-150): chunkwise == recurrence over chunk and
  sub-chunk sizes, with initial states and under fast decay; decode == the
  recurrence; multi-token decode == repeated single steps; ragged and
  segmented prefill == one pass.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import (chunk_gdn2, chunk_local_cumsum, decode_loop, make_inputs, prefill,
                    recurrent_gdn2, rel_err, strict_tril_pairwise)
from tests.golden.make_golden import config0_inputs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "config0.npz")


# ---------------------------------------------------------------------------
# golden vectors (config 0)
# ---------------------------------------------------------------------------

def test_golden_inputs_unchanged():
    ref = np.load(GOLDEN)
    sums = np.array([float(t.double().sum()) for t in config0_inputs()])
    np.testing.assert_allclose(sums, ref["input_sums"], rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 2e-6)])
def test_recurrence_matches_golden(dtype, tol):
    ref = np.load(GOLDEN)
    o, s = recurrent_gdn2(*config0_inputs(), output_final_state=True, dtype=dtype)
    assert rel_err(o, torch.from_numpy(ref["o"])) < tol
    assert rel_err(s, torch.from_numpy(ref["S"])) < tol


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-11), (torch.float32, 2e-5)])
def test_chunkwise_matches_golden(dtype, tol):
    ref = np.load(GOLDEN)
    o, s = chunk_gdn2(*config0_inputs(), output_final_state=True, dtype=dtype)
    assert rel_err(o, torch.from_numpy(ref["o"])) < tol
    assert rel_err(s, torch.from_numpy(ref["S"])) < tol


def test_prefill_matches_golden():
    ref = np.load(GOLDEN)
    o, s = prefill(*config0_inputs())
    assert rel_err(o, torch.from_numpy(ref["o"])) < 2e-5
    assert rel_err(s, torch.from_numpy(ref["S"])) < 2e-5


# ---------------------------------------------------------------------------
# chunkwise form == the recurrence
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("S,BS,BC", [(128, 64, 16), (256, 64, 32), (192, 32, 16), (64, 64, 8)])
def test_chunk_matches_recurrent(S, BS, BC):
    q, k, v, g, b, w = make_inputs(2, S, 3, 32, 48)
    o_ref, s_ref = recurrent_gdn2(q, k, v, g, b, w, output_final_state=True)
    o, s = chunk_gdn2(q, k, v, g, b, w, output_final_state=True, chunk_size=BS, sub_chunk_size=BC)
    assert rel_err(o, o_ref) < 2e-5
    assert rel_err(s, s_ref) < 2e-5


def test_chunk_with_initial_state():
    q, k, v, g, b, w = make_inputs(2, 128, 3, 32, 48)
    s0 = torch.randn(2, 3, 32, 48, generator=torch.Generator().manual_seed(3)) * 0.5
    o_ref, s_ref = recurrent_gdn2(q, k, v, g, b, w, initial_state=s0, output_final_state=True)
    o, s = chunk_gdn2(q, k, v, g, b, w, initial_state=s0, output_final_state=True)
    assert rel_err(o, o_ref) < 2e-5 and rel_err(s, s_ref) < 2e-5


@pytest.mark.parametrize("decay_scale", [0.0, 1.0, 8.0, 30.0])
def test_fast_decay_does_not_overflow(decay_scale):
    """At decay 30 a channel loses ~e^-1900 per chunk; exp(-G) would overflow."""
    q, k, v, g, b, w = make_inputs(1, 128, 2, 32, 32, decay_scale=decay_scale)
    o_ref, _ = recurrent_gdn2(q, k, v, g, b, w)
    o, _ = chunk_gdn2(q, k, v, g, b, w)
    assert torch.isfinite(o).all()
    assert rel_err(o, o_ref) < 1e-4


def test_chunk_rejects_bad_lengths():
    q, k, v, g, b, w = make_inputs(1, 100, 2, 16, 16)
    with pytest.raises(ValueError, match="divisible by chunk_size"):
        chunk_gdn2(q, k, v, g, b, w)
    q, k, v, g, b, w = make_inputs(1, 64, 2, 16, 16)
    with pytest.raises(ValueError, match="sub_chunk_size"):
        chunk_gdn2(q, k, v, g, b, w, sub_chunk_size=24)


# ---------------------------------------------------------------------------
# closed forms and degeneracies
# ---------------------------------------------------------------------------

def test_tied_gates_reduce_to_kda():
    """b = w = beta (scalar per token) is KDA: S = (I - beta k k^T) diag(a) S + beta k v^T."""
    q, k, v, g, _, _ = make_inputs(2, 128, 3, 32, 32)
    beta = torch.rand(2, 128, 3, 1, generator=torch.Generator().manual_seed(5))
    b = beta.expand(-1, -1, -1, 32).contiguous()
    o, _ = chunk_gdn2(q, k, v, g, b, b.clone())
    S = torch.zeros(2, 3, 32, 32)
    o_kda = torch.empty_like(o)
    for t in range(128):
        S = S * g[:, t].exp().unsqueeze(-1)
        kt, bt = k[:, t], beta[:, t, :, 0][..., None, None]
        S = S - bt * kt.unsqueeze(-1) * torch.einsum("bhkd,bhk->bhd", S, kt).unsqueeze(-2)
        S = S + bt * kt.unsqueeze(-1) * v[:, t].unsqueeze(-2)
        o_kda[:, t] = torch.einsum("bhkd,bhk->bhd", S, q[:, t]) * 32 ** -0.5
    assert rel_err(o, o_kda) < 2e-5


def test_zero_gates_are_pure_decay():
    q, k, v, g, _, _ = make_inputs(1, 128, 2, 32, 32)
    z = torch.zeros(1, 128, 2, 32)
    s0 = torch.randn(1, 2, 32, 32, generator=torch.Generator().manual_seed(7))
    _, s = chunk_gdn2(q, k, v, g, z, z, initial_state=s0, output_final_state=True)
    assert rel_err(s, s0 * g.sum(1).exp().unsqueeze(-1)) < 2e-5


def test_write_gate_changes_output():
    q, k, v, g, b, w = make_inputs(1, 128, 2, 32, 32)
    o1, _ = chunk_gdn2(q, k, v, g, b, w)
    o2, _ = chunk_gdn2(q, k, v, g, b, w * 0.5)
    assert not torch.allclose(o1, o2)


def test_pairwise_products_brute_force():
    """strict_tril_pairwise == float64 triple loop, including a fast-decay case."""
    gen = torch.Generator().manual_seed(11)
    for decay in (1.0, 20.0):
        x = torch.randn(32, 8, generator=gen, dtype=torch.float64)
        y = torch.randn(32, 8, generator=gen, dtype=torch.float64)
        g = -F.softplus(torch.randn(32, 8, generator=gen, dtype=torch.float64)) * decay
        G = g.cumsum(0)
        got = strict_tril_pairwise(x, y, G, 8)
        want = torch.zeros(32, 32, dtype=torch.float64)
        for r in range(32):
            for s in range(r):
                want[r, s] = sum(x[r, c] * y[s, c] * math.exp(G[r, c] - G[s, c]) for c in range(8))
        assert (got - want).abs().max() < 1e-12


def test_unit_lower_solve():
    """(I + Akk) Ai == I for the chunk's strictly-lower Akk."""
    q, k, v, g, b, w = make_inputs(1, 64, 1, 32, 32)
    G = chunk_local_cumsum(g, 64)[0, :, 0]
    T = strict_tril_pairwise(b[0, :, 0] * k[0, :, 0], k[0, :, 0], G, 16).double()
    eye = torch.eye(64, dtype=torch.float64)
    Ai = torch.linalg.solve_triangular(eye + T, eye, upper=False, unitriangular=True)
    assert (Ai @ (eye + T) - eye).abs().max() < 1e-10
    assert torch.equal(torch.triu(Ai, 1), torch.zeros_like(Ai))


# ---------------------------------------------------------------------------
# serving path
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 3, 8, 16])
def test_decode_matches_recurrence(n):
    q, k, v, g, b, w = make_inputs(2, n, 3, 32, 24)
    s0 = torch.randn(2, 3, 32, 24, generator=torch.Generator().manual_seed(2)) * 0.3
    o_ref, s_ref = recurrent_gdn2(q, k, v, g, b, w, None, s0, True)
    st = s0.clone()
    o = decode_loop(q, k, v, g, b, w, st)
    assert rel_err(o, o_ref) < 1e-5 and rel_err(st, s_ref) < 1e-5


def test_decode_multi_equals_single_steps():
    q, k, v, g, b, w = make_inputs(2, 12, 3, 32, 24)
    s0 = torch.randn(2, 3, 32, 24, generator=torch.Generator().manual_seed(2)) * 0.3
    a, c = s0.clone(), s0.clone()
    o_multi = decode_loop(q, k, v, g, b, w, a)
    o_one = torch.cat([decode_loop(*(t[:, i:i + 1] for t in (q, k, v, g, b, w)), c) for i in range(12)], 1)
    assert rel_err(o_multi, o_one) < 1e-5 and rel_err(a, c) < 1e-5


@pytest.mark.parametrize("S", [64, 128, 100, 7])
def test_prefill_matches_recurrence(S):
    q, k, v, g, b, w = make_inputs(2, S, 3, 32, 24)
    s0 = torch.randn(2, 3, 32, 24, generator=torch.Generator().manual_seed(2)) * 0.3
    o_ref, s_ref = recurrent_gdn2(q, k, v, g, b, w, None, s0, True)
    o, s = prefill(q, k, v, g, b, w, s0.clone())
    assert o.shape == (2, S, 3, 24)
    assert rel_err(o, o_ref) < 2e-5 and rel_err(s, s_ref) < 2e-5


def test_segmented_prefill_equals_one_pass():
    q, k, v, g, b, w = make_inputs(2, 192, 3, 32, 24)
    o_all, s_all = prefill(q, k, v, g, b, w)
    outs, st = [], None
    for lo, hi in ((0, 64), (64, 160), (160, 192)):
        o, st = prefill(*(t[:, lo:hi] for t in (q, k, v, g, b, w)), st)
        outs.append(o)
    assert rel_err(torch.cat(outs, 1), o_all) < 2e-5 and rel_err(st, s_all) < 2e-5


def test_log2_space_cumsum():
    """The kernels' log2-space decay (2^(log2e * G)) equals exp(G)."""
    g = make_inputs(1, 128, 2, 16, 16)[3]
    G = chunk_local_cumsum(g, 64)
    assert torch.allclose(torch.exp2(G * math.log2(math.e)), G.exp(), rtol=1e-5, atol=1e-30)


# ---------------------------------------------------------------------------
# LayerOracle: each step against what the mathematics fixes (reference
# gdn2/attention.py:186-229, 290-297, 397-402), on hand-built weights
# ---------------------------------------------------------------------------

def _layer_params(hid, H, HK, DK, DV, K=4, seed=0):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen) * 0.3  # noqa: E731
    dqk, dv = HK * DK, H * DV
    p = {"q_proj.weight": r(dqk, hid), "k_proj.weight": r(dqk, hid), "v_proj.weight": r(dv, hid),
         "b_proj.weight": r(dqk, hid), "w_proj.weight": r(dv, hid), "f_proj.weight": r(dqk, hid),
         "o_gate_proj.weight": r(dv, hid), "o_proj.weight": r(hid, dv),
         "A_log": torch.rand(HK, generator=gen).log(), "dt_bias": r(HK, DK),
         "o_norm.weight": 1.0 + r(DV)}
    if K > 0:
        for name, c in (("q_conv", dqk), ("k_conv", dqk), ("v_conv", dv)):
            p[f"{name}.conv.weight"] = r(c, 1, K)
            p[f"{name}.conv.bias"] = r(c)
    return p


@pytest.mark.parametrize("shift", [0, 1, 3])
def test_layer_oracle_conv_one_hot_taps(shift):
    """A one-hot tap at position K-1-shift is SiLU of the input delayed by
    `shift` tokens plus the channel's bias; the first `shift` outputs read the
    cached tail, and the new tail is the last K-1 inputs."""
    K, C, S = 4, 6, 9
    wgt = torch.zeros(C, 1, K)
    wgt[:, 0, K - 1 - shift] = 1.0
    bias = torch.linspace(-1.0, 1.5, C)
    lo = oracle.LayerOracle({"c.conv.weight": wgt, "c.conv.bias": bias}, 8, 1, 1, 4, 4, conv_size=K)
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(2, S, C, generator=gen)
    tail = torch.randn(2, C, K - 1, generator=gen)
    y, new_tail = lo._conv("c", x, tail)
    seq = torch.cat([tail.transpose(1, 2), x], 1)            # [B, K-1+S, C]
    want = F.silu(seq[:, K - 1 - shift:K - 1 - shift + S] + bias)
    torch.testing.assert_close(y, want, rtol=0, atol=1e-6)
    torch.testing.assert_close(new_tail, x[:, S - (K - 1):].transpose(1, 2), rtol=0, atol=0)


def test_layer_oracle_gates_closed_form():
    """f = 0 (zero f_proj) gives g = -a * softplus(dt_bias) with a = exp(A_log);
    zero b_proj / w_proj give b = erase_scale / 2 and w = 1/2; b is linear in
    erase_scale."""
    hid, H, HK, DK, DV = 8, 4, 2, 3, 2
    p = _layer_params(hid, H, HK, DK, DV, K=0)
    p["f_proj.weight"].zero_()
    p["A_log"] = torch.tensor([math.log(3.0), math.log(0.5)])
    p["dt_bias"] = torch.tensor([[0.0, 1.0, -2.0], [5.0, -1.0, 0.25]])
    x = torch.randn(2, 5, hid, generator=torch.Generator().manual_seed(1))
    g, b, w = oracle.LayerOracle(p, hid, H, HK, DK, DV, conv_size=0, erase_gate_scale=0.7).gates(x)
    sp = lambda z: math.log1p(math.exp(z))  # noqa: E731
    want = torch.tensor([[-3.0 * sp(z) for z in (0.0, 1.0, -2.0)], [-0.5 * sp(z) for z in (5.0, -1.0, 0.25)]])
    assert abs(want[0, 0] + 3.0 * math.log(2.0)) < 1e-12
    torch.testing.assert_close(g, want.expand_as(g), rtol=1e-6, atol=1e-7)
    _, b1, _ = oracle.LayerOracle(p, hid, H, HK, DK, DV, conv_size=0, erase_gate_scale=1.0).gates(x)
    torch.testing.assert_close(b, 0.7 * b1, rtol=1e-6, atol=0)
    p["b_proj.weight"].zero_()
    p["w_proj.weight"].zero_()
    _, b0, w0 = oracle.LayerOracle(p, hid, H, HK, DK, DV, conv_size=0, erase_gate_scale=0.7).gates(x)
    assert torch.all(b0 == 0.35) and torch.all(w0 == 0.5)


def test_layer_oracle_gated_norm_constant_row():
    """A constant row o = c gives rsqrt(c^2 + eps) * c * weight * silu(gate)."""
    DV, eps, c = 5, 1e-5, -0.75
    p = _layer_params(8, 1, 1, 4, DV, K=0)
    lo = oracle.LayerOracle(p, 8, 1, 1, 4, DV, conv_size=0, norm_eps=eps)
    gate = torch.tensor([-2.0, -0.5, 0.0, 1.0, 3.0])
    got = lo.gated_norm(torch.full((1, 1, 1, DV), c), gate.view(1, 1, 1, DV))
    silu = [z / (1.0 + math.exp(-z)) for z in gate.tolist()]
    want = [c / math.sqrt(c * c + eps) * wt * s for wt, s in zip(p["o_norm.weight"].tolist(), silu)]
    torch.testing.assert_close(got.flatten(), torch.tensor(want), rtol=1e-6, atol=1e-7)


def test_layer_oracle_end_to_end_float64():
    """The whole layer (no conv) against a float64 numpy composition of its
    definition: projections, per-key-head L2 norm, the gates, value head h
    reading key head h // (H / HK), the recurrence from tests/golden (written
    independently of oracle/), the gated RMSNorm and o_proj. Prefill in two
    segments, then a decode call, with the state carried."""
    from tests.golden.make_golden import numpy_recurrence

    hid, H, HK, DK, DV, S = 12, 4, 2, 8, 6, 150
    p = _layer_params(hid, H, HK, DK, DV, K=0, seed=3)
    lo = oracle.LayerOracle(p, hid, H, HK, DK, DV, conv_size=0, erase_gate_scale=0.9)
    x = torch.randn(1, S, hid, generator=torch.Generator().manual_seed(2))
    o1, c = lo.prefill(x[:, :70])
    o2, c = lo.prefill(x[:, 70:140], c)
    o3, c = lo.decode(x[:, 140:], c)
    got = torch.cat([o1, o2, o3], 1).double().numpy()

    P = {k: v.double().numpy() for k, v in p.items()}
    xn = x.double().numpy()[0]
    def heads(a, n, d):  # noqa: E306
        return a.reshape(S, n, d)
    nrm = lambda a: a / np.linalg.norm(a, axis=-1, keepdims=True)  # noqa: E731
    sig = lambda a: 1.0 / (1.0 + np.exp(-a))  # noqa: E731
    q = nrm(heads(xn @ P["q_proj.weight"].T, HK, DK))
    k = nrm(heads(xn @ P["k_proj.weight"].T, HK, DK))
    v = heads(xn @ P["v_proj.weight"].T, H, DV)
    f = heads(xn @ P["f_proj.weight"].T, HK, DK) + P["dt_bias"]
    g = -np.exp(P["A_log"])[:, None] * np.log1p(np.exp(f))
    b = sig(heads(xn @ P["b_proj.weight"].T, HK, DK)) * 0.9
    w = sig(heads(xn @ P["w_proj.weight"].T, H, DV))
    kh = [h * HK // H for h in range(H)]
    o, _ = numpy_recurrence(*(a[None][:, :, kh] for a in (q, k)), v[None], *(a[None][:, :, kh] for a in (g, b)),
                            w[None], DK ** -0.5)
    o = o[0]
    gate = heads(xn @ P["o_gate_proj.weight"].T, H, DV)
    o = o / np.sqrt((o ** 2).mean(-1, keepdims=True) + 1e-5) * P["o_norm.weight"] * gate * sig(gate)
    want = o.reshape(S, H * DV) @ P["o_proj.weight"].T
    assert np.abs(got[0] - want).max() / np.abs(want).max() < 2e-5
