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
