"""Layer plumbing on the CPU (no GPU): GatedDeltaNet2's projections, short-conv
cache, gates, head expansion, gated RMSNorm and segment handling, with the
attention op itself replaced by the oracle (the op's own parity is the GPU
tests' job). Mirrors reference tests/test_gdn2.py:150-182 and
tests/test_inference.py:61-178."""

from __future__ import annotations

import pytest
import torch

import oracle
from gdt2_tilelang_amd import GatedDeltaNet2, GatedDeltaNet2Config
from gdt2_tilelang_amd import attention as attn_mod
from oracle import LayerOracle, rel_err

REFERENCE_PARAM_NAMES = {
    "q_proj.weight", "k_proj.weight", "v_proj.weight", "b_proj.weight", "w_proj.weight",
    "f_proj.weight", "o_gate_proj.weight", "o_proj.weight",
    "q_conv.conv.weight", "q_conv.conv.bias", "k_conv.conv.weight", "k_conv.conv.bias",
    "v_conv.conv.weight", "v_conv.conv.bias", "A_log", "dt_bias", "o_norm.weight",
}


@pytest.fixture
def oracle_op(monkeypatch):
    """Route the layer's op calls to the CPU oracle for host-logic tests. The
    layer hands the op grouped key heads; the oracle (like the reference's op)
    takes them repeated up to the value heads."""

    def expand(q, k, v, g, b, w):
        rep = v.shape[2] // q.shape[2]
        q, k, g, b = (t.repeat_interleave(rep, dim=2) for t in (q, k, g, b))
        return q, k, v, g, b, w

    def attention(q, k, v, g, b, w, scale=None, initial_state=None, output_final_state=False,
                  config=None, cu_seqlens=None):
        q, k, v, g, b, w = expand(q, k, v, g, b, w)
        S = q.shape[1]
        pad = (-S) % 64
        if pad:
            q, k, v, g, b, w = (torch.cat([t, t.new_zeros(t.shape[0], pad, *t.shape[2:])], 1)
                                for t in (q, k, v, g, b, w))
        o, st = oracle.chunk_gdn2(q, k, v, g, b, w, scale, initial_state, output_final_state)
        return o[:, :S], st

    def prefill(q, k, v, g, b, w, state=None, scale=None, config=None):
        return oracle.prefill(*expand(q, k, v, g, b, w), state, scale)

    def decode(q, k, v, g, b, w, state, scale=None):
        return oracle.decode_loop(*expand(q, k, v, g, b, w), state, scale)

    monkeypatch.setattr(attn_mod, "gdn2_attention", attention)
    monkeypatch.setattr(attn_mod, "gdn2_prefill", prefill)
    monkeypatch.setattr(attn_mod, "gdn2_decode", decode)


def small_layer(H=2, HK=None, D=16, hid=64, seed=0):
    torch.manual_seed(seed)
    cfg = GatedDeltaNet2Config(hidden_size=hid, num_heads=H, num_kv_heads=HK, head_dim_k=D, head_dim_v=D)
    return GatedDeltaNet2(cfg).eval()


def test_parameter_names_match_reference():
    layer = small_layer()
    assert set(dict(layer.named_parameters())) == REFERENCE_PARAM_NAMES


def test_grouped_heads_rejects_bad_ratio():
    with pytest.raises(ValueError, match="multiple of num_kv_heads"):
        GatedDeltaNet2(GatedDeltaNet2Config(hidden_size=64, num_heads=6, num_kv_heads=4))


def test_packed_sequences_rejected_through_short_conv():
    """The layer's causal conv would mix tokens across packed sequences."""
    layer = small_layer()
    with pytest.raises(NotImplementedError, match="cu_seqlens"):
        layer(torch.randn(1, 8, 64), cu_seqlens=torch.tensor([0, 3, 8]))


@pytest.mark.parametrize("draft", [1, 2, 5])
def test_decode_matches_forward(oracle_op, draft):
    layer = small_layer()
    x = torch.randn(2, 24, 64, generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        full, _ = layer(x)
        cache = layer.init_cache(2)
        parts = [layer.decode(x[:, i:i + draft], cache)[0] for i in range(0, 24, draft)]
    assert rel_err(torch.cat(parts, 1), full) < 1e-4


def test_prefill_step_serving_loop(oracle_op):
    layer = small_layer(H=4, HK=2)
    x = torch.randn(1, 150, 64, generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        full, _ = layer(x)
        pre, cache = layer.prefill(x[:, :70])          # ragged: 64 + 6-token tail
        pre2, cache = layer.prefill(x[:, 70:131], cache)  # second segment
        draft, cache = layer.decode(x[:, 131:135], cache)
        gen = torch.stack([layer.step(x[:, t], cache)[0] for t in range(135, 150)], 1)
    assert rel_err(torch.cat([pre, pre2, draft, gen], 1), full) < 1e-4


def test_forward_use_cache_then_step(oracle_op):
    layer = small_layer()
    x = torch.randn(1, 20, 64, generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        full, _ = layer(x)
        prompt, cache = layer(x[:, :12], use_cache=True)
        gen = [layer.step(x[:, t], cache)[0] for t in range(12, 20)]
    assert rel_err(torch.cat([prompt, torch.stack(gen, 1)], 1), full) < 1e-4


def test_layer_matches_layer_oracle(oracle_op):
    """Same weights through the module and the functional LayerOracle."""
    layer = small_layer(H=4, HK=2, D=16, hid=64)
    ref = LayerOracle(layer.state_dict(), 64, 4, 2, 16, 16)
    x = torch.randn(2, 90, 64, generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        out, cache = layer.prefill(x[:, :80])
        out2, cache = layer.decode(x[:, 80:], cache)
    r1, rc = ref.prefill(x[:, :80])
    r2, rc = ref.decode(x[:, 80:], rc)
    assert rel_err(out, r1) < 1e-5 and rel_err(out2, r2) < 1e-5
    assert rel_err(cache.recurrent_state, rc[0]) < 1e-5
    assert rel_err(cache.conv_state, rc[1]) < 1e-6


def test_bf16_layer_cache_dtypes(oracle_op):
    """A bf16 layer keeps an fp32 state and a bf16 conv tail, and can decode."""
    layer = small_layer().to(torch.bfloat16)
    cache = layer.init_cache(2)
    assert cache.recurrent_state.dtype == torch.float32
    assert cache.conv_state.dtype == torch.bfloat16
    x = torch.randn(2, 3, 64, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    with torch.no_grad():
        out, cache = layer.decode(x, cache)
    assert out.dtype == torch.bfloat16 and torch.isfinite(out.float()).all()
