"""CPU restatement of the ``GatedDeltaNet2`` layer -- TEST INFRASTRUCTURE ONLY.

Functional float32 restatement of ``gdn2/attention.py:232-491`` driven by a
``state_dict`` of the product module, so a test can run the same weights
through both. The maths it follows:

* projections ``q,k,v,b,w,f,o_gate`` and ``o_proj`` (``attention.py:262-272``);
* causal depthwise short conv + SiLU, with a ``kernel-1`` tail cache
  (``attention.py:186-215``);
* L2-normalised q, k per key head (``:397-398``);
* ``g = -exp(A_log) * softplus(f + dt_bias)`` (``:290-293``),
  ``b = sigmoid(.) * erase_scale``, ``w = sigmoid(.)`` (``:401-402``);
* key-head tensors repeated up to the value heads (``:295-297``);
* gated RMSNorm ``x * rsqrt(mean x^2 + eps) * weight * silu(gate)`` (``:218-229``).

The attention op itself is :func:`oracle.gdn2_oracle.prefill` /
:func:`oracle.gdn2_oracle.decode_loop`.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .gdn2_oracle import decode_loop, prefill


class LayerOracle:
    """Float32 CPU restatement of one GDN-2 layer with a serving cache."""

    def __init__(self, state_dict, hidden_size, num_heads, num_kv_heads, head_dim_k,
                 head_dim_v, conv_size=4, norm_eps=1e-5, erase_gate_scale=1.0, chunk_size=64):
        self.p = {k: v.detach().float().cpu() for k, v in state_dict.items()}
        self.H, self.HK = num_heads, num_kv_heads
        self.DK, self.DV = head_dim_k, head_dim_v
        self.conv_size = conv_size
        self.eps = norm_eps
        self.erase = erase_gate_scale
        self.chunk = chunk_size
        self.rep = num_heads // num_kv_heads

    def _lin(self, name, x):
        return x @ self.p[f"{name}.weight"].t()

    def _conv(self, name, x, tail):
        """Causal depthwise conv over ``[tail | x]``; returns (y, new tail)."""
        wgt = self.p[f"{name}.conv.weight"]
        bias = self.p.get(f"{name}.conv.bias")
        buf = torch.cat([tail, x.transpose(1, 2)], dim=-1)
        y = F.conv1d(buf, wgt, bias, groups=wgt.shape[0]).transpose(1, 2)
        return F.silu(y), buf[..., buf.shape[-1] - (self.conv_size - 1):]

    def gates(self, x):
        """``(g, b, w)`` of ``x [B, S, hidden]`` on the key (g, b) and value (w)
        heads: ``g = -exp(A_log) * softplus(f + dt_bias)`` (``attention.py:290-293``),
        ``b = sigmoid(.) * erase_scale``, ``w = sigmoid(.)`` (``:401-402``)."""
        B, S, _ = x.shape
        f = self._lin("f_proj", x).view(B, S, self.HK, self.DK)
        g = -self.p["A_log"].exp()[:, None] * F.softplus(f + self.p["dt_bias"])
        b = torch.sigmoid(self._lin("b_proj", x).view(B, S, self.HK, self.DK)) * self.erase
        w = torch.sigmoid(self._lin("w_proj", x).view(B, S, self.H, self.DV))
        return g, b, w

    def gated_norm(self, o, gate):
        """``o * rsqrt(mean o^2 + eps) * weight * silu(gate)`` per value head
        (``attention.py:218-229``)."""
        o = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + self.eps)
        return o * self.p["o_norm.weight"] * F.silu(gate)

    def init_cache(self, B):
        C = 2 * self.HK * self.DK + self.H * self.DV
        state = torch.zeros(B, self.H, self.DK, self.DV)
        conv = torch.zeros(B, C, self.conv_size - 1) if self.conv_size > 0 else None
        return [state, conv]

    def _mix(self, x, cache, use_decode):
        x = x.float().cpu()
        B, S, _ = x.shape
        H, HK, DK, DV = self.H, self.HK, self.DK, self.DV
        q, k, v = self._lin("q_proj", x), self._lin("k_proj", x), self._lin("v_proj", x)
        if self.conv_size > 0:
            d = HK * DK
            cs = cache[1]
            q, cq = self._conv("q_conv", q, cs[:, :d])
            k, ck = self._conv("k_conv", k, cs[:, d:2 * d])
            v, cv = self._conv("v_conv", v, cs[:, 2 * d:])
            cache[1] = torch.cat([cq, ck, cv], dim=1)
        q = F.normalize(q.view(B, S, HK, DK), dim=-1)
        k = F.normalize(k.view(B, S, HK, DK), dim=-1)
        v = v.view(B, S, H, DV)
        g, b, w = self.gates(x)
        if self.rep > 1:
            q, k, b, g = (t.repeat_interleave(self.rep, dim=2) for t in (q, k, b, g))
        if use_decode:
            o = decode_loop(q, k, v, g, b, w, cache[0], None).float()
        else:
            o, cache[0] = prefill(q, k, v, g, b, w, cache[0], None, chunk_size=self.chunk)
        gate = self._lin("o_gate_proj", x).view(B, S, H, DV)
        o = self.gated_norm(o, gate)
        return self._lin("o_proj", o.reshape(B, S, H * DV))

    def prefill(self, x, cache=None):
        """``GatedDeltaNet2.prefill`` (``attention.py:360-414``)."""
        if cache is None:
            cache = self.init_cache(x.shape[0])
        return self._mix(x, cache, use_decode=False), cache

    def decode(self, x, cache):
        """``GatedDeltaNet2.decode`` (``attention.py:417-465``)."""
        return self._mix(x, cache, use_decode=True), cache
