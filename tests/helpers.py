"""Shared test helpers: seeded inputs on the device in a given dtype."""

from __future__ import annotations

import torch

from oracle import make_config_inputs, make_inputs


def device_inputs(B, S, H, DK, DV, dtype=torch.bfloat16, decay_scale=4.0, seed=0, dist="ref"):
    """(cpu fp32 inputs as the kernel sees them, device inputs).

    q, k, v, b, w are rounded to ``dtype`` first, so the CPU copies hold exactly
    the values the kernel reads; g stays fp32.
    """
    if dist == "ref":
        ins = make_inputs(B, S, H, DK, DV, decay_scale=decay_scale, seed=seed)
    else:
        ins = make_config_inputs(B, S, H, DK, DV, seed=seed)
    q, k, v, g, b, w = ins
    q, k, v, b, w = (t.to(dtype) for t in (q, k, v, b, w))
    cpu = tuple(t.float() for t in (q, k, v)) + (g,) + tuple(t.float() for t in (b, w))
    dev = tuple(t.cuda() for t in (q, k, v, g, b, w))
    return cpu, dev


def seeded_state(B, H, DK, DV, scale=0.2, seed=1):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(B, H, DK, DV, generator=gen) * scale
