"""Write the golden vectors for BASELINE config 0 (CPU plumbing case).

Config 0: B=1 S=256 H=2 DK=DV=64, fp32 inputs drawn from one CPU torch
generator seeded 0 in the order q, k (L2-normalised), v, g = logsigmoid(N(0,1)),
b, w = sigmoid(N(0,1)). The expected outputs come from a float64 numpy
recurrence written here independently of ``oracle/`` -- it is the GDN-2
definition (reference ``gdn2/reference.py:8-23``) read as plain loops:

    S <- diag(exp g_t) S
    u  = w_t * v_t - S^T (b_t * k_t)
    S <- S + k_t u^T
    o_t = scale * S^T q_t

so it pins the oracle rather than restating it. The fixture stores the
outputs plus per-input sums that detect a change in the generator.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def config0_inputs():
    gen = torch.Generator(device="cpu").manual_seed(0)
    kw = dict(generator=gen, dtype=torch.float32)
    B, S, H, D = 1, 256, 2, 64
    q = F.normalize(torch.randn(B, S, H, D, **kw), dim=-1)
    k = F.normalize(torch.randn(B, S, H, D, **kw), dim=-1)
    v = torch.randn(B, S, H, D, **kw)
    g = F.logsigmoid(torch.randn(B, S, H, D, **kw))
    b = torch.sigmoid(torch.randn(B, S, H, D, **kw))
    w = torch.sigmoid(torch.randn(B, S, H, D, **kw))
    return q, k, v, g, b, w


def numpy_recurrence(q, k, v, g, b, w, scale):
    """float64 loops over batch, head and time; returns (o, final state)."""
    q, k, v, g, b, w = (np.asarray(t, dtype=np.float64) for t in (q, k, v, g, b, w))
    Bn, T, H, DK = q.shape
    DV = v.shape[-1]
    o = np.zeros((Bn, T, H, DV))
    final = np.zeros((Bn, H, DK, DV))
    for bi in range(Bn):
        for h in range(H):
            S = np.zeros((DK, DV))
            for t in range(T):
                S = np.exp(g[bi, t, h])[:, None] * S
                u = w[bi, t, h] * v[bi, t, h] - S.T.dot(b[bi, t, h] * k[bi, t, h])
                S = S + np.outer(k[bi, t, h], u)
                o[bi, t, h] = scale * S.T.dot(q[bi, t, h])
            final[bi, h] = S
    return o, final


def main():
    ins = config0_inputs()
    scale = 64 ** -0.5
    o, S = numpy_recurrence(*(t.numpy() for t in ins), scale)
    sums = np.array([float(t.double().sum()) for t in ins])
    path = os.path.join(HERE, "config0.npz")
    np.savez_compressed(path, o=o, S=S, input_sums=sums, scale=np.float64(scale))
    print(f"wrote {path}: o {o.shape}, S {S.shape}")


if __name__ == "__main__":
    main()
