"""CPU restatement of the GDN-2 attention maths -- TEST INFRASTRUCTURE ONLY.

This module is the checker the HIP path is compared against and the CPU
baseline ``bench.py`` times. Nothing in the product package imports it.

What it restates (file:line into the reference ``amaranthine09/GDT2_TileLang``):

* ``recurrent_gdn2`` -- the token recurrence that defines GDN-2,
  ``gdn2/reference.py:56-107``::

      S_t = (I - k_t (b_t * k_t)^T) diag(exp g_t) S_{t-1} + k_t (w_t * v_t)^T
      o_t = scale * S_t^T q_t

* ``chunk_gdn2`` -- the chunkwise WY form, ``gdn2/reference.py:168-261``, with
  the chunk-local cumsum (``:110-113``) and the overflow-safe strictly-lower
  pairwise products (``:116-165``).
* ``decode_loop`` / ``decode_step`` -- the per-token torch loops the reference
  runs off-GPU, ``gdn2/inference.py:337-345`` and ``:183-189``.
* ``prefill`` -- whole chunks through the chunkwise form, a ragged tail through
  the decode loop, ``gdn2/inference.py:517-539``.
* ``make_inputs`` -- the reference's seeded test inputs,
  ``tests/test_gdn2.py:24-35``; ``rel_err`` -- its error metric, ``:38-39``.

How each function is pinned (the tests under ``tests/test_oracle.py``):

* ``recurrent_gdn2`` against golden vectors written by an independent float64
  numpy recurrence (``tests/golden/make_golden.py``), against a KDA loop when
  ``b = w = beta`` and against the closed form ``S0 * exp(sum g)`` when
  ``b = w = 0``.
* ``chunk_gdn2`` against ``recurrent_gdn2`` over several chunk/sub-chunk sizes,
  initial states and decay scales up to 30 (where ``exp(-G)`` would overflow).
* ``strict_tril_pairwise`` against the brute-force ``exp(G_r - G_s)`` sum in
  float64 on tiny inputs.
* The triangular solve against ``(I + T) @ Ai == I``.
* ``decode_loop`` / ``prefill`` against ``recurrent_gdn2``, including ragged
  and segmented prompts.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = [
    "recurrent_gdn2",
    "chunk_local_cumsum",
    "strict_tril_pairwise",
    "chunk_gdn2",
    "decode_loop",
    "decode_step",
    "prefill",
    "make_inputs",
    "make_config_inputs",
    "rel_err",
]


def rel_err(a: torch.Tensor, ref: torch.Tensor) -> float:
    """``max|a - ref| / max|ref|`` -- the reference's metric (``tests/test_gdn2.py:38-39``)."""
    a = a.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return ((a - ref).abs().max() / ref.abs().max().clamp_min(1e-6)).item()


def make_inputs(B, S, H, DK, DV, decay_scale=4.0, device="cpu", seed=0):
    """Seeded inputs drawn exactly as ``tests/test_gdn2.py:24-35`` draws them.

    Order from one CPU generator: q, k (L2-normalised), v, g = -softplus * scale,
    b, w = sigmoid. All fp32.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    kw = dict(generator=gen, dtype=torch.float32)
    q = F.normalize(torch.randn(B, S, H, DK, **kw), dim=-1)
    k = F.normalize(torch.randn(B, S, H, DK, **kw), dim=-1)
    v = torch.randn(B, S, H, DV, **kw)
    g = -F.softplus(torch.randn(B, S, H, DK, **kw)) * decay_scale
    b = torch.sigmoid(torch.randn(B, S, H, DK, **kw))
    w = torch.sigmoid(torch.randn(B, S, H, DV, **kw))
    return tuple(t.to(device) for t in (q, k, v, g, b, w))


def make_config_inputs(B, S, H, DK, DV, seed=0, device="cpu"):
    """The benchmark configs' distributions: q,k ~ N(0,1) L2-normalised,
    v ~ N(0,1), g = logsigmoid(N(0,1)), b,w = sigmoid(N(0,1)); same draw order."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    kw = dict(generator=gen, dtype=torch.float32)
    q = F.normalize(torch.randn(B, S, H, DK, **kw), dim=-1)
    k = F.normalize(torch.randn(B, S, H, DK, **kw), dim=-1)
    v = torch.randn(B, S, H, DV, **kw)
    g = F.logsigmoid(torch.randn(B, S, H, DK, **kw))
    b = torch.sigmoid(torch.randn(B, S, H, DK, **kw))
    w = torch.sigmoid(torch.randn(B, S, H, DV, **kw))
    return tuple(t.to(device) for t in (q, k, v, g, b, w))


def recurrent_gdn2(q, k, v, g, b, w, scale=None, initial_state=None,
                   output_final_state=False, dtype=torch.float32):
    """Token-by-token recurrence (``gdn2/reference.py:56-107``).

    Args are ``[B, T, H, D]``; ``initial_state`` is ``[B, H, DK, DV]``.
    ``dtype`` selects the arithmetic (float32 like the reference, or float64).
    Returns ``(o [B, T, H, DV], final_state or None)``.
    """
    B, T, H, DK = q.shape
    DV = v.shape[-1]
    scale = DK ** -0.5 if scale is None else scale
    q, k, v, g, b, w = (t.to(dtype) for t in (q, k, v, g, b, w))
    if initial_state is None:
        S = torch.zeros(B, H, DK, DV, dtype=dtype)
    else:
        S = initial_state.to(dtype).clone()
    o = torch.empty(B, T, H, DV, dtype=dtype)
    for t in range(T):
        S = S * g[:, t].exp()[..., None]                      # decay on the key axis
        erase = torch.einsum("bhcd,bhc->bhd", S, b[:, t] * k[:, t])
        u = w[:, t] * v[:, t] - erase                          # what the write adds
        S = S + k[:, t][..., None] * u[..., None, :]
        o[:, t] = torch.einsum("bhcd,bhc->bhd", S, q[:, t]) * scale
    return o, (S if output_final_state else None)


def chunk_local_cumsum(g: torch.Tensor, chunk: int) -> torch.Tensor:
    """Inclusive cumsum of ``g`` inside each chunk (``gdn2/reference.py:110-113``)."""
    B, T, H, D = g.shape
    return g.reshape(B, T // chunk, chunk, H, D).cumsum(2).reshape(B, T, H, D)


def strict_tril_pairwise(x, y, G, sub):
    """``M[r, s] = sum_c x_rc y_sc exp(G_rc - G_sc)`` for ``r > s``, zero elsewhere.

    Restates ``gdn2/reference.py:116-165``: off-diagonal ``sub x sub`` blocks
    factor through the decay at the first row of their row block, so both
    exponentials have non-positive arguments; diagonal blocks take the exact
    pairwise difference. ``x, y, G``: ``[..., BS, D]``.
    """
    *lead, BS, D = x.shape
    n = BS // sub
    out = x.new_zeros(*lead, BS, BS)
    strict = torch.ones(sub, sub, dtype=torch.bool).tril(-1)
    for i in range(n):
        rows = slice(i * sub, (i + 1) * sub)
        anchor = G[..., i * sub:i * sub + 1, :]
        xr = x[..., rows, :] * (G[..., rows, :] - anchor).exp()
        for j in range(i):
            cols = slice(j * sub, (j + 1) * sub)
            yc = y[..., cols, :] * (anchor - G[..., cols, :]).exp()
            out[..., rows, cols] = xr @ yc.transpose(-1, -2)
        diff = (G[..., rows, None, :] - G[..., None, rows, :]).clamp_max(0).exp()
        blk = torch.einsum("...rc,...sc,...rsc->...rs", x[..., rows, :], y[..., rows, :], diff)
        out[..., rows, rows] = torch.where(strict, blk, torch.zeros_like(blk))
    return out


def chunk_gdn2(q, k, v, g, b, w, scale=None, initial_state=None,
               output_final_state=False, chunk_size=64, sub_chunk_size=16,
               dtype=torch.float32):
    """Chunkwise WY form (``gdn2/reference.py:168-261``).

    Per chunk, with ``gamma = exp(G)`` and ``S`` the state entering it::

        Akk = strict_tril((b*k*gamma) (k/gamma)^T)    Ai = (I + Akk)^-1
        W = Ai (b*k*gamma)        U = Ai (w*v)        Un = U - W S
        Aqk = scale * tril(q k^T decay)  (diagonal included)
        o   = scale*(q*gamma) S + Aqk Un
        S'  = gamma_last * S + (k * gamma_last/gamma)^T Un
    """
    B, T, H, DK = q.shape
    DV = v.shape[-1]
    BS = chunk_size
    if T % BS:
        raise ValueError(f"sequence length {T} must be divisible by chunk_size {BS}")
    if BS % sub_chunk_size:
        raise ValueError(f"chunk_size {BS} must be divisible by sub_chunk_size {sub_chunk_size}")
    scale = DK ** -0.5 if scale is None else scale
    NC = T // BS
    q, k, v, g, b, w = (t.to(dtype) for t in (q, k, v, g, b, w))
    G = chunk_local_cumsum(g, BS)

    def chunks(x):  # [B, T, H, D] -> [B, H, NC, BS, D]
        return x.reshape(B, NC, BS, H, x.shape[-1]).permute(0, 3, 1, 2, 4)

    qc, kc, vc, Gc, bc, wc = (chunks(t) for t in (q, k, v, G, b, w))
    gamma = Gc.exp()
    E = bc * kc * gamma
    Akk = strict_tril_pairwise(bc * kc, kc, Gc, sub_chunk_size)
    eye = torch.eye(BS, dtype=dtype).expand_as(Akk)
    Ai = torch.linalg.solve_triangular(eye + Akk, eye, upper=False, unitriangular=True)
    W = Ai @ E
    U = Ai @ (wc * vc)
    Aqk = strict_tril_pairwise(qc, kc, Gc, sub_chunk_size)
    Aqk = (Aqk + torch.diag_embed((qc * kc).sum(-1))) * scale
    Qg = qc * gamma * scale
    KG = kc * (Gc[..., -1:, :] - Gc).exp()
    g_last = gamma[..., -1, :]

    S = torch.zeros(B, H, DK, DV, dtype=dtype) if initial_state is None \
        else initial_state.to(dtype).clone()
    o = torch.empty(B, H, NC, BS, DV, dtype=dtype)
    for n in range(NC):
        Un = U[:, :, n] - W[:, :, n] @ S
        o[:, :, n] = Qg[:, :, n] @ S + Aqk[:, :, n] @ Un
        S = g_last[:, :, n, :, None] * S + KG[:, :, n].transpose(-1, -2) @ Un
    o = o.permute(0, 2, 3, 1, 4).reshape(B, T, H, DV)
    return o, (S if output_final_state else None)


def decode_loop(q, k, v, g, b, w, state, scale=None):
    """``n`` tokens, ``state`` updated in place (``gdn2/inference.py:337-345``).

    Inputs ``[B, n, H, D]``; ``state`` fp32 ``[B, H, DK, DV]``. Returns ``o`` in
    ``v.dtype``, as the reference does.
    """
    DK = q.shape[-1]
    scale = DK ** -0.5 if scale is None else scale
    outs = []
    for t in range(q.shape[1]):
        state.mul_(g[:, t].float().exp()[..., None])
        erase = torch.einsum("bhcd,bhc->bhd", state, (b[:, t] * k[:, t]).float())
        u = (w[:, t] * v[:, t]).float() - erase
        state.add_(k[:, t].float()[..., None] * u[..., None, :])
        outs.append(torch.einsum("bhcd,bhc->bhd", state, q[:, t].float() * scale))
    return torch.stack(outs, 1).to(v.dtype)


def decode_step(q, k, v, g, b, w, state, scale=None):
    """One token in ``[B, H, D]`` layout (``gdn2/inference.py:183-189``)."""
    o = decode_loop(*(t.unsqueeze(1) for t in (q, k, v, g, b, w)), state, scale)
    return o[:, 0]


def prefill(q, k, v, g, b, w, state=None, scale=None, chunk_size=64, sub_chunk_size=16):
    """Prefill: whole chunks chunkwise, ragged tail through the decode loop
    (``gdn2/inference.py:517-539``). Returns ``(o, state)``."""
    B, S, H, DK = q.shape
    DV = v.shape[-1]
    scale = DK ** -0.5 if scale is None else scale
    n_full = (S // chunk_size) * chunk_size
    if state is None:
        state = torch.zeros(B, H, DK, DV)
    else:
        state = state.float().contiguous()
    outs = []
    if n_full:
        o1, state = chunk_gdn2(*(t[:, :n_full] for t in (q, k, v, g, b, w)), scale, state, True,
                               chunk_size=chunk_size, sub_chunk_size=sub_chunk_size)
        outs.append(o1)
    if S > n_full:
        outs.append(decode_loop(*(t[:, n_full:] for t in (q, k, v, g, b, w)), state, scale).float())
    return torch.cat(outs, 1), state
