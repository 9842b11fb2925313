"""Training-form forward entry point on the gfx950 kernels.

``chunk_gdn2_fwd`` keeps the reference's signature (``gdn2/forward.py:832-899``)
but runs the serving pipeline: the chunk-local kernel then the fused
scan + output kernel, so the per-chunk states ``h`` are never materialised
(the reference's ``state_kernel`` / ``output_kernel`` pair stores them only
for its backward, which this backend does not provide). Sequences that are
not a chunk multiple are zero-padded; the padding is inert because g = 0
keeps the decay at 1 and b = w = 0 removes both erase and write.
"""

from __future__ import annotations

import torch

from .config import DEFAULT_KERNEL_CONFIG, GDN2Config
from .inference import _check_shapes, _prefill_chunks, _require_device, check_prefill_config

__all__ = ["chunk_gdn2_fwd", "chunk_gdn2_bwd"]


def _pad_to_chunk(x: torch.Tensor, total: int) -> torch.Tensor:
    """Right-pad the sequence axis of ``[B, S, H, D]`` with zeros to ``total``."""
    if x.shape[1] == total:
        return x.contiguous()
    pad = x.new_zeros(x.shape[0], total - x.shape[1], *x.shape[2:])
    return torch.cat([x, pad], dim=1)


@torch.no_grad()
def chunk_gdn2_fwd(q, k, v, g, b, w, scale, initial_state=None, output_final_state=False,
                   config: GDN2Config = DEFAULT_KERNEL_CONFIG, return_intermediates=False):
    """Chunkwise forward; returns ``(o [B, S, H, DV], final_state or None)``.

    ``o`` is in ``config.output_dtype`` or, as in the reference, ``q.dtype``.
    ``initial_state`` is read, never modified.
    """
    if return_intermediates:
        raise NotImplementedError("the hip backend is forward-only; it keeps no backward intermediates")
    dev = _require_device(q, k, v, g, b, w)
    _check_shapes(q, k, v, g, b, w)
    check_prefill_config(config)
    B, S, _, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    if DK not in (64, 128) or DV % 32:
        raise ValueError(f"hip prefill supports DK in (64, 128) and DV % 32 == 0; got DK={DK}, DV={DV}")
    BS = config.chunk_size
    S_pad = ((S + BS - 1) // BS) * BS
    q, k, v, b, w = (_pad_to_chunk(t, S_pad) for t in (q, k, v, b, w))
    g = _pad_to_chunk(g.float(), S_pad)
    if initial_state is not None:
        _require_device(q, initial_state)
        initial_state = initial_state.to(torch.float32).contiguous()
    final = torch.empty(B, H, DK, DV, dtype=torch.float32, device=dev)
    o = torch.empty(B, S_pad, H, DV, dtype=config.output_dtype or q.dtype, device=dev)
    if S_pad:
        _prefill_chunks(q, k, v, g, b, w, initial_state, final, o, S_pad, 0, S_pad, scale)
    elif initial_state is not None:
        final.copy_(initial_state)
    else:
        final.zero_()
    return o[:, :S], (final if output_final_state else None)


def chunk_gdn2_bwd(*args, **kwargs):
    """Not provided: the hip backend is a forward / serving backend."""
    raise NotImplementedError("the hip backend is forward-only; the GDN-2 backward is not implemented")
