"""Training-form forward entry point on the gfx950 kernels.

``chunk_gdn2_fwd`` keeps the reference's signature (``gdn2/forward.py:832-899``)
but runs the serving pipeline: the chunk-local kernel then the fused
scan + output kernel, so the per-chunk states ``h`` are never materialised
(the reference's ``state_kernel`` / ``output_kernel`` pair stores them only
for its backward, which this backend does not provide). A sequence that is
not a chunk multiple needs no padded copy (the reference zero-pads,
``gdn2/forward.py:748-753``): the kernels read the missing rows of the last
chunk as zeros, which are inert because g = 0 keeps the decay at 1 and
b = w = 0 removes both erase and write.
"""

from __future__ import annotations

import torch

from .config import DEFAULT_KERNEL_CONFIG, GDN2Config
from .inference import _check_shapes, _prefill_chunks, _require_device, _token_layout, check_prefill_config

__all__ = ["chunk_gdn2_fwd", "chunk_gdn2_bwd"]


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
    (q, k, v, g, b, w), s_alloc = _token_layout((q, k, v, g.float(), b, w))
    if initial_state is not None:
        _require_device(q, initial_state)
        initial_state = initial_state.to(torch.float32).contiguous()
    final = torch.empty(B, H, DK, DV, dtype=torch.float32, device=dev)
    o = torch.empty(B, S, H, DV, dtype=config.output_dtype or q.dtype, device=dev)
    if S:
        _prefill_chunks(q, k, v, g, b, w, initial_state, final, o, s_alloc, 0, S, scale)
    elif initial_state is not None:
        final.copy_(initial_state)
    else:
        final.zero_()
    return o, (final if output_final_state else None)


def chunk_gdn2_bwd(*args, **kwargs):
    """Not provided: the hip backend is a forward / serving backend."""
    raise NotImplementedError("the hip backend is forward-only; the GDN-2 backward is not implemented")
