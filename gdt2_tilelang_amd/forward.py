"""Training-form forward entry point on the gfx950 kernels.

``chunk_gdn2_fwd`` keeps the reference's signature (``gdn2/forward.py:832-899``)
but runs the serving pipeline: the chunk-local kernel then the fused
scan + output kernel, so the per-chunk states ``h`` are never materialised
(the reference's ``state_kernel`` / ``output_kernel`` pair stores them only
for its backward; ``chunk_gdn2_bwd`` here recomputes what it needs). A sequence that is
not a chunk multiple needs no padded copy (the reference zero-pads,
``gdn2/forward.py:748-753``): the kernels read the missing rows of the last
chunk as zeros, which are inert because g = 0 keeps the decay at 1 and
b = w = 0 removes both erase and write.
"""

from __future__ import annotations

import torch

from . import _hip
from .config import DEFAULT_KERNEL_CONFIG, GDN2Config
from .inference import _check_shapes, _prefill_chunks, _require_device, _token_layout, check_prefill_config

__all__ = ["chunk_gdn2_fwd", "chunk_gdn2_varlen_fwd", "chunk_gdn2_bwd", "chunk_gdn2_varlen_bwd"]


@torch.no_grad()
def chunk_gdn2_fwd(q, k, v, g, b, w, scale, initial_state=None, output_final_state=False,
                   config: GDN2Config = DEFAULT_KERNEL_CONFIG, return_intermediates=False):
    """Chunkwise forward; returns ``(o [B, S, H, DV], final_state or None)``.

    ``o`` is in ``config.output_dtype`` or, as in the reference, ``q.dtype``.
    ``initial_state`` is read, never modified.
    """
    if return_intermediates:
        raise NotImplementedError("return_intermediates is not provided: chunk_gdn2_bwd recomputes what it needs")
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
        # the reference casts to config.state_dtype first (forward.py:874-877)
        initial_state = initial_state.to(config.state_dtype).to(torch.float32).contiguous()
    final = torch.empty(B, H, DK, DV, dtype=torch.float32, device=dev)
    o = torch.empty(B, S, H, DV, dtype=config.output_dtype or q.dtype, device=dev)
    if S:
        _prefill_chunks(q, k, v, g, b, w, initial_state, final, o, s_alloc, 0, S, scale)
    elif initial_state is not None:
        final.copy_(initial_state)
    else:
        final.zero_()
    if config.state_dtype != torch.float32:
        final = final.to(config.state_dtype)
    return o, (final if output_final_state else None)


def check_cu_seqlens(cu_seqlens, T: int) -> torch.Tensor:
    """Validate packed-sequence offsets on the host; returns them as int32 on
    the host. ``cu_seqlens`` is a 1-D integer tensor ``[N + 1]`` with
    ``cu[0] == 0``, ``cu[N] == T`` and non-decreasing entries (empty sequences
    allowed), the convention of packed-batch kernels (FLA ``cu_seqlens``)."""
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D tensor of N + 1 offsets (N >= 1)")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"cu_seqlens must be int32 or int64; got {cu_seqlens.dtype}")
    cu = cu_seqlens.detach().to("cpu", torch.int64)
    if int(cu[0]) != 0 or int(cu[-1]) != T:
        raise ValueError(f"cu_seqlens must start at 0 and end at the packed length {T}; "
                         f"got {int(cu[0])} .. {int(cu[-1])}")
    if bool((cu[1:] < cu[:-1]).any()):
        raise ValueError("cu_seqlens must be non-decreasing")
    return cu.to(torch.int32)


@torch.no_grad()
def chunk_gdn2_varlen_fwd(q, k, v, g, b, w, scale, cu_seqlens, initial_state=None, output_final_state=False,
                          config: GDN2Config = DEFAULT_KERNEL_CONFIG):
    """Packed variable-length forward: N sequences concatenated along one
    ``[1, T, H, D]`` batch row, sequence i holding tokens
    ``cu_seqlens[i] : cu_seqlens[i + 1]``, each an independent recurrence.

    Args:
        q, k, b, g: ``[1, T, HK, DK]``; v, w: ``[1, T, H, DV]``.
        cu_seqlens: ``[N + 1]`` int32 / int64 offsets (see ``check_cu_seqlens``).
        initial_state: ``[N, H, DK, DV]`` or ``None`` (zeros); never modified.

    Returns:
        ``(o [1, T, H, DV], final_state [N, H, DK, DV] in config.state_dtype or None)``. Both
        kernels run once for the whole batch; sequence i's result equals a
        separate call on its tokens alone.
    """
    dev = _require_device(q, k, v, g, b, w)
    _check_shapes(q, k, v, g, b, w)
    check_prefill_config(config)
    B, T, HK, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    if B != 1:
        raise ValueError(f"packed sequences (cu_seqlens) need batch size 1; got {B}")
    if DK not in (64, 128) or DV % 32:
        raise ValueError(f"hip prefill supports DK in (64, 128) and DV % 32 == 0; got DK={DK}, DV={DV}")
    cu = check_cu_seqlens(cu_seqlens, T).to(dev, non_blocking=False)
    N = cu.numel() - 1
    (q, k, v, g, b, w), _ = _token_layout((q, k, v, g.float(), b, w))
    if initial_state is not None:
        _require_device(q, initial_state)
        if tuple(initial_state.shape) != (N, H, DK, DV):
            raise ValueError(f"initial_state has shape {tuple(initial_state.shape)}, expected {(N, H, DK, DV)}")
        initial_state = initial_state.to(config.state_dtype).to(torch.float32).contiguous()
    final = torch.empty(N, H, DK, DV, dtype=torch.float32, device=dev)
    o = torch.empty(1, T, H, DV, dtype=config.output_dtype or q.dtype, device=dev)
    st_dt = config.state_dtype
    if T == 0:                          # every sequence empty: the states pass through
        if initial_state is not None:
            final.copy_(initial_state)
        else:
            final.zero_()
        return o, (final.to(st_dt) if output_final_state else None)
    lib = _hip.lib()
    ws = torch.empty(lib.gdn2_hip_prefill_varlen_workspace_bytes(N, HK, DK, T), dtype=torch.uint8, device=dev)
    _hip.check(lib.gdn2_hip_prefill_varlen(
        _hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(g), _hip.ptr(b), _hip.ptr(w),
        _hip.dtype_code(q.dtype), _hip.ptr(cu), N, _hip.ptr(initial_state), _hip.ptr(final), _hip.ptr(o),
        _hip.dtype_code(o.dtype), _hip.ptr(ws), H, HK, DK, DV, T, float(scale),
        _hip.stream_of(dev)), "gdn2_hip_prefill_varlen")
    return o, (final.to(st_dt) if output_final_state else None)


def _check_state_arg(name, t, shape, dev):
    """A per-sequence state argument (initial state or final-state gradient):
    None, or a tensor of ``shape`` on the op's device."""
    if t is None:
        return
    if t.device != dev:
        raise ValueError(f"all tensors must be on {dev}; got {t.device} for {name}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def chunk_gdn2_bwd(q, k, v, g, b, w, scale, initial_state, do, dht, config: GDN2Config = DEFAULT_KERNEL_CONFIG):
    """Chunkwise training backward on the gfx950 kernels.

    Same contract as the reference (``gdn2/backward.py:912-994``): the
    gradients of ``(o * do).sum() + (final_state * dht).sum()`` with respect
    to the forward inputs. Returns ``(dq, dk, dv, dg, db, dw, dinitial_state)``;
    the last is ``None`` when ``initial_state`` is ``None``. Each gradient has
    its input's dtype. The arithmetic is fp32 throughout (chunk 64):
    ``gdn2_hip_backward`` recomputes the per-chunk factors, scans the
    chunk-entry states forward and the state gradients backward, then forms
    every chunk's gradients in parallel.
    """
    dev = _require_device(q, k, v, g, b, w, do)
    _check_shapes(q, k, v, g, b, w)
    B, S, HK, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    if DK not in (32, 64, 128) or DV % 16:
        raise ValueError(f"hip backward supports DK in (32, 64, 128) and DV % 16 == 0; got DK={DK}, DV={DV}")
    if tuple(do.shape) != (B, S, H, DV):
        raise ValueError(f"do has shape {tuple(do.shape)}, expected {(B, S, H, DV)}")
    _check_state_arg("initial_state", initial_state, (B, H, DK, DV), dev)
    _check_state_arg("dht", dht, (B, H, DK, DV), dev)
    scale = DK ** -0.5 if scale is None else scale
    q, k, v, b, w, do = (t.contiguous() for t in (q, k, v, b, w, do))
    g32 = g.float().contiguous()
    s0 = None
    if initial_state is not None:
        _require_device(q, initial_state)
        s0 = initial_state.to(config.state_dtype).to(torch.float32).contiguous()
    dht32 = None if dht is None else dht.to(torch.float32).contiguous()
    dq, dk, db = (torch.empty(B, S, HK, DK, dtype=q.dtype, device=dev) for _ in range(3))
    dv, dw = (torch.empty(B, S, H, DV, dtype=q.dtype, device=dev) for _ in range(2))
    dg = torch.empty(B, S, HK, DK, dtype=torch.float32, device=dev)
    ds0 = None if s0 is None else torch.empty(B, H, DK, DV, dtype=torch.float32, device=dev)
    lib = _hip.lib()
    ws = torch.empty(max(lib.gdn2_hip_backward_workspace_bytes(B, H, HK, DK, DV, S), 1), dtype=torch.uint8,
                     device=dev)
    _hip.check(lib.gdn2_hip_backward(
        _hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(g32), _hip.ptr(b), _hip.ptr(w), _hip.dtype_code(q.dtype),
        float(scale), _hip.ptr(s0), _hip.ptr(do), _hip.dtype_code(do.dtype), _hip.ptr(dht32),
        _hip.ptr(dq), _hip.ptr(dk), _hip.ptr(dv), _hip.ptr(dg), _hip.ptr(db), _hip.ptr(dw), _hip.ptr(ds0),
        _hip.ptr(ws), B, S, H, HK, DK, DV, _hip.stream_of(dev)), "gdn2_hip_backward")
    return (dq, dk, dv, dg.to(g.dtype), db, dw,
            None if ds0 is None else ds0.to(initial_state.dtype))


def chunk_gdn2_varlen_bwd(q, k, v, g, b, w, scale, cu_seqlens, initial_state, do, dht,
                          config: GDN2Config = DEFAULT_KERNEL_CONFIG):
    """Backward of ``chunk_gdn2_varlen_fwd``: each packed sequence is an
    independent recurrence and gets the gradients of its own tokens and
    initial state (an empty sequence passes its final-state gradient through
    to its initial state). All sequences run in one ``gdn2_hip_backward_varlen``
    call: the per-chunk kernels take the forward's record slots and the scans
    run per (sequence, value head, column tile).

    Returns ``(dq, dk, dv, dg, db, dw, dinitial_state [N, H, DK, DV] or None)``.
    """
    dev = _require_device(q, k, v, g, b, w, do)
    _check_shapes(q, k, v, g, b, w)
    B, T, HK, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    if B != 1:
        raise ValueError(f"packed sequences (cu_seqlens) need batch size 1; got {B}")
    if DK not in (32, 64, 128) or DV % 16:
        raise ValueError(f"hip backward supports DK in (32, 64, 128) and DV % 16 == 0; got DK={DK}, DV={DV}")
    if tuple(do.shape) != (1, T, H, DV):
        raise ValueError(f"do has shape {tuple(do.shape)}, expected {(1, T, H, DV)}")
    cu = check_cu_seqlens(cu_seqlens, T).to(dev)
    N = cu.numel() - 1
    scale = DK ** -0.5 if scale is None else scale
    q, k, v, b, w, do = (t.contiguous() for t in (q, k, v, b, w, do))
    g32 = g.float().contiguous()
    _check_state_arg("initial_state", initial_state, (N, H, DK, DV), dev)
    _check_state_arg("dht", dht, (N, H, DK, DV), dev)
    s0 = None
    if initial_state is not None:
        s0 = initial_state.to(config.state_dtype).to(torch.float32).contiguous()
    dht32 = None if dht is None else dht.to(torch.float32).contiguous()
    dq, dk, db = (torch.empty(1, T, HK, DK, dtype=q.dtype, device=dev) for _ in range(3))
    dv, dw = (torch.empty(1, T, H, DV, dtype=q.dtype, device=dev) for _ in range(2))
    dg = torch.empty(1, T, HK, DK, dtype=torch.float32, device=dev)
    ds0 = None if s0 is None else torch.empty(N, H, DK, DV, dtype=torch.float32, device=dev)
    lib = _hip.lib()
    ws = torch.empty(max(lib.gdn2_hip_backward_varlen_workspace_bytes(N, H, HK, DK, DV, T), 1),
                     dtype=torch.uint8, device=dev)
    _hip.check(lib.gdn2_hip_backward_varlen(
        _hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(g32), _hip.ptr(b), _hip.ptr(w), _hip.dtype_code(q.dtype),
        float(scale), _hip.ptr(s0), _hip.ptr(do), _hip.dtype_code(do.dtype), _hip.ptr(dht32),
        _hip.ptr(dq), _hip.ptr(dk), _hip.ptr(dv), _hip.ptr(dg), _hip.ptr(db), _hip.ptr(dw), _hip.ptr(ds0),
        _hip.ptr(ws), _hip.ptr(cu), N, T, H, HK, DK, DV, _hip.stream_of(dev)), "gdn2_hip_backward_varlen")
    return (dq, dk, dv, dg.to(g.dtype), db, dw,
            None if ds0 is None else ds0.to(initial_state.dtype))
