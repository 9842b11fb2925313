"""Serving entry points on the gfx950 kernels: prefill and decode.

Mirrors the reference's ``gdn2/inference.py`` API:

    gdn2_prefill(q, k, v, g, b, w, state=None, scale=None, config)  -> (o, state)
    gdn2_decode(q, k, v, g, b, w, state, scale=None)                  -> o  (state in place)
    gdn2_decode_step(q, k, v, g, b, w, state, scale=None)             -> o  ([B, H, D] layout)

Prefill runs the prompt's 64-token chunks through the two prefill kernels
(chunk-local WY stage, then the fused state scan + output that never
materialises the per-chunk states); a ragged tail rides along as a last, partly
filled chunk whose missing rows the kernels read as zeros. The reference sends
that tail through its decode kernel instead (``gdn2/inference.py:517-555``);
both compute the same recurrence, and a prompt shorter than one chunk still
goes through decode with the state updated in place, as in the reference.
Decode keeps the state resident across the ``n`` tokens of a call.

Grouped heads: q, k, b, g may carry HK key heads where v, w (and the state)
carry H value heads, HK dividing H; value head h then reads key head
h // (H // HK), which equals the reference's ``repeat_interleave`` expansion
(``gdn2/attention.py:295-297``) without materialising it. With HK == H the
calls are exactly the reference's.

Every call enqueues on the current HIP stream and returns without syncing.
There is no CPU path: CPU tensors raise ``ValueError``.
"""

from __future__ import annotations

import torch

from . import _hip
from .config import DEFAULT_KERNEL_CONFIG, GDN2Config

__all__ = ["gdn2_prefill", "gdn2_decode", "gdn2_decode_step", "check_state_dtype"]

_PREFILL_DK = (64, 128)
_DECODE_DK = (32, 64, 128, 256)


def _require_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError("backend 'hip' requires a CUDA device (a ROCm GPU); got CPU tensors")
    for t in ts:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}; got {t.device}")
    return dev


def _check_shapes(q, k, v, g, b, w):
    if q.dim() != 4:
        raise ValueError(f"expected [B, S, H, D] tensors, got q of shape {tuple(q.shape)}")
    for name, t in (("k", k), ("g", g), ("b", b)):
        if t.shape != q.shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(q.shape)}")
    if v.dim() != 4 or v.shape[:2] != q.shape[:2] or v.shape[2] % q.shape[2]:
        raise ValueError(f"v has shape {tuple(v.shape)}, incompatible with q {tuple(q.shape)} "
                         "(value heads must be a multiple of the key heads)")
    if w.shape != v.shape:
        raise ValueError(f"w has shape {tuple(w.shape)}, expected {tuple(v.shape)}")
    dts = {t.dtype for t in (q, k, v, b, w)}
    if len(dts) != 1:
        raise TypeError(f"q, k, v, b, w must share one dtype; got {sorted(map(str, dts))}")
    _hip.dtype_code(q.dtype)


def _token_layout(ts):
    """(tensors, s_alloc): every tensor as a contiguous [B, S, H, D] block.

    The kernels address token t of batch b at ``(b * s_alloc + t) * H * D``;
    contiguous inputs pass through untouched, anything else is copied.
    """
    return [t if t.is_contiguous() else t.contiguous() for t in ts], ts[0].shape[1]


_STATE_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def check_state_dtype(dt: torch.dtype) -> None:
    """The state dtypes the reference's kernels take (``_tl_dtype``,
    ``gdn2/forward.py:733-745``); anything else is a ``TypeError``."""
    if dt not in _STATE_DTYPES:
        raise TypeError(f"unsupported state dtype {dt}; use float32, bfloat16 or float16")


def _check_state(state, B, H, DK, DV, dev):
    if state.dtype != torch.float32:
        raise TypeError(f"the hip kernels carry an fp32 state; got {state.dtype}")
    if tuple(state.shape) != (B, H, DK, DV):
        raise ValueError(f"state has shape {tuple(state.shape)}, expected {(B, H, DK, DV)}")
    if state.device != dev:
        raise ValueError(f"state must be on {dev}")


def _decode_into(q, k, v, g, b, w, state, o, s_alloc, t0, n, scale):
    B, _, HK, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    if DK not in _DECODE_DK or DV % 32:
        raise ValueError(f"hip decode supports DK in {_DECODE_DK} and DV % 32 == 0; got DK={DK}, DV={DV}")
    _hip.check(_hip.lib().gdn2_hip_decode(
        _hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(g), _hip.ptr(b), _hip.ptr(w),
        _hip.dtype_code(q.dtype), _hip.ptr(state), _hip.ptr(o), _hip.dtype_code(o.dtype),
        B, H, HK, DK, DV, s_alloc, t0, n, float(scale), _hip.stream_of(q.device)), "gdn2_hip_decode")


def gdn2_decode(q, k, v, g, b, w, state, scale=None):
    """Decode ``n`` tokens, updating ``state`` in place.

    Args:
        q, k, b: ``[B, n, HK, DK]``; v, w: ``[B, n, H, DV]`` (fp32, bf16 or fp16);
            HK == H as in the reference, or HK dividing H (grouped heads).
        g: ``[B, n, HK, DK]`` log decay (<= 0), used as fp32.
        state: contiguous ``[B, H, DK, DV]`` (fp32, or bf16 / fp16 as the
            reference's kernels also take), mutated. The kernel carries it in
            fp32 across the call's tokens; a bf16 / fp16 state is rounded back
            once at the end, as the reference's kernel stores it.
        scale: query scale; defaults to ``DK ** -0.5``.

    Returns:
        ``[B, n, H, DV]`` outputs in ``v.dtype``.
    """
    dev = _require_device(q, k, v, g, b, w, state)
    _check_shapes(q, k, v, g, b, w)
    B, n, _, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    check_state_dtype(state.dtype)
    work = state if state.dtype == torch.float32 else state.float()
    _check_state(work, B, H, DK, DV, dev)
    if not state.is_contiguous():
        raise ValueError("state must be contiguous (it is updated in place)")
    scale = DK ** -0.5 if scale is None else scale
    g = g.float()
    (q, k, v, g, b, w), s_alloc = _token_layout((q, k, v, g, b, w))
    o = torch.empty(B, s_alloc, H, DV, dtype=v.dtype, device=dev)
    if n:
        _decode_into(q, k, v, g, b, w, work, o, s_alloc, 0, n, scale)
        if work is not state:
            state.copy_(work)
    return o


def gdn2_decode_step(q, k, v, g, b, w, state, scale=None):
    """One autoregressive step; inputs ``[B, H, D]``, ``state`` updated in place.

    Returns ``[B, H, DV]`` in ``v.dtype``.
    """
    if q.dim() != 3:
        raise ValueError(f"expected [B, H, D] inputs, got q of shape {tuple(q.shape)}")
    o = gdn2_decode(*(t.unsqueeze(1) for t in (q, k, v, g, b, w)), state, scale)
    return o[:, 0]


def _prefill_chunks(q, k, v, g, b, w, state_in, state_out, o, s_alloc, t0, n_tokens, scale):
    B, _, HK, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    nbytes = _hip.lib().gdn2_hip_prefill_workspace_bytes(B, HK, DK, n_tokens)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    _hip.check(_hip.lib().gdn2_hip_prefill_chunks(
        _hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(g), _hip.ptr(b), _hip.ptr(w),
        _hip.dtype_code(q.dtype), _hip.ptr(state_in), _hip.ptr(state_out), _hip.ptr(o),
        _hip.dtype_code(o.dtype), _hip.ptr(ws), B, H, HK, DK, DV, s_alloc, t0, n_tokens,
        float(scale), _hip.stream_of(q.device)), "gdn2_hip_prefill_chunks")


def check_prefill_config(config: GDN2Config) -> None:
    """The reference's tiling validity rules plus the hip kernels' own."""
    BS, BC = config.chunk_size, config.sub_chunk_size
    if BS < 1 or BS & (BS - 1):
        raise ValueError(f"chunk_size must be a power of two, got {BS}")
    if BC < 1 or BS % BC:
        raise ValueError(f"chunk_size {BS} must be divisible by sub_chunk_size {BC}")
    if BS // BC < 2:
        raise ValueError(f"need at least 2 sub-chunks per chunk, got chunk {BS} / sub-chunk {BC}")
    if BS != 64:
        raise ValueError(f"the hip kernels are built for chunk_size 64, got {BS}")
    check_state_dtype(config.state_dtype)


@torch.no_grad()
def gdn2_prefill(q, k, v, g, b, w, state=None, scale=None, config: GDN2Config = DEFAULT_KERNEL_CONFIG):
    """Prefill a prompt; returns ``(o, state)`` to decode from.

    The prompt goes through the chunk-local kernel and the fused scan + output
    kernel, a ragged tail as a last, partly filled chunk (the reference runs
    the tail through its decode kernel, ``inference.py:537-553``; both compute
    the same recurrence). A prompt shorter than one chunk goes through the
    decode kernel.
    Call repeatedly, passing the state back, to prefill in segments.

    Args:
        q, k, b: ``[B, S, HK, DK]``; v, w: ``[B, S, H, DV]``; g: ``[B, S, HK, DK]``
            (HK == H as in the reference, or HK dividing H: grouped heads).
        state: ``[B, H, DK, DV]`` to continue from, or ``None`` for zeros. As in
            the reference it is first cast to ``config.state_dtype``, and a
            prompt shorter than one chunk updates that (contiguous) state in
            place, so a state already in ``state_dtype`` is mutated.
        scale: query scale; defaults to ``DK ** -0.5``.
        config: kernel configuration (``output_dtype`` selects the dtype of o).

    Returns:
        ``(o [B, S, H, DV], state [B, H, DK, DV])``, the state in
        ``config.state_dtype`` (the kernels compute in fp32 and round once).
    """
    dev = _require_device(q, k, v, g, b, w)
    _check_shapes(q, k, v, g, b, w)
    check_prefill_config(config)
    B, S, _, DK = q.shape
    H, DV = v.shape[2], v.shape[3]
    if DK not in _PREFILL_DK or DV % 32:
        raise ValueError(f"hip prefill supports DK in {_PREFILL_DK} and DV % 32 == 0; got DK={DK}, DV={DV}")
    scale = DK ** -0.5 if scale is None else scale
    BS = config.chunk_size
    n_full = (S // BS) * BS
    st_dt = config.state_dtype
    if state is None:
        state = torch.zeros(B, H, DK, DV, dtype=st_dt, device=dev)
    else:
        _require_device(q, state)
        state = state.to(st_dt).contiguous()
    work = state if st_dt == torch.float32 else state.float()
    _check_state(work, B, H, DK, DV, dev)
    out_dtype = config.output_dtype or v.dtype
    _hip.dtype_code(out_dtype)
    g = g.float()
    (q, k, v, g, b, w), s_alloc = _token_layout((q, k, v, g, b, w))
    o = torch.empty(B, s_alloc, H, DV, dtype=out_dtype, device=dev)
    if n_full:
        # the ragged tail rides along as a last, partly filled chunk (its missing
        # rows read as zeros, which the chunkwise form treats as inert)
        new_state = torch.empty_like(work)
        _prefill_chunks(q, k, v, g, b, w, work, new_state, o, s_alloc, 0, S, scale)
        state = new_state if st_dt == torch.float32 else new_state.to(st_dt)
    elif S:
        # shorter than one chunk: the recurrence, updating state in place as the
        # reference's decode path does
        _decode_into(q, k, v, g, b, w, work, o, s_alloc, 0, S, scale)
        if work is not state:
            state.copy_(work)
    return o, state
