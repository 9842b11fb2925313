"""Configuration objects (mirrors the reference's gdn2/config.py:22-89).

``GDN2Config`` says how the kernels run, ``GatedDeltaNet2Config`` what the
model is. Field names and defaults follow the reference so configs move
across unchanged. For the hip backend the tiling fields are fixed by the
gfx950 kernels: ``chunk_size`` must be 64 (the MFMA-tiled chunk) and
``sub_chunk_size`` only has to satisfy the reference's validity rules --
the kernels always rescale per 16-token block. ``output_dtype`` is an
addition: ``None`` keeps the reference behaviour (``o`` in ``v.dtype``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

__all__ = ["GDN2Config", "GatedDeltaNet2Config", "DEFAULT_KERNEL_CONFIG"]


@dataclass(frozen=True)
class GDN2Config:
    """Execution knobs. Nothing here changes the maths.

    Attributes:
        chunk_size: chunk length ``BS``; the hip kernels are built for 64.
        sub_chunk_size: ``BC``; must divide ``chunk_size`` with >= 2 blocks.
        block_DK, block_DV, threads, num_stages: accepted for compatibility
            with the reference's TileLang tiling; unused by the hip kernels.
        state_dtype: dtype of the state a call accepts and returns (fp32,
            bf16 or fp16): an initial state is first cast to it and the final
            state is returned in it, as in the reference; the kernels carry
            the state in fp32 between those two casts.
        backend: ``"auto"``, ``"hip"``, ``"tilelang"`` (the reference's GPU
            backend name; selects ``"hip"``) or ``"torch"``.
        backward: accepted for compatibility; autograd runs the hip backward.
        output_dtype: dtype of ``o``; ``None`` means ``v.dtype``.
    """

    chunk_size: int = 64
    sub_chunk_size: int = 16
    block_DK: int = 64
    block_DV: int = 64
    threads: int = 128
    num_stages: int = 2
    state_dtype: torch.dtype = torch.float32
    backend: str = "auto"
    backward: str = "torch"
    output_dtype: torch.dtype | None = None


DEFAULT_KERNEL_CONFIG = GDN2Config()


@dataclass
class GatedDeltaNet2Config:
    """Model configuration for :class:`GatedDeltaNet2` (reference config.py:55-89)."""

    hidden_size: int
    num_heads: int
    num_kv_heads: int | None = None
    head_dim_k: int = 128
    head_dim_v: int | None = None
    conv_size: int = 4
    norm_eps: float = 1e-5
    erase_gate_scale: float = 1.0
    a_init_range: tuple[float, float] = (1.0, 16.0)
    dt_init_range: tuple[float, float] = (0.001, 0.1)
    kernel: GDN2Config = field(default_factory=GDN2Config)
