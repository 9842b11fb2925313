"""MI355X-native (gfx950 HIP) backend for Gated DeltaNet-2 attention.

Drop-in for the reference ``gdn2`` package's forward / serving path:

    from gdt2_tilelang_amd import GatedDeltaNet2, GatedDeltaNet2Config
    from gdt2_tilelang_amd import gdn2_attention, gdn2_prefill, gdn2_decode

Module layout::

    config.py      GDN2Config / GatedDeltaNet2Config
    attention.py   gdn2_attention, resolve_backend, GDN2Cache, GatedDeltaNet2
    inference.py   gdn2_prefill, gdn2_decode, gdn2_decode_step
    forward.py     chunk_gdn2_fwd (fused scan; no per-chunk states), chunk_gdn2_bwd
    _hip.py        ctypes binding of _lib/libgdn2_hip.so (include/gdn2_hip.h)
    build.py       hipcc build of csrc/*.hip for gfx950
    csrc/          the HIP kernels and the C ABI

The reference's torch oracles (``recurrent_gdn2``, ``chunk_gdn2_torch``) are
not part of this package.
"""

from .attention import GDN2Cache, GatedDeltaNet2, gdn2_attention, resolve_backend
from .config import DEFAULT_KERNEL_CONFIG, GDN2Config, GatedDeltaNet2Config
from .forward import chunk_gdn2_bwd, chunk_gdn2_fwd, chunk_gdn2_varlen_bwd, chunk_gdn2_varlen_fwd
from .inference import gdn2_decode, gdn2_decode_step, gdn2_prefill

__all__ = [
    "GatedDeltaNet2",
    "GatedDeltaNet2Config",
    "GDN2Cache",
    "gdn2_attention",
    "gdn2_prefill",
    "gdn2_decode",
    "gdn2_decode_step",
    "GDN2Config",
    "DEFAULT_KERNEL_CONFIG",
    "chunk_gdn2_fwd",
    "chunk_gdn2_varlen_fwd",
    "chunk_gdn2_bwd",
    "chunk_gdn2_varlen_bwd",
    "resolve_backend",
]
