"""CPU oracle for the GDN-2 attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the timed
CPU baseline. The product package ``gdt2_tilelang_amd`` never imports it: on a
GPU the HIP library runs or the call fails loudly.
"""

from .gdn2_oracle import (  # noqa: F401
    chunk_gdn2,
    chunk_local_cumsum,
    decode_loop,
    decode_step,
    make_inputs,
    make_config_inputs,
    prefill,
    recurrent_gdn2,
    rel_err,
    strict_tril_pairwise,
)
from .layer_oracle import LayerOracle  # noqa: F401
