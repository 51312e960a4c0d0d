"""MI355X-native FP8 paged-attention decode (drop-in for FlyDSL's pa_decode_ps_launch).

Public API (same names and signatures as kernels/pa_decode_fp8.py of the
reference): :func:`pa_decode_ps_launch`, :func:`get_recommended_splits`,
:func:`get_pa_metadata`.  Device work runs in the hand-written gfx950 HIP
kernels of ``libpa_fp8.so`` (C ABI: ``include/pa_fp8.h``).
"""

from .pa_decode import (  # noqa: F401
    KV_COMPUTE_BLOCK,
    PreparedDecode,
    get_pa_metadata,
    get_recommended_splits,
    pa_decode_ps_launch,
    prepare_pa_decode,
)

__all__ = [
    "pa_decode_ps_launch",
    "get_recommended_splits",
    "get_pa_metadata",
    "prepare_pa_decode",
    "PreparedDecode",
    "KV_COMPUTE_BLOCK",
]
