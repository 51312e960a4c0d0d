"""MI355X-native FP8 paged-attention decode (drop-in for FlyDSL's pa_decode_ps_launch).

Public API (same names and signatures as the reference):
  * kernels/pa_decode_fp8.py: :func:`pa_decode_ps_launch`,
    :func:`get_recommended_splits`, :func:`get_pa_metadata`;
  * kernels/fused_rope_cache_kernel.py: :func:`build_fused_rope_cache_module`
    (the KV-cache writer that produces the cache the decode reads);
  * kernels/qk_norm_rope_quant.py: :func:`flydsl_qk_norm_rope_quant`,
    :func:`compile_flydsl_qk_norm_rope_quant` (fused RMSNorm + GPT-J RoPE +
    fp8 quant of Q and the KV row);
  * kernels/mla_fwd_decode.py: :func:`flydsl_mla_fwd_decode` (MLA fp8 decode),
    with :func:`get_mla_metadata_info_v1`, :func:`get_mla_metadata_v1` and
    :func:`mla_reduce_v1` in place of the aiter calls its test makes.
Device work runs in the hand-written gfx950 HIP kernels of ``libpa_fp8.so``
(C ABI: ``include/pa_fp8.h``).
"""

from .pa_decode import (  # noqa: F401
    KV_COMPUTE_BLOCK,
    PreparedDecode,
    get_pa_metadata,
    get_recommended_splits,
    pa_decode_ps_launch,
    prepare_pa_decode,
)
from .mla_decode import (  # noqa: F401
    flydsl_mla_fwd_decode,
    get_mla_metadata_info_v1,
    get_mla_metadata_v1,
    mla_reduce_v1,
)
from .qk_norm_rope import compile_flydsl_qk_norm_rope_quant, flydsl_qk_norm_rope_quant  # noqa: F401
from .rope_cache import build_fused_rope_cache_module  # noqa: F401

__all__ = [
    "pa_decode_ps_launch",
    "get_recommended_splits",
    "get_pa_metadata",
    "prepare_pa_decode",
    "PreparedDecode",
    "KV_COMPUTE_BLOCK",
    "build_fused_rope_cache_module",
    "flydsl_qk_norm_rope_quant",
    "compile_flydsl_qk_norm_rope_quant",
    "flydsl_mla_fwd_decode",
    "get_mla_metadata_info_v1",
    "get_mla_metadata_v1",
    "mla_reduce_v1",
]
