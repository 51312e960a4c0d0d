"""KV-cache writer: NeoX RoPE on Q and K, K and V into the paged cache.

Drop-in for the reference's ``build_fused_rope_cache_module``
(kernels/fused_rope_cache_kernel.py:49-512): same builder parameters and
errors, and the returned ``launch_fused_rope_cache`` takes the same
arguments (Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache,
ValueCache, Q_out, K_out, num_tokens, KScale, VScale, stream).  The work is
one launch of the library's ``pa_fp8_rope_cache`` (flydsl_amd/csrc/
rope_cache.hip).

Layouts (``flash_layout``):
  * True:  KeyCache, ValueCache [num_blocks, block_size, KH, D]
  * False: KeyCache [num_blocks, KH, D/16, block_size, 16] and ValueCache
           [num_blocks, KH, D, block_size] -- the reference's ATOM layout --
           or ValueCache [num_blocks, KH, block_size/16, D, 16], the value
           layout the decode kernels read fastest (chosen by its rank).
With ``apply_scale`` the caches are fp8 e4m3fn (torch.float8_e4m3fn or
uint8) holding value / scale, saturated at +-448.

Differences from the reference, by design: head_dim must be a multiple of
16 in [16, 512] (the reference's flash layout also takes other even sizes,
such as 72, that its atom layouts reject); positions outside the cos/sin
tables are clamped into them and slots past the cache are skipped instead of
reading or writing out of bounds; the fp8 path saturates instead of writing
NaN for values beyond the fp8 range.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16}


def build_fused_rope_cache_module(
    head_dim: int = 64,
    rotary_dim: int = -1,
    num_q_heads: int = 8,
    num_kv_heads: int = 1,
    block_size: int = 16,
    is_neox: bool = True,
    flash_layout: bool = True,
    dtype_str: str = "bf16",
    apply_scale: bool = False,
    reuse_freqs_front_part: bool = True,
    pos_dtype: str = "i32",
):
    """Validate the configuration and return ``launch_fused_rope_cache``."""
    if rotary_dim == -1:
        rotary_dim = head_dim
    if not is_neox:
        raise NotImplementedError("Only NeoX-style RoPE is supported")
    if rotary_dim != head_dim:
        raise NotImplementedError("Partial rotation not yet supported")
    if dtype_str not in _DTYPES:
        raise ValueError(f"dtype_str must be 'bf16' or 'f16', got {dtype_str!r}")
    if rotary_dim % 2 != 0:
        raise ValueError(f"rotary_dim must be even, got {rotary_dim}")
    if head_dim % 16 != 0 or not 16 <= head_dim <= 512:
        raise ValueError(f"head_dim must be a multiple of 16 in [16, 512], got {head_dim}")
    if pos_dtype not in ("i32", "i64"):
        raise ValueError(f"pos_dtype must be 'i32' or 'i64', got {pos_dtype!r}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    dtype = _DTYPES[dtype_str]
    index_dtype = torch.int32 if pos_dtype == "i32" else torch.int64
    cos_cols = head_dim // 2 if reuse_freqs_front_part else head_dim
    D = head_dim

    def _check(name, t, shape, dt):
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
        if t.dtype not in (dt if isinstance(dt, tuple) else (dt,)):
            raise ValueError(f"{name} has dtype {t.dtype}")
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must be contiguous in its last dimension")

    def prepare(Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache, ValueCache, Q_out, K_out, num_tokens,
                KScale, VScale, stream=None):
        """Validate and marshal one call; ``.launch()`` then issues it with
        no further Python work (the tensors must stay alive)."""
        T = int(num_tokens)
        _check("Q", Q, (T, num_q_heads, D), dtype)
        _check("K", K, (T, num_kv_heads, D), dtype)
        _check("V", V, (T, num_kv_heads, D), dtype)
        _check("Q_out", Q_out, (T, num_q_heads, D), dtype)
        _check("K_out", K_out, (T, num_kv_heads, D), dtype)
        for name, t in (("Positions", Positions), ("SlotMapping", SlotMapping)):
            if t.dtype != index_dtype or t.dim() != 1 or t.shape[0] < T or t.stride(0) != 1:
                raise ValueError(f"{name} must be a contiguous {index_dtype} tensor of at least {T} entries")
        for name, t in (("CosCache", CosCache), ("SinCache", SinCache)):
            if t.dim() != 2 or t.shape[1] != cos_cols or t.dtype != dtype or t.stride(-1) != 1:
                raise ValueError(f"{name} must be [max_pos, {cos_cols}] {dtype} with a contiguous last dimension")
        if CosCache.shape[0] != SinCache.shape[0]:
            raise ValueError("CosCache and SinCache must have the same number of rows")
        cache_dt = (torch.float8_e4m3fn, torch.uint8) if apply_scale else (dtype,)
        nb = KeyCache.shape[0]
        if flash_layout:
            layout = _lib.CACHE_FLASH
            _check("KeyCache", KeyCache, (nb, block_size, num_kv_heads, D), cache_dt)
            _check("ValueCache", ValueCache, (nb, block_size, num_kv_heads, D), cache_dt)
        else:
            _check("KeyCache", KeyCache, (nb, num_kv_heads, D // 16, block_size, 16), cache_dt)
            if ValueCache.dim() == 5:
                if block_size % 16:
                    raise ValueError("a [NB, KH, bs/16, D, 16] value cache needs block_size % 16 == 0")
                layout = _lib.CACHE_ATOM_TRANS_V
                _check("ValueCache", ValueCache, (nb, num_kv_heads, block_size // 16, D, 16), cache_dt)
            else:
                layout = _lib.CACHE_ATOM
                _check("ValueCache", ValueCache, (nb, num_kv_heads, D, block_size), cache_dt)
        if not (KeyCache.is_contiguous() and ValueCache.is_contiguous()):
            raise ValueError("KeyCache and ValueCache must be contiguous")
        if apply_scale:
            for name, t in (("KScale", KScale), ("VScale", VScale)):
                if t is None or t.dtype != torch.float32 or t.numel() < 1:
                    raise ValueError(f"{name} must be a float32 tensor with at least one element")
        dev = Q.device
        tensors = [Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache, ValueCache, Q_out, K_out]
        if apply_scale:
            tensors += [KScale, VScale]
        for t in tensors:
            if t.device != dev:
                raise ValueError("all tensors must be on the same device")

        a = _lib.RopeCacheArgs()
        a.abi_version = _lib.ABI_VERSION
        a.q, a.k, a.v = Q.data_ptr(), K.data_ptr(), V.data_ptr()
        a.positions, a.slot_mapping = Positions.data_ptr(), SlotMapping.data_ptr()
        a.cos_cache, a.sin_cache = CosCache.data_ptr(), SinCache.data_ptr()
        a.key_cache, a.value_cache = KeyCache.data_ptr(), ValueCache.data_ptr()
        a.q_out, a.k_out = Q_out.data_ptr(), K_out.data_ptr()
        if apply_scale:
            a.k_scale, a.v_scale = KScale.data_ptr(), VScale.data_ptr()
        a.stride_q_tok, a.stride_q_head = Q.stride(0), Q.stride(1)
        a.stride_k_tok, a.stride_k_head = K.stride(0), K.stride(1)
        a.stride_v_tok, a.stride_v_head = V.stride(0), V.stride(1)
        a.stride_qo_tok, a.stride_qo_head = Q_out.stride(0), Q_out.stride(1)
        a.stride_ko_tok, a.stride_ko_head = K_out.stride(0), K_out.stride(1)
        a.stride_cos_pos, a.stride_sin_pos = CosCache.stride(0), SinCache.stride(0)
        a.num_tokens, a.num_q_heads, a.num_kv_heads, a.head_dim = T, num_q_heads, num_kv_heads, D
        a.block_size, a.num_blocks, a.max_pos = block_size, nb, CosCache.shape[0]
        a.dtype = _lib.DTYPE_BF16 if dtype_str == "bf16" else _lib.DTYPE_F16
        a.cache_layout = layout
        a.apply_scale = int(bool(apply_scale))
        a.reuse_freqs_front_part = int(bool(reuse_freqs_front_part))
        a.index_i64 = int(pos_dtype == "i64")
        if T == 0:  # no tokens: validated, nothing to launch
            return PreparedRopeCache(a, None, tuple(tensors))
        s = stream if stream is not None else torch.cuda.current_stream(dev)
        return PreparedRopeCache(a, s, tuple(tensors))

    def launch_fused_rope_cache(Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache, ValueCache, Q_out, K_out,
                                num_tokens, KScale, VScale, stream=None):
        prepare(Q, K, V, Positions, CosCache, SinCache, SlotMapping, KeyCache, ValueCache, Q_out, K_out, num_tokens,
                KScale, VScale, stream).launch()

    launch_fused_rope_cache.prepare = prepare
    return launch_fused_rope_cache


class PreparedRopeCache:
    """A validated writer call with its C-ABI arguments marshalled."""

    def __init__(self, args, stream, keepalive):
        self.args = args
        self._keep = keepalive
        if stream is None:  # zero tokens: launch() does nothing
            self._stream = self._lib = None
            return
        self._stream = ctypes.c_void_p(stream.cuda_stream)
        self._lib = _lib.load()

    def launch(self) -> None:
        if self._lib is None:
            return
        _lib.check(self._lib.pa_fp8_rope_cache(ctypes.byref(self.args), self._stream), "pa_fp8_rope_cache")
