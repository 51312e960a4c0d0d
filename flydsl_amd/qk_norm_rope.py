"""Fused per-token RMSNorm + GPT-J RoPE + optional FP8 quant of Q and KV.

Drop-in for kernels/qk_norm_rope_quant.py: :func:`flydsl_qk_norm_rope_quant`
(:739-955) keeps the reference's signature, validation errors and return
value, and :func:`compile_flydsl_qk_norm_rope_quant` (:709-736) returns a
cached launcher for callers that already hold every buffer.  The work is one
launch of the library's ``pa_fp8_qk_norm_rope_quant`` (flydsl_amd/csrc/
qk_norm_rope.hip): one wave per (token, head) row, Q heads and the KV row
of a token in the same launch.

Semantics (reference kernel :259-640): rstd = rsqrt(mean(x^2) + 1e-6) of the
unweighted bf16 row; Q rows are optionally weighted by ``q_weight``, the KV
row always by ``kv_weight``; the last ``rope_head_dim`` elements are rotated
in GPT-J pairs (2k, 2k+1) by cos/sin[position, k].  Without quant the
outputs are bf16 ``x * w * rstd`` (rotated).  With quant they are fp8
e4m3fn ``x * w * factor`` with one scale per ``quant_group_size`` elements:
float32 ``amax * rstd * sqrt2 / 448`` (factor ``448 / (sqrt2 * amax)``), or
an e8m0 exponent byte.

Differences from the reference, by design: head_dim may be 128, 256 or 512
(the reference kernel is built for 512 only); one launch covers any token
count (the reference splits at 65535 tokens for its grid); provided output
buffers must be contiguous (the reference writes them as dense without
checking).
"""

from __future__ import annotations

import ctypes
import functools
from typing import Optional, Tuple

import torch

from . import _lib

GROUP_SIZE_OPTIONS = (32, 64, 128)
SCALE_DTYPE_FP32 = "fp32"
SCALE_DTYPE_E8M0 = "e8m0"
SCALE_DTYPE_OPTIONS = (SCALE_DTYPE_FP32, SCALE_DTYPE_E8M0)
_TORCH_DTYPE_FOR_SCALE = {SCALE_DTYPE_FP32: torch.float32, SCALE_DTYPE_E8M0: torch.uint8}
FP8_DTYPE = torch.float8_e4m3fn  # gfx950's native fp8 (OCP e4m3fn)
LANES = 64  # one wave per row


def _check_config(H: int, D: int, RD: int, group_size: int, scale_dtype: str) -> None:
    """The kernel's shape rules (the reference asserts its own, :201-242)."""
    if D not in (128, 256, 512):
        raise AssertionError(f"head_dim={D} unsupported: 128, 256 or 512 (one wave of {LANES} lanes per row)")
    vec = D // LANES
    if H < 0:
        raise AssertionError(f"num_q_heads={H} must be non-negative")
    if RD % 2 != 0:
        raise AssertionError("rope_head_dim must be even (GPT-J pair layout)")
    if RD < 0 or RD > D or RD % vec != 0:
        raise AssertionError(f"RD={RD} must be a multiple of VEC={vec} no larger than head_dim={D}")
    if not (group_size > 0 and D % group_size == 0):
        raise AssertionError(f"group_size {group_size} must divide head_dim {D}")
    if group_size % vec != 0:
        raise AssertionError(f"group_size {group_size} must be a multiple of VEC {vec}")
    tpg = group_size // vec
    if tpg & (tpg - 1):
        raise AssertionError(f"TPG {tpg} must be a power of 2 (for butterfly reduce)")
    if scale_dtype not in SCALE_DTYPE_OPTIONS:
        raise AssertionError(f"scale_dtype {scale_dtype!r} must be one of {SCALE_DTYPE_OPTIONS}")


class QkNormRopeLauncher:
    """Launcher for one (H, D, RD, quant, group_size, scale_dtype, q_weighted)
    configuration: ``launcher(q_in, kv_in, q_weight, kv_weight, cos_cache,
    sin_cache, positions, q_out, kv_out, q_scale, kv_scale, kv_in_row_stride,
    num_tokens, stream=None)`` with the reference launcher's argument order
    (:650-665); tensors instead of raw pointers."""

    def __init__(self, H, D, RD, quant, group_size, scale_dtype, q_weighted):
        self.H, self.D, self.RD = H, D, RD
        self.quant, self.group_size, self.scale_dtype, self.q_weighted = quant, group_size, scale_dtype, q_weighted
        self._lib = _lib.load()

    def prepare(self, q_in, kv_in, q_weight, kv_weight, cos_cache, sin_cache, positions, q_out, kv_out, q_scale,
                kv_scale, kv_in_row_stride, num_tokens, stream=None) -> "PreparedQkNormRope":
        a = _lib.QkNormRopeArgs()
        a.abi_version = _lib.ABI_VERSION
        a.q, a.kv = q_in.data_ptr(), kv_in.data_ptr()
        a.q_weight = q_weight.data_ptr() if self.q_weighted else None
        a.kv_weight = kv_weight.data_ptr()
        a.cos_cache, a.sin_cache = cos_cache.data_ptr(), sin_cache.data_ptr()
        a.positions = positions.data_ptr()
        a.q_out, a.kv_out = q_out.data_ptr(), kv_out.data_ptr()
        if self.quant:
            a.q_scale, a.kv_scale = q_scale.data_ptr(), kv_scale.data_ptr()
        a.stride_q_tok = self.H * self.D if q_in.dim() != 3 else q_in.stride(0)
        a.stride_kv_tok = int(kv_in_row_stride)
        a.num_tokens, a.num_q_heads, a.head_dim, a.rope_head_dim = int(num_tokens), self.H, self.D, self.RD
        a.max_pos = cos_cache.shape[0]
        a.quant = int(bool(self.quant))
        a.group_size = self.group_size
        a.scale_e8m0 = int(self.quant and self.scale_dtype == SCALE_DTYPE_E8M0)
        s = stream if stream is not None else torch.cuda.current_stream(q_in.device)
        keep = (q_in, kv_in, q_weight, kv_weight, cos_cache, sin_cache, positions, q_out, kv_out, q_scale, kv_scale)
        return PreparedQkNormRope(self._lib, a, s, keep)

    def __call__(self, *args, stream=None) -> None:
        self.prepare(*args, stream=stream).launch()


class PreparedQkNormRope:
    """A marshalled call: ``launch()`` issues it with no further Python work."""

    def __init__(self, lib, args, stream, keepalive):
        self._lib = lib
        self.args = args
        self._stream = ctypes.c_void_p(stream.cuda_stream)
        self._keep = keepalive

    def launch(self) -> None:
        _lib.check(self._lib.pa_fp8_qk_norm_rope_quant(ctypes.byref(self.args), self._stream),
                   "pa_fp8_qk_norm_rope_quant")


@functools.lru_cache(maxsize=32)
def compile_flydsl_qk_norm_rope_quant(*, num_q_heads: int, head_dim: int, rope_head_dim: int, quant: bool,
                                      group_size: int, scale_dtype: str, q_weighted: bool) -> QkNormRopeLauncher:
    """Validated, cached launcher for one configuration (reference :709-736)."""
    _check_config(num_q_heads, head_dim, rope_head_dim, group_size, scale_dtype)
    return QkNormRopeLauncher(num_q_heads, head_dim, rope_head_dim, quant, group_size, scale_dtype, q_weighted)


def flydsl_qk_norm_rope_quant(
    q: torch.Tensor,
    kv: torch.Tensor,
    kv_weight: torch.Tensor,
    cos_cache: torch.Tensor,
    sin_cache: torch.Tensor,
    positions: torch.Tensor,
    *,
    num_q_heads: int,
    head_dim: int,
    rope_head_dim: int,
    q_weight: Optional[torch.Tensor] = None,
    quant: bool = False,
    quant_group_size: Optional[int] = None,
    scale_dtype: str = SCALE_DTYPE_FP32,
    q_out: Optional[torch.Tensor] = None,
    kv_out: Optional[torch.Tensor] = None,
    q_scale: Optional[torch.Tensor] = None,
    kv_scale: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Fused RMSNorm + GPT-J RoPE + optional FP8 quant for Q and KV in one
    launch (reference :739-955).  Returns ``(q_out [T, H, D], kv_out [T, D],
    q_scale [T, H, NG] or None, kv_scale [T, NG] or None)``."""
    if q.dtype != torch.bfloat16:
        raise TypeError(f"q must be bf16, got {q.dtype}")
    if kv.dtype != torch.bfloat16:
        raise TypeError(f"kv must be bf16, got {kv.dtype}")
    if kv_weight.dtype != torch.bfloat16:
        raise TypeError(f"kv_weight must be bf16, got {kv_weight.dtype}")
    if kv.stride(-1) != 1:
        raise ValueError(f"kv must be dense in the last dim, stride={kv.stride()}")
    if kv.stride(0) % 2 != 0:
        raise ValueError(
            "kv row stride (in bf16 elements) must be even for dword-cast "
            f"buffer loads, got kv.stride(0)={kv.stride(0)}"
        )
    if positions.dtype != torch.int64:
        raise TypeError(f"positions must be int64, got {positions.dtype}")
    if scale_dtype not in SCALE_DTYPE_OPTIONS:
        raise ValueError(f"scale_dtype {scale_dtype!r} not in {SCALE_DTYPE_OPTIONS}")
    if q_weight is not None and q_weight.dtype != torch.bfloat16:
        raise TypeError(f"q_weight must be bf16, got {q_weight.dtype}")

    H, D, RD = num_q_heads, head_dim, rope_head_dim
    T_tok = q.shape[0]
    G = quant_group_size if quant_group_size is not None else D
    NG = D // G
    if D % G != 0:
        raise ValueError(f"head_dim {D} must be divisible by quant_group_size {G}")
    q_weighted = q_weight is not None

    if q.dim() == 2:
        if q.shape[1] != H * D:
            raise ValueError(f"q shape {tuple(q.shape)} != [T, H*D={H*D}]")
        if not q.is_contiguous():
            raise ValueError("2D q must be contiguous to .view as [T,H,D]")
        q_view = q.view(T_tok, H, D)
    else:
        if q.dim() != 3 or q.shape != (T_tok, H, D):
            raise ValueError(f"q shape {tuple(q.shape)} != (T, H, D)=({T_tok}, {H}, {D})")
        q_view = q
        if q_view.stride(-1) != 1 or q_view.stride(-2) != D:
            raise ValueError(
                "3D q must be contiguous in the (H, D) inner block "
                f"(stride(-1)==1 and stride(-2)==D={D}), got stride={q_view.stride()}"
            )

    if cos_cache.shape[-1] != RD // 2:
        raise ValueError(f"cos_cache last dim {cos_cache.shape[-1]} != RD/2 ({RD // 2})")
    if sin_cache.shape != cos_cache.shape:
        raise ValueError("cos/sin shape mismatch")
    if not (cos_cache.is_contiguous() and sin_cache.is_contiguous()):
        raise ValueError("cos/sin must be contiguous")
    cos_2d = cos_cache.view(cos_cache.shape[0], RD // 2)
    sin_2d = sin_cache.view(sin_cache.shape[0], RD // 2)
    if cos_2d.dtype != torch.bfloat16 or sin_2d.dtype != torch.bfloat16:
        raise TypeError(f"cos/sin must be bf16, got {cos_2d.dtype}")
    if kv.dim() != 2 or kv.shape[1] != D or kv.shape[0] < T_tok:
        raise ValueError(f"kv shape {tuple(kv.shape)} != [T, D={D}]")
    if positions.dim() != 1 or positions.shape[0] < T_tok or not positions.is_contiguous():
        raise ValueError(f"positions must be a contiguous [T={T_tok}] tensor")
    for name, w in (("kv_weight", kv_weight), ("q_weight", q_weight)):
        if w is not None and (w.numel() != D or not w.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous [{D}] tensor")

    out_dtype = FP8_DTYPE if quant else torch.bfloat16
    if q_out is None:
        q_out = torch.empty((T_tok, H, D), dtype=out_dtype, device=q.device)
    if kv_out is None:
        kv_out = torch.empty((T_tok, D), dtype=out_dtype, device=kv.device)
    for name, t, shape in (("q_out", q_out, (T_tok, H, D)), ("kv_out", kv_out, (T_tok, D))):
        if t.numel() != T_tok * (H * D if name == "q_out" else D) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous tensor of shape {shape}")
        if t.element_size() != (1 if quant else 2):
            raise ValueError(f"{name} must be {'fp8' if quant else 'bf16'}, got {t.dtype}")

    scale_torch_dtype = _TORCH_DTYPE_FOR_SCALE[scale_dtype]
    if quant:
        if q_scale is None:
            q_scale = torch.empty((T_tok, H, NG), dtype=scale_torch_dtype, device=q.device)
        if kv_scale is None:
            kv_scale = torch.empty((T_tok, NG), dtype=scale_torch_dtype, device=kv.device)
        for name, t, n in (("q_scale", q_scale, T_tok * H * NG), ("kv_scale", kv_scale, T_tok * NG)):
            if t.numel() != n or not t.is_contiguous() or t.dtype != scale_torch_dtype:
                raise ValueError(f"{name} must be a contiguous {scale_torch_dtype} tensor of {n} elements")

    launcher = compile_flydsl_qk_norm_rope_quant(
        num_q_heads=H, head_dim=D, rope_head_dim=RD, quant=quant, group_size=G, scale_dtype=scale_dtype,
        q_weighted=q_weighted,
    )
    if T_tok > 0:
        launcher(q_view, kv, q_weight if q_weighted else kv_weight, kv_weight, cos_2d, sin_2d, positions, q_out,
                 kv_out, q_scale, kv_scale, kv.stride(0), T_tok, stream=stream)
    return q_out, kv_out, (q_scale if quant else None), (kv_scale if quant else None)
