"""CPU restatement of the fused per-token RMSNorm + GPT-J RoPE + optional
FP8 quant of Q and KV (test infrastructure only).

Follows kernels/qk_norm_rope_quant.py (the reference ships no test for it):

  * rows: every Q head row of x_q [T, H, D] (optionally weighted by
    q_weight, :545-555) and the KV row kv [T, D] (always weighted by
    kv_weight, :600-605); x in float32 from bf16;
  * RMSNorm statistic over the unweighted row (:330-331):
        rstd = rsqrt(sum(x^2) * (1/D) + 1e-6)                          (:364)
  * no quant: y = (x * w) * rstd                              (:439-444, :462-467)
  * fp32 quant (:394-405): amax over each group of G elements of |x * w|
    (|x| unweighted, :333-337), am = max(amax, 1e-12),
        factor = f32(448/sqrt2) * (1/am),  scale = am * rstd * f32(sqrt2/448),
        y = (x * w) * factor  (rstd cancels: y * scale = x * w * rstd);
  * e8m0 quant (:367-393): amax_post = am * rstd * f32(sqrt2),
        e = clamp(((bits(amax_post) + 0x400000) & 0xff800000) >> 23) - 7, 0, 255),
        factor = rstd * 2^(127 - e) (float bits (254 - e) << 23), stored byte e;
  * GPT-J rotation of the last RD elements (:425-456): pair (2k, 2k+1) of the
    rope part with cos[pos, k], sin[pos, k]:
        y[2k] = e*c - o*s,  y[2k+1] = e*s + o*c;
    positions outside the cos/sin table read zeros (the reference's buffer
    loads return 0 out of range);
  * stores: bf16 round to nearest even (:121-131), or e4m3fn bytes after
    clamping values in (-2^-8, 0) to +0 (:133-171).

Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline use this.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch

FP8_MAX = 448.0
SQRT2 = math.sqrt(2.0)
F32_MAX_OVER_SQRT2 = np.float32(FP8_MAX / SQRT2)
F32_INV_MAX_SQRT2 = np.float32(SQRT2 / FP8_MAX)
F32_SQRT2 = np.float32(SQRT2)
E8M0_HEADROOM = 7
EPS = np.float32(1e-6)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 (round to nearest even) -> float32, on the bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def fp8_bytes(y: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn bytes with the reference's small-negative clamp."""
    y = np.where((y < 0) & (y > -(2.0**-8)), np.float32(0.0), y).astype(np.float32)
    y = np.clip(y, -FP8_MAX, FP8_MAX)
    return torch.from_numpy(np.ascontiguousarray(y)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _rows(x, w, cos_rows, sin_rows, d, rd, quant, g, e8m0):
    """x [T, R, D] float32, w [D] float32 or None, cos/sin rows [T, RD/2]."""
    t, r, _ = x.shape
    f32 = np.float32
    sumsq = np.sum(x * x, axis=-1, dtype=np.float32)
    rstd = (f32(1.0) / np.sqrt(sumsq * f32(1.0 / d) + EPS)).astype(np.float32)
    xw = (x * w).astype(np.float32) if w is not None else x
    scale = None
    if quant:
        ng = d // g
        am = np.max(np.abs(xw).reshape(t, r, ng, g), axis=-1)
        am = np.maximum(am, f32(1e-12)).astype(np.float32)
        if e8m0:
            post = (am * rstd[..., None]).astype(np.float32) * F32_SQRT2
            bits = post.astype(np.float32).view(np.uint32).astype(np.int64)
            ef = ((bits + 0x400000) & 0xFF800000) >> 23
            e = np.clip(ef - E8M0_HEADROOM, 0, 255)
            qs = ((254 - e) << 23).astype(np.uint32).view(np.float32)
            factor = (rstd[..., None] * qs).astype(np.float32)
            scale = e.astype(np.uint8)
        else:
            factor = (F32_MAX_OVER_SQRT2 * (f32(1.0) / am)).astype(np.float32)
            scale = ((am * rstd[..., None]).astype(np.float32) * F32_INV_MAX_SQRT2).astype(np.float32)
        y = (xw * np.repeat(factor, g, axis=-1)).astype(np.float32)
    else:
        y = (xw * rstd[..., None]).astype(np.float32)
    nope = d - rd
    e_ = y[..., nope::2].copy()
    o_ = y[..., nope + 1 :: 2].copy()
    c = cos_rows[:, None, :]
    s = sin_rows[:, None, :]
    y[..., nope::2] = (e_ * c).astype(np.float32) - (o_ * s).astype(np.float32)
    y[..., nope + 1 :: 2] = (e_ * s).astype(np.float32) + (o_ * c).astype(np.float32)
    return y, scale


def qk_norm_rope_quant(
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
    scale_dtype: str = "fp32",
):
    """Returns (q_out [T, H, D], kv_out [T, D], q_scale, kv_scale) as numpy
    arrays: float32 values of the bf16 outputs, or e4m3fn bytes (uint8) when
    quant; scales float32 [T, H, NG] / [T, NG], uint8 for e8m0, None
    without quant."""
    h, d, rd = num_q_heads, head_dim, rope_head_dim
    t = q.shape[0]
    g = quant_group_size or d
    xq = q.reshape(t, h, d).float().numpy().astype(np.float32)
    xkv = kv.float().numpy().astype(np.float32)[:, None, :]
    cos2 = cos_cache.reshape(cos_cache.shape[0], rd // 2).float().numpy()
    sin2 = sin_cache.reshape(sin_cache.shape[0], rd // 2).float().numpy()
    pos = positions.to(torch.int64).numpy() & 0xFFFFFFFF
    pos = np.where(pos >= 2**31, pos - 2**32, pos)  # the kernel's int32 truncation
    inside = (pos >= 0) & (pos < cos2.shape[0])
    idx = np.where(inside, pos, 0)
    c = np.where(inside[:, None], cos2[idx], 0.0).astype(np.float32)
    s = np.where(inside[:, None], sin2[idx], 0.0).astype(np.float32)
    wq = q_weight.float().numpy().astype(np.float32) if q_weight is not None else None
    wkv = kv_weight.float().numpy().astype(np.float32)
    e8 = scale_dtype == "e8m0"
    yq, sq = _rows(xq, wq, c, s, d, rd, quant, g, e8)
    ykv, skv = _rows(xkv, wkv, c, s, d, rd, quant, g, e8)
    if quant:
        return fp8_bytes(yq), fp8_bytes(ykv[:, 0]), sq, skv[:, 0]
    return bf16_round(yq), bf16_round(ykv[:, 0]), None, None


def rope_table(max_pos: int, rope_dim: int, base: float = 10000.0):
    """GPT-J cos/sin tables [max_pos, RD/2] in bf16 (test inputs)."""
    inv = 1.0 / (base ** (torch.arange(0, rope_dim, 2, dtype=torch.float64) / rope_dim))
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16)
