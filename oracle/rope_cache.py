"""CPU restatement of the KV-cache writer (test infrastructure only).

Follows the reference's torch semantics of the fused RoPE + KV-cache kernel
(tests/kernels/test_fused_rope_cache.py:162-237, kernel
kernels/fused_rope_cache_kernel.py:105-412):

  * NeoX rotation in the input dtype, every product and the sum rounded to
    it (torch ops on bf16 / f16 CPU tensors):
        out[:D/2] = x1 * cos[:D/2] - x2 * sin[:D/2]
        out[D/2:] = x2 * cos[D/2:] + x1 * sin[D/2:]
    with cos / sin = [row, row] when only the first half is stored
    (reuse_freqs_front_part, :186-190 of the test);
  * the cache takes the rotated K and the unrotated V of every token whose
    slot is >= 0 (:218-234), block slot // bs, position slot % bs, in the
    flash layout [NB, bs, KH, D] or the ATOM layout K [NB, KH, D/16, bs, 16],
    V [NB, KH, D, bs] (kernel :29-35), or V [NB, KH, bs/16, D, 16] (the
    decode kernels' layout; no counterpart in the reference writer);
  * the fp8 cache (apply_scale, kernel :277-300) holds e4m3fn of
    value * (1 / scale) in float32; this build saturates at +-448 where a
    plain conversion would give NaN;
  * int64 positions and slots are read as their low 32-bit words (the
    kernel's stride-2 int32 view, :183-187, :238-243).

Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline use this.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

FLASH, ATOM, ATOM_TRANS_V = "flash", "atom", "atom_trans_v"
FP8_MAX = 448.0


def low_words(index: torch.Tensor) -> torch.Tensor:
    """int32 / int64 index tensor -> int64 values of the low 32-bit words."""
    x = index.to(torch.int64) & 0xFFFFFFFF
    return torch.where(x >= 2**31, x - 2**32, x)


def rope_neox(x: torch.Tensor, cos_rows: torch.Tensor, sin_rows: torch.Tensor, reuse_freqs_front_part: bool):
    """x [T, H, D] (bf16 / f16), cos/sin rows [T, D/2 or D] of the same dtype."""
    d = x.shape[-1]
    h = d // 2
    cos = cos_rows.unsqueeze(1)
    sin = sin_rows.unsqueeze(1)
    if reuse_freqs_front_part:
        cos = torch.cat([cos, cos], dim=-1)
        sin = torch.cat([sin, sin], dim=-1)
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat([x1 * cos[..., :h] - x2 * sin[..., :h], x2 * cos[..., h:] + x1 * sin[..., h:]], dim=-1)


def fp8_bytes(x: torch.Tensor, scale: float) -> torch.Tensor:
    """e4m3fn bytes (uint8) of float32(x) * float32(1 / scale), saturated."""
    rcp = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(scale, dtype=torch.float32)
    y = (x.to(torch.float32) * rcp).clamp(-FP8_MAX, FP8_MAX)
    return y.to(torch.float8_e4m3fn).view(torch.uint8)


def rope_cache_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    positions: torch.Tensor,
    cos_cache: torch.Tensor,
    sin_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    *,
    block_size: int,
    layout: str,
    reuse_freqs_front_part: bool = True,
    apply_scale: bool = False,
    k_scale: Optional[float] = None,
    v_scale: Optional[float] = None,
    inplace: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(q_out, k_out, key_cache', value_cache') on the CPU.

    The caches are returned as new tensors (or written in place with
    ``inplace``); with apply_scale they are uint8 (fp8 e4m3fn bytes),
    otherwise of q's dtype.  Positions index the cos / sin tables after
    clamping into [0, max_pos), as the kernel does.
    """
    pos = low_words(positions).clamp(0, cos_cache.shape[0] - 1)
    cos_rows, sin_rows = cos_cache[pos], sin_cache[pos]
    q_out = rope_neox(q, cos_rows, sin_rows, reuse_freqs_front_part)
    k_out = rope_neox(k, cos_rows, sin_rows, reuse_freqs_front_part)
    kc, vc = (key_cache, value_cache) if inplace else (key_cache.clone(), value_cache.clone())
    if apply_scale:
        kw, vw = fp8_bytes(k_out, k_scale), fp8_bytes(v, v_scale)
    else:
        kw, vw = k_out, v
    nb = kc.shape[0]
    kh, d = k.shape[1], k.shape[2]
    for i, slot in enumerate(low_words(slot_mapping).tolist()):
        if slot < 0:
            continue
        bi, bp = slot // block_size, slot % block_size
        if bi >= nb:
            continue
        if layout == FLASH:
            kc[bi, bp] = kw[i]
            vc[bi, bp] = vw[i]
        else:
            kc[bi, :, :, bp, :] = kw[i].reshape(kh, d // 16, 16)
            if layout == ATOM:
                vc[bi, :, :, bp] = vw[i]
            else:
                vc[bi, :, bp // 16, :, bp % 16] = vw[i]
    return q_out, k_out, kc, vc
