"""Restatement of the reference's torch path for FP8 paged decode (CPU, fp32).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Written from the semantics of the reference test harness, never imported
from it (that module needs aiter at import time):

  create_kv_cache                tests/kernels/test_pa.py:177-211
  pertoken_quant                 tests/utils.py:29-73
  per_tensor_quant               aiter per-tensor quantiser as called at
                                 tests/kernels/test_pa.py:404-405
                                 (one scale = amax / dtype max)
  quantize_kv_cache_symmetric    tests/kernels/test_pa.py:334-376
  quantize_kv_cache_per_tensor   tests/kernels/test_pa.py:379-416
  shuffle_value_cache_layout     tests/kernels/test_pa.py:419-429
  reference_masked_attention     tests/kernels/test_pa.py:214-274
  torch_mha_extend               tests/kernels/test_pa.py:277-331
  lse_merge                      kernels/pa_decode_swa.py:954-1130
  slot_partials                  per-slot (exp_sum, max_logit, normalised
                                 output) that the partition kernel of
                                 kernels/pa_decode_fp8.py:2291-2320 stores,
                                 computed directly from the gathered tokens.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from . import plan

FP8 = torch.float8_e4m3fn
FP8_MAX = float(torch.finfo(FP8).max)  # 448


# --------------------------------------------------------------------------
# KV-cache construction and quantisers
# --------------------------------------------------------------------------


def create_kv_cache(
    num_blocks: int,
    block_size: int,
    num_heads: int,
    head_size: int,
    *,
    dtype: torch.dtype = torch.bfloat16,
    seed: int = 0,
    dist: str = "uniform",
    generator: Optional[torch.Generator] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Unquantised paged cache in the reference's layouts.

    K: ``[num_blocks, num_heads, head_size // 16, block_size, 16]``
    V: ``[num_blocks, num_heads, head_size, block_size]``
    ``dist="uniform"`` draws U(-1, 1) like the reference harness;
    ``dist="normal"`` draws N(0, 1) as the benchmark configurations ask.
    """
    if head_size % 16:
        raise ValueError(f"Does not support fp8 key cache with head_size={head_size}")
    g = generator if generator is not None else torch.Generator().manual_seed(seed)
    k_shape = (num_blocks, num_heads, head_size // 16, block_size, 16)
    v_shape = (num_blocks, num_heads, head_size, block_size)
    if dist == "uniform":
        k = torch.rand(k_shape, generator=g, dtype=torch.float32) * 2.0 - 1.0
        v = torch.rand(v_shape, generator=g, dtype=torch.float32) * 2.0 - 1.0
    elif dist == "normal":
        k = torch.randn(k_shape, generator=g, dtype=torch.float32)
        v = torch.randn(v_shape, generator=g, dtype=torch.float32)
    else:
        raise ValueError(f"unknown dist {dist!r}")
    return k.to(dtype), v.to(dtype)


def pertoken_quant(x: torch.Tensor, quant_dtype: torch.dtype = FP8) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row-wise symmetric quantisation over the last dimension.

    scale = amax(|row|) / dtype_max (1 where the row is all zero); the input
    is sanitised first (NaN -> 0, +-inf -> +-dtype_max); q = x / scale cast
    to ``quant_dtype``.  Returns (q, scale[..., 1] float32).
    """
    dmax = float(torch.finfo(quant_dtype).max)
    xf = torch.nan_to_num(x.to(torch.float32), nan=0.0, posinf=dmax, neginf=-dmax)
    amax = torch.maximum(xf.amax(dim=-1, keepdim=True), -xf.amin(dim=-1, keepdim=True))
    scale = amax / dmax
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    scale = torch.nan_to_num(scale, nan=1.0, posinf=1.0, neginf=1.0)
    return (xf / scale).to(quant_dtype), scale.to(torch.float32)


def per_tensor_quant(x: torch.Tensor, quant_dtype: torch.dtype = FP8) -> Tuple[torch.Tensor, torch.Tensor]:
    """One scale for the whole tensor: amax / dtype_max.  Returns (q, scale[1])."""
    dmax = float(torch.finfo(quant_dtype).max)
    xf = x.to(torch.float32)
    amax = xf.abs().amax()
    scale = amax / dmax
    if float(scale) == 0.0:
        scale = torch.ones((), dtype=torch.float32)
    return (xf / scale).to(quant_dtype), scale.reshape(1).to(torch.float32)


def _k_rows(key_cache: torch.Tensor) -> torch.Tensor:
    """[NB, H, D/16, bs, 16] -> [NB, H, bs, D] (token-major rows)."""
    nb, h, dc, bs, e = key_cache.shape
    return key_cache.permute(0, 1, 3, 2, 4).reshape(nb, h, bs, dc * e)


def _v_rows(value_cache: torch.Tensor) -> torch.Tensor:
    """[NB, H, D, bs] -> [NB, H, bs, D]."""
    return value_cache.permute(0, 1, 3, 2)


def quantize_kv_cache_symmetric(key_cache: torch.Tensor, value_cache: torch.Tensor, quant_dtype: torch.dtype = FP8):
    """Per-token-per-head quantisation (one scale per 128-element head vector).

    Returns (qK, k_scales_flat [H, NB*bs], qV, v_scales_flat [H, NB*bs],
    k_scales [NB, H, bs, 1], v_scales [NB, H, bs, 1]) with qK, qV in the
    unshuffled reference layouts.
    """
    nb, h, d, bs = value_cache.shape
    qk_rows, ks = pertoken_quant(_k_rows(key_cache).contiguous(), quant_dtype)
    qv_rows, vs = pertoken_quant(_v_rows(value_cache).contiguous(), quant_dtype)
    qk = qk_rows.reshape(nb, h, bs, d // 16, 16).permute(0, 1, 3, 2, 4).contiguous()
    qv = qv_rows.permute(0, 1, 3, 2).contiguous()
    ks_flat = ks.permute(1, 0, 2, 3).reshape(h, nb * bs).contiguous()
    vs_flat = vs.permute(1, 0, 2, 3).reshape(h, nb * bs).contiguous()
    return qk, ks_flat, qv, vs_flat, ks, vs


def quantize_kv_cache_per_tensor(key_cache: torch.Tensor, value_cache: torch.Tensor, quant_dtype: torch.dtype = FP8):
    """One scale for all of K and one for all of V (same return layout)."""
    nb, h, d, bs = value_cache.shape
    qk, ks = per_tensor_quant(key_cache, quant_dtype)
    qv, vs = per_tensor_quant(value_cache, quant_dtype)
    return qk, ks.expand(h, nb * bs), qv, vs.expand(h, nb * bs), ks, vs


def shuffle_value_cache_layout(value_cache: torch.Tensor) -> torch.Tensor:
    """[NB, H, D, bs] -> trans-V [NB, H, bs/16, D, 16] (16-byte token groups)."""
    per_vec = 16 // value_cache.element_size()
    nb, h, d, bs = value_cache.shape
    return value_cache.reshape(nb, h, d, bs // per_vec, per_vec).permute(0, 1, 3, 2, 4).contiguous()


def unshuffle_value_cache_layout(value_cache_t: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`shuffle_value_cache_layout`."""
    nb, h, groups, d, per_vec = value_cache_t.shape
    return value_cache_t.permute(0, 1, 3, 2, 4).reshape(nb, h, d, groups * per_vec).contiguous()


# --------------------------------------------------------------------------
# Attention
# --------------------------------------------------------------------------


def reference_masked_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    softmax_scale: float,
    output_dtype: torch.dtype,
    is_causal: bool = True,
    sliding_window: int = 0,
) -> torch.Tensor:
    """Dense attention of ``s_q`` queries over ``s_k`` keys, fp32 math.

    query [s_q, Hq, D], key/value [s_k, Hkv, D].  KV heads are repeated to
    the query heads (GQA).  Causal: a bias of -3.4e38 on keys past the
    diagonal ``tril(diagonal = s_k - s_q)``.  Query ``i`` sits at position
    ``s_k - s_q + i``; with a window W, keys at distance >= W + 1 are set
    to -inf.  Softmax over keys, then the weighted sum of values.
    """
    q = query.to(torch.float32)
    k = key.to(torch.float32)
    v = value.to(torch.float32)
    s_q, hq, _ = q.shape
    s_k, hkv, _ = k.shape
    rep = hq // hkv
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    logits = torch.einsum("qhd,khd->hqk", q, k) * softmax_scale
    if is_causal:
        allowed = torch.ones(s_q, s_k, dtype=torch.bool).tril(diagonal=s_k - s_q)
        bias = torch.zeros(s_q, s_k, dtype=torch.float32).masked_fill(~allowed, float(-3.4e38))
        logits = logits + bias
    if sliding_window > 0:
        q_pos = torch.arange(s_q) if s_q == s_k else torch.arange(s_k - s_q, s_k)
        k_pos = torch.arange(s_k)
        far = (q_pos[:, None] - k_pos[None, :]) >= sliding_window + 1
        logits = logits.masked_fill(far.unsqueeze(0).expand_as(logits), float("-inf"))
    weights = torch.softmax(logits, dim=-1)
    return torch.einsum("hqk,khd->qhd", weights, v).to(output_dtype)


def gather_tokens(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table_row: Sequence[int],
    context_length: int,
    key_scale_flat: Optional[torch.Tensor] = None,
    value_scale_flat: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dequantised K, V [ctx, Hkv, D] float32 of one sequence.

    Logical token t lives in physical slot ``bt[t // bs] * bs + t % bs`` of
    the flattened cache; scales are ``[Hkv, NB * bs]`` (per-tensor scales
    broadcast).  Accepts the unshuffled ([NB,H,D,bs]) or trans ([NB,H,bs/16,D,16])
    value layout.
    """
    if value_cache.dim() == 5:
        value_cache = unshuffle_value_cache_layout(value_cache)
    nb, h, d, bs = value_cache.shape
    k_flat = key_cache.permute(0, 3, 1, 2, 4).reshape(nb * bs, h, d)
    v_flat = value_cache.permute(0, 3, 1, 2).reshape(nb * bs, h, d)
    bt = torch.as_tensor(list(block_table_row), dtype=torch.int64)
    t = torch.arange(context_length, dtype=torch.int64)
    slots = bt.repeat_interleave(bs)[:context_length] * bs + t % bs
    k = k_flat[slots].to(torch.float32)
    v = v_flat[slots].to(torch.float32)
    if key_scale_flat is not None:
        k = k * key_scale_flat[:, slots].t().unsqueeze(-1).to(torch.float32)
    if value_scale_flat is not None:
        v = v * value_scale_flat[:, slots].t().unsqueeze(-1).to(torch.float32)
    return k, v


def torch_mha_extend(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lengths: torch.Tensor,
    query_output_indptr: torch.Tensor,
    key_scale: Optional[torch.Tensor] = None,
    value_scale: Optional[torch.Tensor] = None,
    sliding_window: int = 0,
    softmax_scale: Optional[float] = None,
) -> torch.Tensor:
    """Paged decode reference: per sequence, gather, dequantise, attend.

    ``key_scale``/``value_scale`` are the flat ``[Hkv, NB*bs]`` forms.  The
    softmax scale defaults to 1/sqrt(head_size) as in the reference.
    Returns ``[total_queries, Hq, D]`` in the query dtype.
    """
    vc = value_cache if value_cache.dim() == 4 else unshuffle_value_cache_layout(value_cache)
    head_size = vc.shape[2]
    scale = softmax_scale if softmax_scale is not None else 1.0 / (head_size**0.5)
    indptr = [int(x) for x in query_output_indptr.tolist()]
    outs: List[torch.Tensor] = []
    for b in range(len(indptr) - 1):
        q = query[indptr[b] : indptr[b + 1]]
        ctx = int(context_lengths[b])
        k, v = gather_tokens(key_cache, vc, block_tables[b].tolist(), ctx, key_scale, value_scale)
        outs.append(reference_masked_attention(q, k, v, scale, query.dtype, True, sliding_window))
    return torch.cat(outs)


# --------------------------------------------------------------------------
# Split-context partials and their log-sum-exp merge
# --------------------------------------------------------------------------


def slot_partials(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lengths: torch.Tensor,
    key_scale_flat: Optional[torch.Tensor],
    value_scale_flat: Optional[torch.Tensor],
    num_partitions: int,
    softmax_scale: float,
    *,
    query_length: int = 1,
    sliding_window: int = 0,
    dtype: torch.dtype = torch.float64,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """What each split-context slot stores, computed directly.

    For slot z of (sequence b, kv head h) and column e = qi * gqa + g:
    ``max_logits = max`` of the scaled logits of the visible tokens in the
    slot's token range (-inf if none), ``exp_sums = sum exp(l - max)`` (0 if
    none) and ``tmp_out = sum exp(l - max) v / exp_sums`` (0 if none).
    Slot ranges come from :func:`plan.slot_token_range`.  Returns
    (exp_sums, max_logits [B, Hkv, P, ql*gqa], tmp_out [B, Hkv, P, ql*gqa, D]).
    """
    vc = value_cache if value_cache.dim() == 4 else unshuffle_value_cache_layout(value_cache)
    nb, hkv, d, bs = vc.shape
    batch = int(context_lengths.shape[0])
    hq = query.shape[1]
    gqa = hq // hkv
    eq = query_length * gqa
    es = torch.zeros(batch, hkv, num_partitions, eq, dtype=dtype)
    ml = torch.full((batch, hkv, num_partitions, eq), float("-inf"), dtype=dtype)
    to = torch.zeros(batch, hkv, num_partitions, eq, d, dtype=dtype)
    for b in range(batch):
        ctx = int(context_lengths[b])
        k, v = gather_tokens(key_cache, vc, block_tables[b].tolist(), ctx, key_scale_flat, value_scale_flat)
        k = k.to(dtype)
        v = v.to(dtype)
        q = query[b * query_length : (b + 1) * query_length].to(dtype)
        for z in range(num_partitions):
            t0, t1 = plan.slot_token_range(ctx, num_partitions, z, sliding_window=sliding_window, query_length=query_length)
            if t1 <= t0:
                continue
            for qi in range(query_length):
                lo, hi = plan.visible_token_range(ctx, qi, query_length, sliding_window)
                a, e_ = max(t0, lo), min(t1, hi)
                if e_ <= a:
                    continue
                for h in range(hkv):
                    kk = k[a:e_, h]  # [n, D]
                    vv = v[a:e_, h]
                    for g in range(gqa):
                        col = qi * gqa + g
                        l = (kk @ q[qi, h * gqa + g]) * softmax_scale
                        m = l.max()
                        p = torch.exp(l - m)
                        s = p.sum()
                        es[b, h, z, col] = s
                        ml[b, h, z, col] = m
                        to[b, h, z, col] = (p[:, None] * vv).sum(0) / s
    return es, ml, to


def range_partial(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table_row,
    ctx: int,
    key_scale_flat: Optional[torch.Tensor],
    value_scale_flat: Optional[torch.Tensor],
    b: int,
    h: int,
    t0: int,
    t1: int,
    softmax_scale: float,
    *,
    query_length: int = 1,
    sliding_window: int = 0,
    dtype: torch.dtype = torch.float64,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention of sequence b's queries of kv head h over keys [t0, t1)
    only (each query further limited to the keys it may see): the normalised
    output [ql, gqa, D] and its log-sum-exp [ql, gqa] (natural log; -inf and
    a zero row when no key is visible) -- what one work of the persistent
    route stores (kernels/pa_decode_fp8.py:1600-1643)."""
    vc = value_cache if value_cache.dim() == 4 else unshuffle_value_cache_layout(value_cache)
    hkv, d = vc.shape[1], vc.shape[2]
    gqa = query.shape[1] // hkv
    k, v = gather_tokens(key_cache, vc, list(block_table_row), ctx, key_scale_flat, value_scale_flat)
    k, v = k.to(dtype), v.to(dtype)
    q = query[b * query_length : (b + 1) * query_length].to(dtype)
    out = torch.zeros(query_length, gqa, d, dtype=dtype)
    lse = torch.full((query_length, gqa), float("-inf"), dtype=dtype)
    for qi in range(query_length):
        lo, hi = plan.visible_token_range(ctx, qi, query_length, sliding_window)
        a, e_ = max(t0, lo), min(t1, hi)
        if e_ <= a:
            continue
        kk, vv = k[a:e_, h], v[a:e_, h]
        for g in range(gqa):
            l = (kk @ q[qi, h * gqa + g]) * softmax_scale
            m = l.max()
            p = torch.exp(l - m)
            s = p.sum()
            out[qi, g] = (p[:, None] * vv).sum(0) / s
            lse[qi, g] = m + torch.log(s)
    return out, lse


def lse_merge(exp_sums: torch.Tensor, max_logits: torch.Tensor, tmp_out: torch.Tensor) -> torch.Tensor:
    """Merge P slot partials: out = sum_p w_p tmp_p with
    w_p = s_p e^{m_p - M} / sum_q s_q e^{m_q - M}, M = max_p m_p.

    Inputs [..., P, E] and [..., P, E, D]; returns [..., E, D] float64.  An
    all-empty row (M = -inf or zero total) yields 0, matching the guarded
    division of the reference reduce.
    """
    m = max_logits.to(torch.float64)
    s = exp_sums.to(torch.float64)
    big = m.amax(dim=-2, keepdim=True)
    safe_big = torch.where(torch.isfinite(big), big, torch.zeros_like(big))
    w = torch.where(torch.isfinite(m), s * torch.exp(m - safe_big), torch.zeros_like(s))
    tot = w.sum(dim=-2, keepdim=True)
    w = w / torch.where(tot > 0, tot, torch.ones_like(tot))
    return (w.unsqueeze(-1) * tmp_out.to(torch.float64)).sum(dim=-3)
