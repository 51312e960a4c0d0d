"""Synthetic inputs for the benchmark configurations (seeded, any device).

Shapes follow the reference's decode layouts (kernels/pa_decode_fp8.py:
2812-2832; tests/kernels/test_pa.py:177-211, 334-429): query [B*ql, Hq, 128]
bf16; K [NB, Hkv, 8, bs, 16] fp8 e4m3fn; trans V [NB, Hkv, bs/16, 128, 16]
fp8; per-tensor scales [1] or per-token-per-head scales [NB, Hkv, bs, 1]
(amax / 448); block tables of randomly permuted physical pages.

  c1_tiny    B4,   ql1, Hq8/Hkv2,   bs16, ctx U[1, 512], per tensor, NB = 256
  c2_llama8b B64,  ql1, Hq32/Hkv8,  bs16, ctx 4096,      per tensor
  c3_ragged  B128, ql1, Hq32/Hkv8,  bs16, ctx lognormal(median 2048, sigma 1)
                                          clipped to [16, 32768], per token
  c4_window  B32,  ql1, Hq32/Hkv8,  bs16, W 4096, ctx U[8192, 32768], per tensor
  c5_mtp     B256, ql4, Hq64/Hkv4,  bs64, ctx U[4096, 8192], per token
  c3_ragged_p1024  C3's batch on 1024-token pages: the persistent
             (work-list) route of get_pa_metadata + pa_decode_ps_launch
  c5_mtp_p1024     C5's batch on 1024-token pages: the same route with
             64 query columns per kv head (cooperative bins)
  c2_d64, c2_d256  C2's batch at head sizes 64 and 256 (the generic kernels)
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, List, Optional

import numpy as np
import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
HEAD = 128


@dataclasses.dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    query_length: int
    num_query_heads: int
    num_kv_heads: int
    block_size: int
    ctx: str  # "fixed:N" | "uniform:LO:HI" | "lognormal:MEDIAN:SIGMA:LO:HI"
    per_token: bool
    sliding_window: int = 0
    num_blocks: Optional[int] = None  # physical pages; default = pages needed
    head_size: int = HEAD

    @property
    def gqa(self) -> int:
        return self.num_query_heads // self.num_kv_heads


CONFIGS: Dict[str, DecodeConfig] = {
    "c1_tiny": DecodeConfig("c1_tiny", 4, 1, 8, 2, 16, "uniform:1:512", False, num_blocks=256),
    "c2_llama8b": DecodeConfig("c2_llama8b", 64, 1, 32, 8, 16, "fixed:4096", False),
    "c3_ragged": DecodeConfig("c3_ragged", 128, 1, 32, 8, 16, "lognormal:2048:1.0:16:32768", True),
    "c4_window": DecodeConfig("c4_window", 32, 1, 32, 8, 16, "uniform:8192:32768", False, sliding_window=4096),
    "c5_mtp": DecodeConfig("c5_mtp", 256, 4, 64, 4, 64, "uniform:4096:8192", True),
    "c3_ragged_p1024": DecodeConfig("c3_ragged_p1024", 128, 1, 32, 8, 1024, "lognormal:2048:1.0:16:32768", True),
    "c5_mtp_p1024": DecodeConfig("c5_mtp_p1024", 256, 4, 64, 4, 1024, "uniform:4096:8192", True),
    "c2_d64": DecodeConfig("c2_d64", 64, 1, 32, 8, 16, "fixed:4096", False, head_size=64),
    "c2_d256": DecodeConfig("c2_d256", 64, 1, 32, 8, 16, "fixed:4096", False, head_size=256),
}


def sample_context_lengths(cfg: DecodeConfig, seed: int) -> List[int]:
    rng = np.random.default_rng(seed)
    kind, *params = cfg.ctx.split(":")
    if kind == "fixed":
        return [int(params[0])] * cfg.batch
    if kind == "uniform":
        lo, hi = int(params[0]), int(params[1])
        return [int(x) for x in rng.integers(lo, hi + 1, size=cfg.batch)]
    if kind == "lognormal":
        med, sigma, lo, hi = float(params[0]), float(params[1]), int(params[2]), int(params[3])
        x = np.exp(rng.normal(math.log(med), sigma, size=cfg.batch))
        return [int(v) for v in np.clip(np.round(x), lo, hi)]
    raise ValueError(cfg.ctx)


def _quant_per_tensor(x: torch.Tensor):
    amax = x.abs().amax().float()
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    return (x / scale).to(FP8), scale.reshape(1).to(torch.float32)


def _quant_rows(x: torch.Tensor):
    """Quantise along the last dim (one scale per row): returns q, scale[..., 1]."""
    amax = x.abs().amax(dim=-1, keepdim=True).float()
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    return (x / scale).to(FP8), scale


def build_inputs(
    cfg: DecodeConfig,
    device="cpu",
    seed: int = 0,
    context_lengths: Optional[List[int]] = None,
    dist: str = "normal",
) -> dict:
    """All tensors of one decode call for ``cfg``; random values from ``seed``.

    K and V are drawn per (page, head) in float32 and quantised to fp8
    e4m3fn (per tensor or per token and head).  Pages are a random
    permutation of the physical cache, dealt to sequences in order.
    """
    device = torch.device(device)
    ctx = context_lengths if context_lengths is not None else sample_context_lengths(cfg, seed)
    bs = cfg.block_size
    pages_per_seq = [math.ceil(c / bs) for c in ctx]
    need = sum(pages_per_seq)
    nb = cfg.num_blocks if cfg.num_blocks is not None else max(need, 1)
    if nb < need:
        raise ValueError(f"{cfg.name}: {nb} pages cannot hold {need}")
    rng = np.random.default_rng(seed + 1)
    perm = rng.permutation(nb).astype(np.int32)
    max_pages = max(max(pages_per_seq), 1)
    bt = np.zeros((cfg.batch, max_pages), dtype=np.int32)
    pos = 0
    for b, n in enumerate(pages_per_seq):
        bt[b, :n] = perm[pos : pos + n]
        pos += n
    gen = torch.Generator(device=device).manual_seed(seed)
    hkv, d = cfg.num_kv_heads, cfg.head_size
    rows = cfg.batch * cfg.query_length
    if dist == "normal":
        query = torch.randn(rows, cfg.num_query_heads, d, generator=gen, device=device, dtype=torch.float32)
    else:
        query = torch.rand(rows, cfg.num_query_heads, d, generator=gen, device=device) * 2 - 1
    query = query.to(torch.bfloat16)

    def draw(shape):
        if dist == "normal":
            return torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
        return torch.rand(shape, generator=gen, device=device, dtype=torch.float32) * 2 - 1

    # token-major rows [NB, Hkv, bs, D]; quantise, then lay out.
    k_rows = draw((nb, hkv, bs, d))
    v_rows = draw((nb, hkv, bs, d))
    if cfg.per_token:
        qk, ks = _quant_rows(k_rows)
        qv, vs = _quant_rows(v_rows)
    else:
        qk, ks = _quant_per_tensor(k_rows)
        qv, vs = _quant_per_tensor(v_rows)
    del k_rows, v_rows
    key_cache = qk.view(torch.uint8).reshape(nb, hkv, bs, d // 16, 16).permute(0, 1, 3, 2, 4).contiguous()
    # trans V: [NB, Hkv, bs/16, D, 16]
    value_cache = qv.view(torch.uint8).reshape(nb, hkv, bs // 16, 16, d).permute(0, 1, 2, 4, 3).contiguous()
    del qk, qv
    return {
        "config": cfg,
        "query": query,
        "key_cache": key_cache.view(FP8),
        "value_cache": value_cache.view(FP8),
        "block_tables": torch.from_numpy(bt).to(device),
        "context_lengths": torch.tensor(ctx, dtype=torch.int32, device=device),
        "key_scale": ks.contiguous(),
        "value_scale": vs.contiguous(),
        "softmax_scale": 1.0 / math.sqrt(d),
        "query_length": cfg.query_length,
        "sliding_window": cfg.sliding_window,
    }


def attended_tokens(ctx: List[int], query_length: int, sliding_window: int) -> List[int]:
    """Distinct keys read per sequence (union over its queries)."""
    out = []
    for c in ctx:
        hi = c
        lo = max(c - query_length - sliding_window, 0) if sliding_window > 0 else 0
        out.append(max(hi - lo, 0))
    return out


def kv_bytes(cfg: DecodeConfig, ctx: List[int], include_scales: bool = False) -> int:
    """Algorithmic bytes of one decode step: attended K + V (+ scales)."""
    toks = sum(attended_tokens(ctx, cfg.query_length, cfg.sliding_window))
    per_tok = cfg.num_kv_heads * cfg.head_size * 2
    if include_scales and cfg.per_token:
        per_tok += cfg.num_kv_heads * 8
    return toks * per_tok


# ---------------------------------------------------------------------------
# KV-cache writer workloads (NeoX RoPE on Q/K + paged K/V cache write)
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class RopeCacheConfig:
    name: str
    num_tokens: int
    num_q_heads: int
    num_kv_heads: int
    head_size: int
    block_size: int
    num_blocks: int
    tokens_per_seq: int  # consecutive tokens of one sequence (1: decode, one token per sequence)
    max_pos: int = 8192


# Llama-3-8B heads, fp8 cache in the decode kernels' layout (K [NB, KH, D/16,
# bs, 16], V [NB, KH, bs/16, D, 16]), per-tensor scales, half cos/sin tables:
#   decode:  one new token for each of 64 sequences (the C2 batch)
#   prefill: 4 sequences x 4096 tokens
ROPE_CONFIGS: Dict[str, RopeCacheConfig] = {
    "rope_decode_llama8b": RopeCacheConfig("rope_decode_llama8b", 64, 32, 8, 128, 16, 16384, 1),
    "rope_prefill_llama8b": RopeCacheConfig("rope_prefill_llama8b", 16384, 32, 8, 128, 16, 16384, 4096),
}


def build_rope_inputs(cfg: RopeCacheConfig, device="cpu", seed: int = 0) -> dict:
    """Inputs of one writer call: bf16 Q/K/V N(0,1), half cos/sin tables of
    a 10000-base rotary embedding, token positions and cache slots (each
    sequence's tokens fill its pages in order; pages are a random
    permutation of the cache), fp8 caches and per-tensor scales."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    T, d = cfg.num_tokens, cfg.head_size
    q = torch.randn(T, cfg.num_q_heads, d, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(T, cfg.num_kv_heads, d, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(T, cfg.num_kv_heads, d, generator=gen, device=device).to(torch.bfloat16)
    inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = torch.arange(cfg.max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    cos = torch.cos(ang).to(torch.bfloat16).to(device)
    sin = torch.sin(ang).to(torch.bfloat16).to(device)
    rng = np.random.default_rng(seed + 1)
    nseq = T // cfg.tokens_per_seq
    pages = -(-cfg.tokens_per_seq // cfg.block_size)
    perm = rng.permutation(cfg.num_blocks)[: nseq * pages].reshape(nseq, pages)
    tok = np.arange(cfg.tokens_per_seq)
    if cfg.tokens_per_seq == 1:
        # decode: the new token of a sequence whose context already fills part of a page
        pos = rng.integers(1, cfg.max_pos, size=nseq)
        slots = perm[:, 0] * cfg.block_size + pos % cfg.block_size
    else:
        pos = np.tile(tok, nseq)
        slots = (perm[:, tok // cfg.block_size] * cfg.block_size + tok % cfg.block_size).reshape(-1)
    nb, kh, bs = cfg.num_blocks, cfg.num_kv_heads, cfg.block_size
    return {
        "config": cfg,
        "q": q,
        "k": k,
        "v": v,
        "cos": cos,
        "sin": sin,
        "positions": torch.from_numpy(pos.astype(np.int32)).to(device),
        "slot_mapping": torch.from_numpy(slots.astype(np.int32)).to(device),
        "key_cache": torch.zeros(nb, kh, d // 16, bs, 16, dtype=torch.uint8, device=device).view(FP8),
        "value_cache": torch.zeros(nb, kh, bs // 16, d, 16, dtype=torch.uint8, device=device).view(FP8),
        "k_scale": torch.tensor([k.abs().max().item() / FP8_MAX * 1.5], dtype=torch.float32, device=device),
        "v_scale": torch.tensor([v.abs().max().item() / FP8_MAX], dtype=torch.float32, device=device),
    }


def rope_bytes(cfg: RopeCacheConfig) -> int:
    """Algorithmic HBM bytes of one writer call: Q/K/V, cos/sin rows and the
    two indices read per token; Q_out/K_out and the fp8 K/V cache rows
    written."""
    d, qh, kh = cfg.head_size, cfg.num_q_heads, cfg.num_kv_heads
    read = (qh + 2 * kh) * d * 2 + 2 * (d // 2) * 2 + 2 * 4
    write = (qh + kh) * d * 2 + 2 * kh * d
    return cfg.num_tokens * (read + write)


@dataclasses.dataclass(frozen=True)
class QkNormRopeConfig:
    name: str
    num_tokens: int
    num_q_heads: int
    head_dim: int
    rope_head_dim: int
    quant: bool
    group_size: int
    scale_dtype: str
    max_pos: int = 8192


# DeepSeek-V4-shaped rows (the reference kernel's shape: D 512, RD 64), 16
# query heads per GPU plus the KV row, weightless Q, fp8 out with float32
# scales per 128 elements:
#   prefill: 8192 tokens;  decode: 64 tokens (one per sequence)
QKNR_CONFIGS: Dict[str, QkNormRopeConfig] = {
    "qknr_prefill_v4": QkNormRopeConfig("qknr_prefill_v4", 8192, 16, 512, 64, True, 128, "fp32"),
    "qknr_decode_v4": QkNormRopeConfig("qknr_decode_v4", 64, 16, 512, 64, True, 128, "fp32"),
}


def build_qknr_inputs(cfg: QkNormRopeConfig, device="cpu", seed: int = 0) -> dict:
    """Inputs of one fused RMSNorm + RoPE call: bf16 Q [T, H*D] and KV [T, D]
    N(0,1), a KV weight around 1, 10000-base GPT-J cos/sin tables [max_pos,
    RD/2] and random int64 positions."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    T, H, d, rd = cfg.num_tokens, cfg.num_q_heads, cfg.head_dim, cfg.rope_head_dim
    inv = 1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float64) / rd))
    ang = torch.arange(cfg.max_pos, dtype=torch.float64)[:, None] * inv[None, :]
    return {
        "config": cfg,
        "q": torch.randn(T, H * d, generator=gen, device=device).to(torch.bfloat16),
        "kv": torch.randn(T, d, generator=gen, device=device).to(torch.bfloat16),
        "kv_weight": (1.0 + 0.1 * torch.randn(d, generator=gen, device=device)).to(torch.bfloat16),
        "cos_cache": torch.cos(ang).to(torch.bfloat16).to(device),
        "sin_cache": torch.sin(ang).to(torch.bfloat16).to(device),
        "positions": torch.randint(0, cfg.max_pos, (T,), generator=gen, device=device, dtype=torch.int64),
    }


def qknr_bytes(cfg: QkNormRopeConfig) -> int:
    """Algorithmic HBM bytes of one call: every row read (bf16) and written
    (fp8 or bf16), its scales, and per token one position and one cos and
    one sin row (the per-channel weight is read once)."""
    rows = cfg.num_q_heads + 1
    out_el = 1 if cfg.quant else 2
    ng = cfg.head_dim // cfg.group_size if cfg.quant else 0
    scale_el = 4 if cfg.scale_dtype == "fp32" else 1
    per_tok = rows * (cfg.head_dim * 2 + cfg.head_dim * out_el + ng * scale_el) + 8 + 2 * (cfg.rope_head_dim // 2) * 2
    return cfg.num_tokens * per_tok + cfg.head_dim * 2


@dataclasses.dataclass(frozen=True)
class MlaConfig:
    """MLA decode workload (tests/kernels/test_mla_decode.py:60-68 shapes:
    128 query heads, one 576-dim latent kv head, page size 1, one query row
    per sequence)."""

    name: str
    batch: int
    context: int


MLA_CONFIGS: Dict[str, MlaConfig] = {
    # the reference test's largest configuration
    "mla_b32_c8192": MlaConfig("mla_b32_c8192", 32, 8192),
    # a full serving batch at the same context
    "mla_b128_c8192": MlaConfig("mla_b128_c8192", 128, 8192),
}


def mla_bytes(cfg: MlaConfig) -> int:
    """Algorithmic HBM bytes of one decode: every key/value row once (576 B
    fp8), the fp8 query rows and the bf16 output rows."""
    return cfg.batch * cfg.context * 576 + cfg.batch * 128 * 576 + cfg.batch * 128 * 512 * 2


def mla_flops(cfg: MlaConfig) -> int:
    """Algorithmic FLOPs: 128 heads x (576 + 512) multiply-adds per token."""
    return cfg.batch * cfg.context * 128 * (576 + 512) * 2


def build_mla_inputs(cfg: MlaConfig, device, seed: int = 7, copies: int = 1):
    """fp8 query [B, 128, 576] and `copies` fp8 KV buffers [pages, 1, 1, 576]
    from seeded normals; pages of each sequence in random order."""
    import torch

    g = torch.Generator().manual_seed(seed)
    total = cfg.batch * cfg.context
    kv_indptr = torch.arange(cfg.batch + 1, dtype=torch.int32) * cfg.context
    kv_indices = torch.randperm(total, generator=g).to(torch.int32)
    q = torch.randn(cfg.batch, 128, 576, generator=g).to(torch.bfloat16).to(torch.float8_e4m3fn)
    kv = torch.randn(total, 1, 1, 576, generator=g).to(torch.bfloat16).to(torch.float8_e4m3fn).to(device)
    kvs = [kv] + [kv.clone() for _ in range(copies - 1)]
    return {"q": q.to(device), "kvs": kvs, "kv_indptr": kv_indptr, "kv_indices": kv_indices.to(device),
            "qo_indptr": torch.arange(cfg.batch + 1, dtype=torch.int32),
            "kv_last_page_lens": torch.ones(cfg.batch, dtype=torch.int32)}
