"""Shared case builders for the CPU and GPU tests."""

from __future__ import annotations

import math
from typing import List, Optional

import numpy as np
import torch

from flydsl_amd import workloads
from flydsl_amd.workloads import DecodeConfig
from oracle import np_ref, torch_ref


def make_case(
    *,
    batch: int = 3,
    query_length: int = 1,
    num_query_heads: int = 8,
    num_kv_heads: int = 2,
    block_size: int = 16,
    ctx: Optional[List[int]] = None,
    ctx_range=(1, 200),
    per_token: bool = False,
    sliding_window: int = 0,
    seed: int = 0,
    extra_pages: int = 4,
    dist: str = "normal",
    head_size: int = 128,
    device="cpu",
) -> dict:
    rng = np.random.default_rng(seed + 17)
    if ctx is None:
        ctx = [int(x) for x in rng.integers(ctx_range[0], ctx_range[1] + 1, size=batch)]
    need = sum(math.ceil(c / block_size) for c in ctx)
    cfg = DecodeConfig(
        "case",
        len(ctx),
        query_length,
        num_query_heads,
        num_kv_heads,
        block_size,
        "fixed:0",
        per_token,
        sliding_window,
        num_blocks=need + extra_pages,
        head_size=head_size,
    )
    return workloads.build_inputs(cfg, device=device, seed=seed, context_lengths=ctx, dist=dist)


def flat_scales(case: dict):
    """[Hkv, NB*bs] scale views the reference oracle takes."""
    kc = case["key_cache"]
    nb, h, _, bs, _ = kc.shape
    ks, vs = case["key_scale"].cpu(), case["value_scale"].cpu()
    if ks.dim() > 1:
        return (
            ks.reshape(nb, h, bs).permute(1, 0, 2).reshape(h, nb * bs),
            vs.reshape(nb, h, bs).permute(1, 0, 2).reshape(h, nb * bs),
        )
    return ks.expand(h, nb * bs), vs.expand(h, nb * bs)


def indptr(case: dict) -> torch.Tensor:
    b = case["context_lengths"].shape[0]
    ql = case["query_length"]
    return torch.arange(0, (b + 1) * ql, ql, dtype=torch.int32)


def torch_oracle(case: dict, *, float_out: bool = True) -> torch.Tensor:
    """torch_mha_extend on the CPU; fp32 output unless float_out=False."""
    q = case["query"].cpu()
    if float_out:
        q = q.float()
    ks, vs = flat_scales(case)
    return torch_ref.torch_mha_extend(
        q,
        case["key_cache"].cpu(),
        case["value_cache"].cpu(),
        case["block_tables"].cpu(),
        case["context_lengths"].cpu(),
        indptr(case),
        ks,
        vs,
        sliding_window=case["sliding_window"],
        softmax_scale=case["softmax_scale"],
    )


def numpy_oracle(case: dict) -> np.ndarray:
    ks, vs = case["key_scale"].cpu(), case["value_scale"].cpu()
    per_token = ks.dim() > 1
    return np_ref.paged_decode_f64(
        case["query"].cpu().float().numpy(),
        case["key_cache"].cpu().view(torch.uint8).numpy(),
        case["value_cache"].cpu().view(torch.uint8).numpy(),
        case["block_tables"].cpu().numpy(),
        case["context_lengths"].cpu().numpy(),
        case["query_length"],
        case["softmax_scale"],
        ks.numpy() if per_token else float(ks[0]),
        vs.numpy() if per_token else float(vs[0]),
        sliding_window=case["sliding_window"],
    )


def slot_partials(case: dict, num_partitions: int):
    ks, vs = flat_scales(case)
    return torch_ref.slot_partials(
        case["query"].cpu(),
        case["key_cache"].cpu(),
        case["value_cache"].cpu(),
        case["block_tables"].cpu(),
        case["context_lengths"].cpu(),
        ks,
        vs,
        num_partitions,
        case["softmax_scale"],
        query_length=case["query_length"],
        sliding_window=case["sliding_window"],
    )
