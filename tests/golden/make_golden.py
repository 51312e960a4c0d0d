"""Writes the golden fixtures of this directory from the CPU oracle.

The reference ships no golden vectors for the decode path or the KV-cache
writer (its tests recompute a torch reference every run), so these fixtures
freeze the outputs of the pinned oracle (oracle/) on small seeded inputs:
the CPU tests check that the oracle still reproduces them, the GPU tests
check the HIP library against them without running the oracle.

    python -m tests.golden.make_golden      # from the repository root

Files:
  decode.npz    four decode calls: inputs (query as bf16 bits, fp8 K/V cache
                bytes, block tables, context lengths, scales) and the
                oracle's float32 output (torch_mha_extend restatement)
  planner.npz   get_recommended_splits over a grid, slot token ranges, and
                two get_pa_metadata work lists
  rope_cache.npz  three KV-cache writer calls: inputs and the oracle's
                Q_out / K_out / key and value caches, as raw bits
  qk_norm_rope.npz  four fused RMSNorm + GPT-J RoPE (+ fp8 quant) calls:
                inputs as raw bits and the oracle's outputs and scales
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import torch

from oracle import plan, worklist
from oracle import qk_norm_rope as qnr
from oracle import rope_cache as rc
from tests._cases import make_case, torch_oracle

HERE = os.path.dirname(os.path.abspath(__file__))

# name -> make_case keyword arguments
DECODE_CASES = {
    "tensor_scale": dict(batch=3, ctx=[1, 37, 300], num_query_heads=8, num_kv_heads=2, seed=101),
    "token_scale_mtp3": dict(ctx=[5, 129, 257], query_length=3, num_query_heads=16, num_kv_heads=2,
                             per_token=True, seed=102),
    "window100_page64_mtp2": dict(ctx=[90, 350], query_length=2, num_query_heads=8, num_kv_heads=1,
                                  block_size=64, sliding_window=100, seed=103),
    "gqa16_long": dict(ctx=[1100], num_query_heads=16, num_kv_heads=1, seed=104),
}

SPLIT_GRID = [
    # (num_sequences, num_kv_heads, split_kv_blocks, sliding_window, query_length, num_cu)
    (1, 1, 1, 0, 1, 256), (4, 8, 1, 0, 1, 256), (128, 8, 1, 0, 1, 256), (3, 2, 16, 0, 1, 256),
    (64, 8, 1, 0, 4, 256), (7, 1, 1, 0, 1, 80), (2, 8, 1, 4096, 1, 256), (2, 8, 1, 100, 2, 256),
    (5, 4, 1, 256, 1, 256), (1, 1, 1, 1, 1, 256),
]

SLOT_CTXS = [1, 255, 256, 257, 1000, 4097]

WORKLISTS = {
    "ragged_h2": dict(context_lens=[700, 3, 2049, 0, 256, 1500, 12], num_heads_k=2, gqa=4, query_length=1,
                      num_cu=16, kv_granularity=256),
    "mtp_h1": dict(context_lens=[4000, 10, 600], num_heads_k=1, gqa=8, query_length=4, num_cu=5,
                   kv_granularity=16),
}

# name -> (T, QH, KH, D, bs, NB, max_pos, dtype, layout, apply_scale, reuse, index dtype, slot kind)
ROPE_CASES = {
    "prefill_trans_fp8": (48, 4, 2, 64, 16, 8, 64, "bf16", rc.ATOM_TRANS_V, True, True, torch.int32, "runs"),
    "decode_atom_f16_i64": (7, 8, 1, 128, 16, 4, 32, "f16", rc.ATOM, False, False, torch.int64, "scatter"),
    "flash_bf16_skips": (9, 2, 2, 32, 16, 2, 16, "bf16", rc.FLASH, False, True, torch.int32, "skips"),
}
ROPE_SCALES = (0.1, 0.07)


def _bits(t: torch.Tensor) -> np.ndarray:
    """Raw bits of a CPU tensor as an unsigned numpy array."""
    view = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[t.element_size()]
    a = t.contiguous().view(view).numpy()
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32}[t.element_size()])


def decode_fixture() -> dict:
    arrays, meta = {}, {}
    for name, kw in DECODE_CASES.items():
        case = make_case(**kw)
        out = torch_oracle(case)
        arrays[f"{name}/query_bf16"] = _bits(case["query"])
        arrays[f"{name}/key_cache"] = _bits(case["key_cache"])
        arrays[f"{name}/value_cache"] = _bits(case["value_cache"])
        arrays[f"{name}/block_tables"] = case["block_tables"].numpy()
        arrays[f"{name}/context_lengths"] = case["context_lengths"].numpy()
        arrays[f"{name}/key_scale"] = case["key_scale"].numpy()
        arrays[f"{name}/value_scale"] = case["value_scale"].numpy()
        arrays[f"{name}/out"] = out.float().numpy()
        meta[name] = dict(query_length=case["query_length"], sliding_window=case["sliding_window"],
                          softmax_scale=case["softmax_scale"])
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    return arrays


def planner_fixture() -> dict:
    splits = [plan.get_recommended_splits(b, h, s, sliding_window=w, query_length=ql, num_cu=cu)
              for b, h, s, w, ql, cu in SPLIT_GRID]
    slots = []
    for ctx in SLOT_CTXS:
        for P in (1, 3, 8):
            for z in range(P + 1):
                slots.append((ctx, P, z, 0, 1, *plan.slot_token_range(ctx, P, z)))
        for W, ql in ((100, 2), (4096, 1)):
            if ctx < ql:
                continue
            P = plan.sw_partition_count(W, query_length=ql)
            for z in range(P + 1):
                slots.append((ctx, P, z, W, ql, *plan.slot_token_range(ctx, P, z, sliding_window=W, query_length=ql)))
    arrays = {"split_grid": np.array(SPLIT_GRID, np.int32), "splits": np.array(splits, np.int32),
              "slot_ranges": np.array(slots, np.int64)}
    for name, kw in WORKLISTS.items():
        ref = worklist.pa_metadata_v1(**kw)
        n, g = ref["num_works"], ref["num_groups"]
        used = int(ref["reduce_indptr"][-1])
        arrays[f"{name}/work_indptr"] = ref["work_indptr"]
        arrays[f"{name}/work_info"] = ref["work_info"][:n]
        arrays[f"{name}/reduce_indptr"] = ref["reduce_indptr"]
        arrays[f"{name}/reduce_final_map"] = ref["reduce_final_map"][:g]
        arrays[f"{name}/reduce_partial_map"] = ref["reduce_partial_map"][:used]
    arrays["worklist_args"] = np.frombuffer(json.dumps(WORKLISTS).encode(), dtype=np.uint8)
    return arrays


def rope_inputs(name: str) -> dict:
    """Seeded inputs of one writer case (CPU tensors)."""
    T, QH, KH, D, bs, NB, max_pos, dt, layout, apply_scale, reuse, idt, slots_kind = ROPE_CASES[name]
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    cols = D // 2 if reuse else D
    theta = torch.rand(max_pos, cols, generator=g) * 6.3
    if slots_kind == "runs":  # sequences of 16, 20 and 12 tokens filling pages from position 0
        pages = torch.randperm(NB, generator=g).tolist()
        slots, p = [], 0
        for n in (16, 20, 12):
            need = math.ceil(n / bs)
            slots += [pages[p + i // bs] * bs + i % bs for i in range(n)]
            p += need
        slots = torch.tensor(slots)
    elif slots_kind == "scatter":
        slots = torch.randperm(NB * bs, generator=g)[:T]
    else:
        slots = torch.tensor([0, -1, 5, 17, -7, 31, 32, 40, 2])  # 32, 40: past the cache
    cache_dt = torch.uint8 if apply_scale else tdt
    if layout == rc.FLASH:
        kc = torch.zeros(NB, bs, KH, D, dtype=cache_dt)
        vc = torch.zeros(NB, bs, KH, D, dtype=cache_dt)
    else:
        kc = torch.zeros(NB, KH, D // 16, bs, 16, dtype=cache_dt)
        vc = (torch.zeros(NB, KH, D, bs, dtype=cache_dt) if layout == rc.ATOM
              else torch.zeros(NB, KH, bs // 16, D, 16, dtype=cache_dt))
    return dict(
        q=torch.randn(T, QH, D, generator=g).to(tdt),
        k=torch.randn(T, KH, D, generator=g).to(tdt),
        v=(torch.randn(T, KH, D, generator=g) * 20).to(tdt),
        positions=torch.randint(0, max_pos, (T,), generator=g).to(idt),
        cos=torch.cos(theta).to(tdt),
        sin=torch.sin(theta).to(tdt),
        slots=slots.to(idt),
        key_cache=kc,
        value_cache=vc,
    )


def rope_reference(name: str, inp: dict):
    T, QH, KH, D, bs, NB, max_pos, dt, layout, apply_scale, reuse, idt, _ = ROPE_CASES[name]
    return rc.rope_cache_ref(inp["q"], inp["k"], inp["v"], inp["positions"], inp["cos"], inp["sin"], inp["slots"],
                             inp["key_cache"], inp["value_cache"], block_size=bs, layout=layout,
                             reuse_freqs_front_part=reuse, apply_scale=apply_scale, k_scale=ROPE_SCALES[0],
                             v_scale=ROPE_SCALES[1])


def rope_fixture() -> dict:
    arrays = {}
    for name in ROPE_CASES:
        inp = rope_inputs(name)
        for key, t in inp.items():
            arrays[f"{name}/{key}"] = _bits(t) if t.is_floating_point() else t.numpy()
        for key, t in zip(("q_out", "k_out", "key_cache_out", "value_cache_out"), rope_reference(name, inp)):
            arrays[f"{name}/{key}"] = _bits(t)
    return arrays


# name -> (T, H, D, RD, quant, group_size, scale_dtype, q_weighted, max_pos, kv row stride)
QKNR_CASES = {
    "v4_bf16": (6, 4, 512, 64, False, None, "fp32", False, 32, 512),
    "v4_fp8_g128_qw": (5, 3, 512, 64, True, 128, "fp32", True, 32, 640),
    "d256_fp8_e8m0_g64": (4, 2, 256, 128, True, 64, "e8m0", False, 16, 256),
    "d128_full_rope_oob": (7, 1, 128, 128, True, 32, "fp32", True, 8, 192),
}


def qknr_inputs(name: str) -> dict:
    """Seeded inputs of one fused RMSNorm + RoPE call (CPU tensors; kv is a
    [T, D] view with the case's row stride)."""
    T, H, D, RD, quant, G, sd, qw, max_pos, kv_stride = QKNR_CASES[name]
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    cos, sin = qnr.rope_table(max_pos, RD)
    kv_wide = torch.randn(T, kv_stride, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int64)
    if name.endswith("oob"):
        pos[0], pos[1] = -1, max_pos
    return dict(
        q=torch.randn(T, H, D, generator=g).to(torch.bfloat16),
        kv=kv_wide[:, :D],
        kv_weight=(1.0 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16),
        q_weight=(1.0 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16) if qw else None,
        cos_cache=cos,
        sin_cache=sin,
        positions=pos,
    )


def qknr_reference(name: str, inp: dict):
    T, H, D, RD, quant, G, sd, qw, max_pos, kv_stride = QKNR_CASES[name]
    return qnr.qk_norm_rope_quant(inp["q"], inp["kv"], inp["kv_weight"], inp["cos_cache"], inp["sin_cache"],
                                  inp["positions"], num_q_heads=H, head_dim=D, rope_head_dim=RD,
                                  q_weight=inp["q_weight"], quant=quant, quant_group_size=G, scale_dtype=sd)


def qknr_fixture() -> dict:
    arrays = {}
    for name in QKNR_CASES:
        inp = qknr_inputs(name)
        for key, t in inp.items():
            if t is not None:
                arrays[f"{name}/{key}"] = _bits(t) if t.is_floating_point() else t.numpy()
        for key, a in zip(("q_out", "kv_out", "q_scale", "kv_scale"), qknr_reference(name, inp)):
            if a is not None:
                arrays[f"{name}/{key}"] = np.ascontiguousarray(a)
    return arrays


def main() -> None:
    torch.set_num_threads(1)
    np.savez_compressed(os.path.join(HERE, "decode.npz"), **decode_fixture())
    np.savez_compressed(os.path.join(HERE, "planner.npz"), **planner_fixture())
    np.savez_compressed(os.path.join(HERE, "rope_cache.npz"), **rope_fixture())
    np.savez_compressed(os.path.join(HERE, "qk_norm_rope.npz"), **qknr_fixture())


if __name__ == "__main__":
    main()
