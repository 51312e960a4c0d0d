"""Integer planning of the split-context decode (test infrastructure).

Pure-Python restatement of the reference's index arithmetic.  The HIP
library computes the same quantities in ``flydsl_amd/csrc/pa_plan.h``; the
CPU tests compare the two bit for bit.

  get_recommended_splits   kernels/pa_decode_fp8.py:1922-1949
  sw_partition_count       kernels/pa_decode_swa.py:832-840
  slot_token_range         kernels/pa_decode_fp8.py:2311-2320 (small-block
                           route) and kernels/pa_decode_swa.py:1356-1368
                           (sliding-window route, generalised from
                           1024-token pages to any page size: a slot is a
                           256-token tile of the logical sequence)
  visible_token_range      causal/window bounds of
                           kernels/pa_decode_swa.py:1597-1620 and
                           tests/kernels/test_pa.py:236-269
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

PARTITION_SIZE = 256  # tokens per context sub-partition (KV_COMPUTE_BLOCK)


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def get_recommended_splits(
    num_sequences: int,
    num_kv_heads: int,
    split_kv_blocks: int = 1,
    *,
    sliding_window: int = 0,
    context_partition_size: int = PARTITION_SIZE,
    query_length: int = 1,
    num_cu: int = 256,
) -> int:
    """Slots per (sequence, kv head).

    Sliding window: enough 256-token tiles to cover ``W + ql - 1`` tokens at
    any alignment, ``cdiv(W + ql - 1, cps) + 1``.  Otherwise an occupancy
    target of two workgroups per CU spread over ``B * Hkv * s`` units, rounded
    up to a multiple of ``s`` (pages per partition) and clamped to [4, 8].
    """
    if sliding_window > 0:
        return cdiv(sliding_window + query_length - 1, context_partition_size) + 1
    target = num_cu * 2
    denom = max(1, num_sequences * num_kv_heads * split_kv_blocks)
    n = cdiv(target, denom) * split_kv_blocks
    return max(4, min(n, 8))


def sw_partition_count(sliding_window: int, context_partition_size: int = PARTITION_SIZE, query_length: int = 1) -> int:
    if sliding_window <= 0:
        return 0
    return cdiv(sliding_window + query_length - 1, context_partition_size) + 1


def slot_subpartitions(context_length: int, num_partitions: int, slot: int) -> Tuple[int, int]:
    """Sub-partition index range [first, end) of a slot (non-window route).

    ``nt = cdiv(ctx, 256)`` sub-partitions are dealt in contiguous runs of
    ``pps = cdiv(nt, P)``; slot z owns ``[z*pps, min((z+1)*pps, nt))``.
    """
    nt = cdiv(context_length, PARTITION_SIZE)
    pps = cdiv(nt, num_partitions) if nt > 0 else 0
    first = slot * pps
    end = min((slot + 1) * pps, nt)
    return first, max(first, end)


def sw_first_tile(context_length: int, sliding_window: int, query_length: int) -> int:
    """First 256-token tile touched by any query's window."""
    start = max(context_length - query_length - sliding_window, 0)
    return start // PARTITION_SIZE


def slot_token_range(
    context_length: int,
    num_partitions: int,
    slot: int,
    *,
    sliding_window: int = 0,
    query_length: int = 1,
) -> Tuple[int, int]:
    """Logical token range [t0, t1) a slot reads (empty when t1 <= t0)."""
    if sliding_window > 0:
        nt = cdiv(context_length, PARTITION_SIZE)
        tile = sw_first_tile(context_length, sliding_window, query_length) + slot
        if tile >= nt:
            return 0, 0
        if num_partitions == 1:
            # fused single-slot launch walks every visible tile
            # (kernels/pa_decode_fp8.py:2920-2925, pa_decode_swa.py:1480-1620)
            return tile * PARTITION_SIZE, context_length
        return tile * PARTITION_SIZE, min((tile + 1) * PARTITION_SIZE, context_length)
    first, end = slot_subpartitions(context_length, num_partitions, slot)
    if end <= first:
        return 0, 0
    return first * PARTITION_SIZE, min(end * PARTITION_SIZE, context_length)


def visible_token_range(context_length: int, qi: int, query_length: int, sliding_window: int) -> Tuple[int, int]:
    """Keys query ``qi`` (0-based among the ``ql`` new tokens) may attend.

    The query sits at position ``ctx - ql + qi``; causal keeps keys up to and
    including it, a window W keeps the W + 1 most recent of those.
    """
    hi = context_length - query_length + 1 + qi
    lo = context_length - query_length - sliding_window + qi if sliding_window > 0 else 0
    return max(lo, 0), max(min(hi, context_length), 0)


def slot_pages(block_table_row: Sequence[int], t0: int, t1: int, block_size: int) -> List[int]:
    """Physical pages holding logical tokens [t0, t1), in logical order."""
    if t1 <= t0:
        return []
    return [int(block_table_row[p]) for p in range(t0 // block_size, cdiv(t1, block_size))]


def attended_tokens(context_lengths: Sequence[int], query_length: int, sliding_window: int) -> List[int]:
    """Per sequence, the number of distinct keys any of its queries attends."""
    out = []
    for ctx in context_lengths:
        lo, _ = visible_token_range(int(ctx), 0, query_length, sliding_window)
        _, hi = visible_token_range(int(ctx), query_length - 1, query_length, sliding_window)
        out.append(max(hi - lo, 0))
    return out
