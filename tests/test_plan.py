"""Bit-exact index planning: the C library's plan vs the Python restatement.

The partition kernel indexes slots and keys through flydsl_amd/csrc/pa_plan.h
(exported as pa_fp8_plan_slot / pa_fp8_plan_visible /
pa_fp8_recommended_splits); oracle/plan.py restates the reference formulas
(kernels/pa_decode_fp8.py:1922-1949, 2311-2320; kernels/pa_decode_swa.py:
832-840, 1356-1368, 1597-1620).  Invariants pin the restatement itself.
"""

from __future__ import annotations

import itertools

import pytest

from flydsl_amd import _lib
from flydsl_amd.workloads import CONFIGS
from oracle import plan

CTXS = [0, 1, 2, 15, 16, 17, 255, 256, 257, 511, 512, 1000, 1024, 1027, 4096, 4097, 8192, 12345, 32768, 40000]


@pytest.mark.parametrize("P", [1, 2, 3, 4, 5, 8, 17])
def test_slot_ranges_match_library(P):
    for ctx in CTXS:
        for z in range(P + 2):
            assert _lib.plan_slot(ctx, P, z, 0, 1) == plan.slot_token_range(ctx, P, z), (ctx, P, z)


@pytest.mark.parametrize("W,ql", [(1, 1), (16, 1), (255, 2), (256, 1), (1023, 4), (4096, 1), (4096, 4)])
def test_window_slot_ranges_match_library(W, ql):
    P = plan.sw_partition_count(W, query_length=ql)
    for ctx in CTXS:
        if ctx < ql:
            continue
        for z in range(P + 1):
            got = _lib.plan_slot(ctx, P, z, W, ql)
            assert got == plan.slot_token_range(ctx, P, z, sliding_window=W, query_length=ql), (ctx, W, ql, z)


def test_visible_ranges_match_library():
    for ctx, ql, W in itertools.product(CTXS, [1, 2, 3, 4], [0, 1, 7, 256, 4096]):
        if ctx < ql:
            continue
        for qi in range(ql):
            assert _lib.plan_visible(ctx, qi, ql, W) == plan.visible_token_range(ctx, qi, ql, W)


def test_recommended_splits_match_library():
    for B, H, s, cu in itertools.product([1, 3, 4, 64, 81, 128, 256, 1000], [1, 2, 4, 8], [1, 4, 16], [80, 256, 304]):
        assert _lib.recommended_splits(B, H, s, 0, 256, 1, cu) == plan.get_recommended_splits(B, H, s, num_cu=cu)
    for W, ql in itertools.product([1, 100, 256, 1023, 4096], [1, 2, 4]):
        got = _lib.recommended_splits(64, 8, 1, W, 256, ql, 256)
        assert got == plan.get_recommended_splits(64, 8, sliding_window=W, query_length=ql)


def test_recommended_splits_for_benchmark_configs():
    """Values the reference heuristic gives on a 256-CU MI355X."""
    got = {}
    for name, c in CONFIGS.items():
        if c.block_size not in (16, 64):
            continue  # the persistent route plans a work list instead
        if c.sliding_window:
            got[name] = plan.get_recommended_splits(c.batch, c.num_kv_heads, sliding_window=c.sliding_window,
                                                    query_length=c.query_length)
        else:
            got[name] = plan.get_recommended_splits(c.batch, c.num_kv_heads, 256 // c.block_size, num_cu=256)
    assert got == {"c1_tiny": 8, "c2_llama8b": 8, "c3_ragged": 8, "c4_window": 17, "c5_mtp": 4,
                   "c2_d64": 8, "c2_d256": 8}


@pytest.mark.parametrize("P", [1, 3, 4, 8])
def test_slots_tile_the_context_disjointly(P):
    for ctx in CTXS:
        covered = []
        for z in range(P):
            t0, t1 = plan.slot_token_range(ctx, P, z)
            if t1 > t0:
                assert t0 % 256 == 0
                covered.append((t0, t1))
        flat = [t for a, b in covered for t in range(a, b)]
        assert flat == list(range(ctx)), (ctx, P)


@pytest.mark.parametrize("W,ql", [(1, 1), (40, 3), (256, 1), (4096, 1), (1000, 4)])
def test_window_slots_cover_every_visible_key_once(W, ql):
    P = plan.sw_partition_count(W, query_length=ql)
    for ctx in [c for c in CTXS if c >= ql]:
        seen = []
        for z in range(P):
            t0, t1 = plan.slot_token_range(ctx, P, z, sliding_window=W, query_length=ql)
            seen.extend(range(t0, t1))
        assert len(seen) == len(set(seen))
        for qi in range(ql):
            lo, hi = plan.visible_token_range(ctx, qi, ql, W)
            assert set(range(lo, hi)) <= set(seen), (ctx, W, ql, qi)
            # brute-force the mask definition: key kp visible to query at
            # position qp iff kp <= qp and qp - kp <= W
            qp = ctx - ql + qi
            assert [kp for kp in range(ctx) if kp <= qp and qp - kp <= W] == list(range(lo, hi))


def test_slot_pages_follow_block_table():
    row = [7, 3, 9, 1, 4]
    assert plan.slot_pages(row, 0, 16, 16) == [7]
    assert plan.slot_pages(row, 15, 33, 16) == [7, 3, 9]
    assert plan.slot_pages(row, 64, 80, 16) == [4]
    assert plan.slot_pages(row, 5, 5, 16) == []


# Hand-computed from the reference's slot formula (kernels/pa_decode_fp8.py:
# 2311-2320): nt = cdiv(ctx, 256) tiles in runs of pps = cdiv(nt, P), slot z
# taking tiles [z*pps, min((z+1)*pps, nt)); trailing slots stay empty.  A
# balanced split (nt // P tiles, one more for the first nt % P slots) gives
# different ranges for each of these contexts.
KNOWN_SLOTS = {
    # 12 tiles, runs of 2: slots 0-5 two tiles each (the last ending at 3000), 6-7 empty
    (3000, 8): [(0, 512), (512, 1024), (1024, 1536), (1536, 2048), (2048, 2560), (2560, 3000), (0, 0), (0, 0)],
    # 5 tiles, runs of 1: five one-tile slots, three empty
    (1027, 8): [(0, 256), (256, 512), (512, 768), (768, 1024), (1024, 1027), (0, 0), (0, 0), (0, 0)],
    # 157 tiles, runs of 20: seven full runs, the last slot 17 tiles
    (40000, 8): [(20 * 256 * z, 20 * 256 * (z + 1)) for z in range(7)] + [(35840, 40000)],
    # 3 tiles over 2 slots: runs of 2, then one
    (600, 2): [(0, 512), (512, 600)],
    # 9 tiles over 4 slots: runs of 3, the last slot empty
    (2100, 4): [(0, 768), (768, 1536), (1536, 2100), (0, 0)],
}


@pytest.mark.parametrize("ctx,P", sorted(KNOWN_SLOTS))
def test_slot_ranges_known_answers(ctx, P):
    want = KNOWN_SLOTS[(ctx, P)]
    assert [plan.slot_token_range(ctx, P, z) for z in range(P)] == want
    assert [_lib.plan_slot(ctx, P, z, 0, 1) for z in range(P)] == want
