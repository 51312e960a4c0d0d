"""Stale page bytes never reach the output.

Page slots that no query of a sequence sees -- the tail of its last page
past the context, slots before a sliding window, pages of no sequence -- may
hold any byte in a real KV pool (torch.empty pages, recycled pages),
e4m3fn NaN (0x7f / 0xff) included, and a zero probability does not cancel
a NaN in the value product.  Every such slot is filled with NaN here (key
and value bytes 0x7f, per-token scales NaN) after the oracle has run on the
clean pool; the visible bytes are unchanged, so the output must match the
oracle's at the usual tolerance (bf16 within atol 2e-2 / rtol 2e-2) on
every route: the partition schedules, the balanced split (per-wave stream
and cooperative kernels) and the work list (bin and cooperative kernels).
"""

from __future__ import annotations

import pytest
import torch

import flydsl_amd.pa_decode as pd
from oracle import plan
from tests._cases import make_case, torch_oracle
from tests.test_gpu_parity import assert_parity, launch
from tests.test_gpu_stream import balanced, cu_count, flat_pages, run, to_dev

NAN_FP8 = 0x7F


def visible_slots(case) -> torch.Tensor:
    """[pages, slots] mask of the page slots some query of some sequence sees."""
    kc = case["key_cache"]
    nb, bs = kc.shape[0], kc.shape[-2]
    seen = torch.zeros(nb, bs, dtype=torch.bool)
    ql, w = case["query_length"], case["sliding_window"]
    bt = case["block_tables"].cpu()
    for b, c in enumerate(case["context_lengths"].cpu().tolist()):
        lo, _ = plan.visible_token_range(c, 0, ql, w)
        _, hi = plan.visible_token_range(c, ql - 1, ql, w)
        if hi <= lo:
            continue
        t = torch.arange(lo, hi)
        seen[bt[b, t // bs].long(), t % bs] = True
    return seen


def poison_stale(case) -> int:
    """NaN into every slot no sequence sees (CPU case, in place); returns
    the number of poisoned slots."""
    stale = ~visible_slots(case)
    kc = case["key_cache"].view(torch.uint8)  # [pages, kv heads, D / 16, slots, 16]
    vc = case["value_cache"].view(torch.uint8)  # [pages, kv heads, slots / 16, D, 16]
    nb, _, _, bs, _ = kc.shape
    kc.permute(0, 3, 1, 2, 4)[stale] = NAN_FP8
    vc.permute(0, 2, 4, 1, 3)[stale.view(nb, bs // 16, 16)] = NAN_FP8
    if case["key_scale"].dim() > 1:  # per token: [pages, kv heads, slots, 1]
        case["key_scale"].permute(0, 2, 1, 3)[stale] = float("nan")
        case["value_scale"].permute(0, 2, 1, 3)[stale] = float("nan")
    return int(stale.sum())


def test_poison_hits_only_stale_slots():
    """The poisoning itself: visible bytes unchanged, every other slot NaN."""
    case = make_case(batch=3, query_length=2, per_token=True, ctx=[5, 40, 70], sliding_window=20, seed=3)
    clean = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    n = poison_stale(case)
    seen = visible_slots(clean)
    assert n == int((~seen).sum()) > 0
    kc, kc0 = case["key_cache"].view(torch.uint8), clean["key_cache"].view(torch.uint8)
    vis = seen[:, None, None, :, None].expand_as(kc)
    assert torch.equal(kc[vis], kc0[vis])
    assert bool((kc[~vis] == NAN_FP8).all())
    # the poison has teeth: a product over whole pages with zero
    # probabilities for the invisible slots (the oracle's) turns NaN
    assert torch.isnan(torch_oracle(case, float_out=False).float()).any()
    assert not torch.isnan(torch_oracle(clean, float_out=False).float()).any()


CASES = {
    # per-wave stream kernel (4 query columns per kv head)
    "gqa4_pt_edges": dict(batch=8, per_token=True, ctx=[1, 17, 31, 33, 250, 1000, 2049, 3001]),
    # cooperative kernel: two waves (32 columns, two-chunk units)
    "coop2_ql2_gqa16": dict(batch=5, query_length=2, num_query_heads=32, num_kv_heads=2, ctx=[2, 33, 300, 1025, 2500]),
    # cooperative kernel: four waves (64 columns, four-chunk units)
    "coop4_ql4_gqa16_pt": dict(batch=6, query_length=4, num_query_heads=64, num_kv_heads=4, per_token=True,
                               ctx=[4, 31, 129, 700, 1500, 4100]),
    "coop4_page64_pt": dict(batch=5, query_length=4, num_query_heads=64, num_kv_heads=4, per_token=True,
                            block_size=64, ctx=[4, 65, 200, 1000, 3000]),
    # window edges: stale slots before the window too
    "window_ql3_pt": dict(batch=5, query_length=3, num_query_heads=16, num_kv_heads=4, per_token=True,
                          sliding_window=100, ctx=[3, 70, 500, 1500, 2000]),
    "window_coop4": dict(batch=4, query_length=4, num_query_heads=64, num_kv_heads=4, sliding_window=200,
                         ctx=[4, 150, 900, 2600]),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_stale_nan_bytes_on_every_route(name):
    case = make_case(seed=400 + len(name), extra_pages=3, **CASES[name])
    ref = torch_oracle(case, float_out=False)
    n = poison_stale(case)
    print(f"[stale] {name}: {n} poisoned slots ctx={case['context_lengths'].tolist()}", flush=True)
    d = to_dev(case)
    for sched in ("auto", "owner", "slot", "wave_slot"):
        out, route, _ = launch(d, sched=sched)
        assert_parity(out, ref, f"stale {name} {sched} {route}")
    for num_cu in (None, 2):
        with balanced(num_cu):
            out, route = run(d)
        assert_parity(out, ref, f"stale {name} balanced cu={num_cu} {route}")


WORKLIST_CASES = {
    "gqa4_pt": dict(batch=5, per_token=True, ctx=[1, 700, 1025, 3000, 6000]),
    "coop_ql4_gqa16_pt": dict(batch=4, query_length=4, num_query_heads=64, num_kv_heads=4, per_token=True,
                              ctx=[4, 1000, 2049, 5000]),
    "coop_gqa32": dict(batch=4, num_query_heads=32, num_kv_heads=1, ctx=[1, 1023, 1025, 7000]),
}


@pytest.mark.gpu
@pytest.mark.parametrize("num_cu", [None, 2])
@pytest.mark.parametrize("name", sorted(WORKLIST_CASES))
def test_stale_nan_bytes_work_list(name, num_cu):
    case = make_case(block_size=1024, seed=500 + len(name), extra_pages=2, **WORKLIST_CASES[name])
    ref = torch_oracle(case, float_out=False)
    n = poison_stale(case)
    print(f"[stale] worklist {name} cu={num_cu}: {n} poisoned slots", flush=True)
    d = to_dev(case)
    pages = flat_pages(case)
    hq, hkv = case["query"].shape[1], case["key_cache"].shape[1]
    with cu_count(num_cu):
        md = pd.get_pa_metadata(d["query"], d["key_cache"], d["context_lengths"], pages[1], hq, hkv)
        out, route = run(d, flat=True, metadata=md, pages=pages)
    assert route == "ps_split_reduce"
    assert_parity(out, ref, f"stale worklist {name} cu={num_cu}")
