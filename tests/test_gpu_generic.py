"""GPU parity of the generic decode kernels against the CPU oracle.

Head sizes other than 128 (64, 192, 256, 320, 384, 448, 512) and more than 64 query columns
per kv head (query_length * gqa up to 128 here) -- shapes the reference's
routes take (kernels/pa_decode_fp8.py:2084-2085, 2101, 3058) -- run on the
library's generic kernels behind the same entry points.  Every route of
pa_decode_ps_launch is exercised: the small-block route under each
schedule (owner launches, one slot per workgroup, four slots per
workgroup), the sliding-window routes (partitioned and fused), the flat
page list with and without the persistent route's work list, the slot
partials (exp_sums / max_logits / tmp_out) cell by cell, the plain value
layout and f32 / f16 outputs.  Tolerance as everywhere: bf16 outputs
within atol 2e-2 / rtol 2e-2 of the oracle, every element.
"""

from __future__ import annotations

import contextlib

import pytest
import torch

import flydsl_amd.pa_decode as pd
from oracle import plan
from oracle.torch_ref import unshuffle_value_cache_layout
from tests._cases import make_case, slot_partials, torch_oracle
import tests.test_gpu_parity as tp
from tests.test_gpu_parity import assert_parity, launch, launch_owner_with_partials, to_dev
from tests.test_gpu_stream import cu_count, flat_pages, run

pytestmark = pytest.mark.gpu

ATOL = RTOL = 2e-2

SHAPES = {
    "d64": dict(head_size=64, num_query_heads=8, num_kv_heads=2),
    "d64_mtp_pt": dict(head_size=64, query_length=3, num_query_heads=16, num_kv_heads=4, per_token=True),
    "d192_pt": dict(head_size=192, num_query_heads=16, num_kv_heads=2, per_token=True),
    "d256": dict(head_size=256, num_query_heads=8, num_kv_heads=1),
    "d256_mtp_pt": dict(head_size=256, query_length=2, num_query_heads=32, num_kv_heads=4, per_token=True),
    "eq128": dict(query_length=8, num_query_heads=32, num_kv_heads=2),  # 8 x gqa 16
    "eq128_pt": dict(query_length=4, num_query_heads=64, num_kv_heads=2, per_token=True),  # 4 x gqa 32
    "eq80_d256": dict(head_size=256, query_length=5, num_query_heads=32, num_kv_heads=2),
    "eq128_d64_pt": dict(head_size=64, query_length=2, num_query_heads=128, num_kv_heads=2, per_token=True),
    # head sizes above 256: one chunk buffer per wave
    "d320": dict(head_size=320, num_query_heads=8, num_kv_heads=2),
    "d384_mtp_pt": dict(head_size=384, query_length=2, num_query_heads=16, num_kv_heads=4, per_token=True),
    "d448_pt": dict(head_size=448, num_query_heads=16, num_kv_heads=2, per_token=True),
    "d512": dict(head_size=512, num_query_heads=8, num_kv_heads=1),
    "d512_mtp_pt": dict(head_size=512, query_length=3, num_query_heads=24, num_kv_heads=2, per_token=True),
}


def build(name, **kw):
    spec = dict(SHAPES[name])
    spec.update(kw)
    ql = spec.get("query_length", 1)
    spec.setdefault("ctx", [ql, ql + 30, 255, 700, 1601])
    spec["ctx"] = [max(c, ql) for c in spec["ctx"]]  # a sequence holds at least its new tokens
    return make_case(batch=len(spec["ctx"]), seed=900 + len(name), **spec)


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_small_block_route_every_schedule(name):
    case = build(name)
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    for sched in ("auto", "owner", "slot", "wave_slot"):
        out, route, _ = launch(d, sched=sched)
        assert route == "ps_small_block"
        assert_parity(out, ref, f"{name} {sched}")


@pytest.mark.parametrize("name", ["d64_mtp_pt", "d256", "eq128", "eq128_d64_pt"])
@pytest.mark.parametrize("P", [1, 3, 8, 13])
def test_any_partition_count(name, P):
    case = build(name, block_size=64, ctx=[5, 64, 1000, 2049, 3000])
    ref = torch_oracle(case, float_out=False)
    out, _, _ = launch(to_dev(case), P=P, sched="slot")
    assert_parity(out, ref, f"{name} P={P}")


@pytest.mark.parametrize("name", ["d64_mtp_pt", "d192_pt", "d256_mtp_pt", "eq128_pt", "d320", "d512_mtp_pt"])
@pytest.mark.parametrize("window", [1, 100, 600])
def test_window_routes(name, window):
    case = build(name, sliding_window=window, ctx=[8, 90, 700, 2100])
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    out, route, _ = launch(d, P=1)
    assert route == "ps_sw_fused_partitioned"
    assert_parity(out, ref, f"{name} fused W={window}")
    out, route, _ = launch(d)
    assert route == "ps_sw_partitioned"
    assert_parity(out, ref, f"{name} W={window}")


@contextlib.contextmanager
def owner_for_any_shape():
    """The owner schedule for every column count (the generic kernels
    walk any number of slots per wave; the tuned ones limit that)."""
    saved = tp.SCHEDULES["owner"]
    tp.SCHEDULES["owner"] = lambda route, batch, kv_heads, P, *rest: P
    try:
        yield
    finally:
        tp.SCHEDULES["owner"] = saved


@pytest.mark.parametrize("name", ["d64", "d256_mtp_pt", "eq128", "eq80_d256", "d320", "d512_mtp_pt"])
@pytest.mark.parametrize("sched", ["owner", "slot"])
def test_slot_partials_match_oracle(name, sched):
    case = build(name, ctx=[3, 100, 256, 700, 1500])
    P = 5
    es_r, ml_r, to_r = slot_partials(case, P)
    if sched == "owner":
        with owner_for_any_shape():
            _, (es, ml, to) = launch_owner_with_partials(to_dev(case), P)
    else:
        _, _, (es, ml, to) = launch(to_dev(case), P=P, partials=True, tmp_dtype=torch.float32, sched=sched)
    es, ml, to = es.cpu().double(), ml.cpu().double(), to.cpu().double()
    empty = torch.isinf(ml_r)
    assert torch.equal(torch.isinf(ml), empty), "non-empty slot set differs"
    assert bool((es[empty] == 0).all()) and bool((to[empty.unsqueeze(-1).expand_as(to)] == 0).all())
    full = ~empty
    torch.testing.assert_close(ml[full], ml_r[full], atol=1e-2, rtol=0)
    torch.testing.assert_close(es[full] * torch.exp(ml[full] - ml_r[full]), es_r[full], rtol=2e-2, atol=1e-3)
    f5 = full.unsqueeze(-1)
    torch.testing.assert_close(to[f5.expand_as(to)], to_r[f5.expand_as(to_r)], atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("name", ["d64_mtp_pt", "d192_pt", "d256", "eq128_pt", "eq80_d256", "d320", "d448_pt",
                                  "d512_mtp_pt"])
@pytest.mark.parametrize("num_cu", [None, 3])
def test_flat_pages_work_list_and_partitions(name, num_cu):
    """Page size 1024: the persistent route's work list (get_pa_metadata,
    work-list decode, reduce) and, without metadata, the partition pass
    over the flat page list."""
    case = build(name, block_size=1024, ctx=[4, 1000, 1025, 5000])
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    pages = flat_pages(case)
    hq, hkv = case["query"].shape[1], case["key_cache"].shape[1]
    with cu_count(num_cu):
        md = pd.get_pa_metadata(d["query"], d["key_cache"], d["context_lengths"], pages[1], hq, hkv)
        md["partial_output"].fill_(float("nan"))
        out, route = run(d, flat=True, metadata=md, pages=pages)
        assert route == "ps_split_reduce"
        assert_parity(out, ref, f"{name} work list cu={num_cu}")
        out, route = run(d, flat=True, pages=pages)
        assert route == "ps_split_reduce"
        assert_parity(out, ref, f"{name} flat partitions cu={num_cu}")


@pytest.mark.parametrize("name", ["d64_mtp_pt", "d256", "eq128_pt", "d384_mtp_pt", "d512"])
def test_plain_value_layout_and_dtypes(name):
    case = build(name, block_size=64, ctx=[2, 64, 500, 1300])
    ref = torch_oracle(case, float_out=True)
    d = to_dev(case)
    d["value_cache"] = unshuffle_value_cache_layout(case["value_cache"].view(torch.uint8)).view(
        torch.float8_e4m3fn).to(d["query"].device)
    out, _, _ = launch(d, out_dtype=torch.float32, tmp_dtype=torch.float32, P=4, partials=True)
    assert_parity(out, ref, f"{name} plain V, f32 out/tmp")
    d["query"] = d["query"].to(torch.float16)
    out16, _, _ = launch(d, out_dtype=torch.float16)
    assert_parity(out16, ref, f"{name} f16 query/out")


def test_window_plan_matches_for_generic_heads():
    """The window route's slot count is the reference's for any head size."""
    case = build("d256", sliding_window=300, ctx=[10, 2000])
    out, route, _ = launch(to_dev(case))
    assert route == "ps_sw_partitioned"
    ref = torch_oracle(case, float_out=False)
    assert_parity(out, ref, "d256 window plan")
    assert plan.sw_partition_count(300, query_length=1) >= 2


@pytest.mark.parametrize("name", ["d64_mtp_pt", "d256"])
@pytest.mark.parametrize("partials", [False, True])
def test_graph_capture_replays(name, partials):
    """Graph replays of the generic kernels equal the eager call, with caller
    partials (slot launch + reduce) and without them (owner launch, one pass
    over each (sequence, kv head); capture without partials needs the owner
    schedule, so it is forced for this small batch, otherwise the launcher
    raises as the reference does); eager calls run between the replays."""
    with tp.schedule("owner") if not partials else contextlib.nullcontext():
        _graph_replays(name, partials)


def _graph_replays(name, partials):
    case = to_dev(build(name))
    q = case["query"]
    B, Hkv, D = len(case["context_lengths"]), case["key_cache"].shape[1], q.shape[-1]
    eq = (q.shape[0] // B) * (q.shape[1] // Hkv)
    P = 5
    kw = {}
    if partials:
        kw = dict(exp_sums=torch.empty((B, Hkv, P, eq), device=q.device),
                  max_logits=torch.empty((B, Hkv, P, eq), device=q.device),
                  temporary_output=torch.empty((B, Hkv, P, eq, D), device=q.device, dtype=torch.bfloat16))
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    s = torch.cuda.Stream()

    def call():
        return pd.pa_decode_ps_launch(out, q, case["key_cache"], case["value_cache"], case["context_lengths"], None,
                                      None, case["softmax_scale"], case["key_scale"], case["value_scale"],
                                      block_tables=case["block_tables"], max_context_partition_num=P, **kw)

    with torch.cuda.stream(s):
        call()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"{name} replay {i}"
        with torch.cuda.stream(s):
            call()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"{name} eager after replay {i}"
