"""GPU parity of the per-wave streaming decodes (balanced split and work
list) against the CPU oracle, at the same tolerance as the partition pass
(bf16 outputs within atol 2e-2 / rtol 2e-2, every element).

Each case runs with the GPU's real CU count (thousands of short runs, most
pairs cut across waves) and with a tiny one (a few long runs, each crossing
many (sequence, kv head) pairs), so both the cut-and-merge and the
walk-across-pairs paths are exercised.  Work-list partials are checked row
by row against the oracle's attention over each work's partition range.
"""

from __future__ import annotations

import contextlib
import math

import numpy as np
import pytest
import torch

import flydsl_amd.pa_decode as pd
from flydsl_amd import pa_decode_ps_launch, prepare_pa_decode, workloads
from oracle import torch_ref
from tests._cases import flat_scales, make_case, torch_oracle

pytestmark = pytest.mark.gpu

ATOL = 2e-2
RTOL = 2e-2
DEV = "cuda:0"


def to_dev(case):
    return {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}


def to_cpu(case):
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}


@contextlib.contextmanager
def balanced(num_cu=None):
    """Force the balanced split (when the shape allows it) and optionally
    pretend the GPU has `num_cu` CUs (fewer, longer runs)."""
    saved = pd._balanced_ok, pd._cu_count
    pd._balanced_ok = lambda route, batch, eqgs, user_partials, owner: (
        route in ("small", "flat") and not user_partials
        and (eqgs <= pd.BALANCED_MAX_COLUMNS or pd.STREAM_MAX_COLUMNS < eqgs <= pd.COOP_MAX_COLUMNS))
    if num_cu is not None:
        pd._cu_count = lambda device=None: num_cu
    try:
        yield
    finally:
        pd._balanced_ok, pd._cu_count = saved


@contextlib.contextmanager
def cu_count(num_cu):
    saved = pd._cu_count
    if num_cu is not None:
        pd._cu_count = lambda device=None: num_cu
    try:
        yield
    finally:
        pd._cu_count = saved


def flat_pages(case):
    bt = case["block_tables"].cpu()
    ctx = case["context_lengths"].cpu().tolist()
    bs = case["key_cache"].shape[-2]
    rows = [bt[b, : math.ceil(c / bs)] for b, c in enumerate(ctx)]
    pages = torch.cat(rows).to(torch.int32)
    indptr = torch.tensor([0] + np.cumsum([len(r) for r in rows]).tolist(), dtype=torch.int32)
    return pages.to(DEV), indptr.to(DEV)


def run(case, *, flat=False, out_dtype=torch.bfloat16, metadata=None, pages=None):
    q = case["query"]
    out = torch.full(q.shape, float("nan"), dtype=out_dtype, device=DEV)
    page_idx = indptr = None
    if flat:
        page_idx, indptr = pages if pages is not None else flat_pages(case)
    route = pa_decode_ps_launch(out, q, case["key_cache"], case["value_cache"], case["context_lengths"], page_idx,
                                indptr, case["softmax_scale"], case["key_scale"], case["value_scale"],
                                sliding_window=case["sliding_window"], block_tables=None if flat else case["block_tables"],
                                metadata=metadata)
    torch.cuda.synchronize()
    return out, route


def assert_parity(out, ref, what):
    out, ref = out.float().cpu(), ref.float().cpu()
    bad = ~torch.isclose(out, ref, atol=ATOL, rtol=RTOL)
    err = (out - ref).abs().max().item()
    print(f"[parity] {what} max_abs_err={err:.3e} bad={int(bad.sum())}/{out.numel()}", flush=True)
    assert not torch.isnan(out).any(), what
    assert int(bad.sum()) == 0, f"{what}: {int(bad.sum())} outside tolerance; max err {err}"


BALANCED_CASES = {
    "c1_tiny": dict(config="c1_tiny"),
    "ragged_pt": dict(batch=12, per_token=True, ctx=[1, 5, 33, 260, 700, 1500, 3000, 7000, 9000, 40, 2, 12000]),
    "ctx_edges": dict(batch=12, ctx=[1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1023]),
    "mtp_ql4_gqa1": dict(batch=6, query_length=4, num_query_heads=4, num_kv_heads=4, ctx_range=(4, 3000)),
    "mtp_ql2_gqa2_pt": dict(batch=6, query_length=2, num_query_heads=4, num_kv_heads=2, per_token=True,
                            ctx_range=(2, 4000)),
    "gqa1": dict(batch=5, num_query_heads=8, num_kv_heads=8, ctx_range=(1, 2500)),
    # head groups of 2 over 6 kv heads and of 4 over 12 (three groups per sequence)
    "gqa4_h6_pt": dict(batch=5, num_query_heads=24, num_kv_heads=6, per_token=True, ctx=[1, 700, 33, 4000, 1500]),
    "gqa2_h12": dict(batch=4, num_query_heads=24, num_kv_heads=12, ctx=[900, 17, 2600, 5]),
    "page64_ragged": dict(batch=7, block_size=64, ctx=[1, 64, 65, 900, 4000, 130, 2049], per_token=True),
    "uniform_data": dict(batch=6, dist="uniform", ctx_range=(1, 3000)),
    # 6, 12 and 24 query columns: the merge's last 16-column block is part-filled
    "mtp_ql3_gqa2": dict(batch=6, query_length=3, num_query_heads=4, num_kv_heads=2, ctx_range=(3, 3000)),
    "mtp_ql3_gqa4_pt": dict(batch=6, query_length=3, num_query_heads=8, num_kv_heads=2, per_token=True,
                            ctx=[3, 17, 300, 1900, 4100, 6000]),
    "mtp_ql3_gqa8": dict(batch=5, query_length=3, num_query_heads=16, num_kv_heads=2, ctx_range=(3, 3500)),
    # cooperative workgroups (17..64 query columns per kv head)
    "coop_ql4_gqa16_pt_page64": dict(batch=6, query_length=4, num_query_heads=64, num_kv_heads=4, block_size=64,
                                     per_token=True, ctx_range=(4, 3000)),
    "coop_ql2_gqa16": dict(batch=5, query_length=2, num_query_heads=16, num_kv_heads=1, ctx_range=(2, 2500)),
    "coop_ql3_gqa16_pt": dict(batch=5, query_length=3, num_query_heads=32, num_kv_heads=2, per_token=True,
                              ctx=[3, 40, 700, 2100, 5000]),
    "coop_gqa32_edges": dict(batch=9, num_query_heads=32, num_kv_heads=1, ctx=[1, 2, 31, 32, 33, 255, 257, 1023, 4000]),
}


def build(spec):
    spec = dict(spec)
    if "config" in spec:
        return workloads.build_inputs(workloads.CONFIGS[spec["config"]], device="cpu", seed=123)
    return make_case(seed=sum(map(ord, str(sorted(spec.items())))) % 1000, **spec)


@pytest.mark.parametrize("num_cu", [None, 2])
@pytest.mark.parametrize("name", sorted(BALANCED_CASES))
def test_balanced_matches_oracle(name, num_cu):
    case = build(BALANCED_CASES[name])
    print(f"[balanced] {name} cu={num_cu} ctx={case['context_lengths'].tolist()[:12]}", flush=True)
    ref = torch_oracle(case, float_out=False)
    with balanced(num_cu):
        out, route = run(to_dev(case))
    assert route == "ps_small_block"
    assert_parity(out, ref, f"balanced {name} cu={num_cu}")


@pytest.mark.parametrize("num_cu", [None, 3])
def test_balanced_flat_pages_and_dtypes(num_cu):
    case = make_case(batch=5, block_size=1024, ctx=[1, 1025, 5000, 3000, 7], per_token=True, seed=131)
    ref = torch_oracle(case, float_out=True)
    d = to_dev(case)
    with balanced(num_cu):
        out, route = run(d, flat=True, out_dtype=torch.float32)
        assert route == "ps_split_reduce"
        assert_parity(out, ref, f"balanced flat f32 cu={num_cu}")
        d["query"] = d["query"].to(torch.float16)
        out16, _ = run(d, flat=True, out_dtype=torch.float16)
    assert_parity(out16, ref, f"balanced flat f16 cu={num_cu}")


def test_balanced_plain_value_layout():
    case = make_case(batch=6, block_size=64, ctx_range=(1, 3000), seed=137)
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    d["value_cache"] = torch_ref.unshuffle_value_cache_layout(case["value_cache"].view(torch.uint8)).view(
        torch.float8_e4m3fn).to(DEV)
    with balanced(5):
        out, _ = run(d)
    assert_parity(out, ref, "balanced plain V")


def test_balanced_graph_capture_replays():
    case = to_dev(make_case(batch=7, ctx_range=(1, 6000), per_token=True, seed=139))
    out = torch.empty(case["query"].shape, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    with balanced():
        call = prepare_pa_decode(out, case["query"], case["key_cache"], case["value_cache"], case["context_lengths"],
                                 None, None, case["softmax_scale"], case["key_scale"], case["value_scale"],
                                 block_tables=case["block_tables"], stream=s)
    assert call._sa is not None and call._pa is None
    with torch.cuda.stream(s):
        call.launch()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call.launch()
    torch.cuda.synchronize()
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        with torch.cuda.stream(s):
            call.launch()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"eager after replay {i}"


def test_balanced_prepared_inside_capture_replays():
    """A call prepared while capturing, with no partial buffers, takes its
    workspace from the graph's memory pool (the reference raises here); the
    graph replays to the eager result."""
    case = to_dev(make_case(batch=9, ctx_range=(1, 5000), per_token=False, seed=141))
    out = torch.empty(case["query"].shape, dtype=torch.bfloat16, device=DEV)
    args = (case["query"], case["key_cache"], case["value_cache"], case["context_lengths"], None, None,
            case["softmax_scale"], case["key_scale"], case["value_scale"])
    with balanced():
        route = pa_decode_ps_launch(out, *args, block_tables=case["block_tables"])
    torch.cuda.synchronize()
    eager = out.clone()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with balanced(), torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        assert pa_decode_ps_launch(out, *args, block_tables=case["block_tables"]) == route
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


def test_balanced_concurrent_streams():
    """Decodes on two side streams with no ordering between them (a per-wave
    and a cooperative balanced launch, each with its workspace from its own
    stream): the library holds no mutable state they could share, so each
    matches the oracle, on every one of several overlapping rounds."""
    cases = [make_case(batch=9, ctx_range=(1, 6000), per_token=True, seed=143),
             make_case(batch=5, query_length=4, num_query_heads=32, num_kv_heads=2, per_token=True,
                       ctx_range=(4, 5000), seed=147)]
    refs = [torch_oracle(c, float_out=False) for c in cases]
    devs = [to_dev(c) for c in cases]
    outs = [torch.empty(d["query"].shape, dtype=torch.bfloat16, device=DEV) for d in devs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for rnd in range(3):
        print(f"[concurrent] round {rnd}", flush=True)
        with balanced():
            for d, out, s in zip(devs, outs, streams):
                with torch.cuda.stream(s):
                    out.fill_(float("nan"))
                    pa_decode_ps_launch(out, d["query"], d["key_cache"], d["value_cache"], d["context_lengths"],
                                        None, None, d["softmax_scale"], d["key_scale"], d["value_scale"],
                                        block_tables=d["block_tables"])
        torch.cuda.synchronize()
        for i, (out, ref) in enumerate(zip(outs, refs)):
            assert_parity(out, ref, f"concurrent stream {i} round {rnd}")


WORKLIST_CASES = {
    "gqa4": dict(batch=6, ctx=[1, 300, 1025, 4096, 7000, 2500]),
    "gqa8_pt": dict(batch=5, num_query_heads=16, num_kv_heads=2, per_token=True, ctx_range=(1, 6000)),
    "ql2_gqa8": dict(batch=4, query_length=2, num_query_heads=16, num_kv_heads=2, ctx_range=(2, 5000)),
    "ql4_gqa4_pt": dict(batch=4, query_length=4, num_query_heads=8, num_kv_heads=2, per_token=True,
                        ctx_range=(4, 5000)),
    "gqa16": dict(batch=3, num_query_heads=16, num_kv_heads=1, ctx_range=(1, 9000)),
    "coop_ql4_gqa16_pt": dict(batch=4, query_length=4, num_query_heads=32, num_kv_heads=2, per_token=True,
                              ctx_range=(4, 6000)),
    "coop_gqa32": dict(batch=4, num_query_heads=32, num_kv_heads=1, ctx_range=(1, 7000)),
    # 128 output rows per reduce group (query length x query heads): the
    # reduce's eight-heads-per-wave form, after the bin kernel
    "ql2_gqa8_h64": dict(batch=5, query_length=2, num_query_heads=64, num_kv_heads=8, ctx_range=(2, 6000)),
}


@pytest.mark.parametrize("num_cu", [None, 2])
@pytest.mark.parametrize("name", sorted(WORKLIST_CASES))
def test_worklist_route_matches_oracle(name, num_cu):
    """Reference persistent route: get_pa_metadata, then the work-list
    decode writes direct rows and float32 partials + LSE; the reduce merges
    them.  Partials of split works are checked against the oracle."""
    spec = dict(WORKLIST_CASES[name])
    case = make_case(block_size=1024, seed=len(name) * 7 + 3, **spec)
    print(f"[worklist] {name} cu={num_cu} ctx={case['context_lengths'].tolist()}", flush=True)
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    pages = flat_pages(case)
    hq, hkv = case["query"].shape[1], case["key_cache"].shape[1]
    ql = case["query_length"]
    with cu_count(num_cu):
        md = pd.get_pa_metadata(d["query"], d["key_cache"], d["context_lengths"], pages[1], hq, hkv)
        md["partial_output"].fill_(float("nan"))
        out, route = run(d, flat=True, metadata=md, pages=pages)
    assert route == "ps_split_reduce"
    assert_parity(out, ref, f"worklist {name} cu={num_cu}")
    # partial rows of split works vs the oracle over the work's range
    info = md["work_info_flat"].view(-1, 8).cpu()
    n = int(md["work_indptr"][-1])
    pbase = md["partition_indptr"].cpu().tolist()
    ks, vs = flat_scales(case)
    po = md["partial_output"].cpu()
    pl = md["partial_lse"].cpu()
    checked = 0
    gqa = hq // hkv
    for w in range(n):
        b, ploc, _, _, kv0, kv1, _, qhr = info[w].tolist()
        if ploc < 0 or checked >= 6:
            continue
        kh = (qhr & 0xFFFF) // gqa
        o, l = torch_ref.range_partial(case["query"], case["key_cache"], case["value_cache"],
                                       case["block_tables"][b].tolist(), int(case["context_lengths"][b]), ks, vs, b,
                                       kh, (kv0 - pbase[b]) * 256, (kv1 - pbase[b]) * 256, case["softmax_scale"],
                                       query_length=ql)
        for qi in range(ql):
            row = ploc + ql + qi
            for g in range(gqa):
                qh = kh * gqa + g
                if math.isinf(float(l[qi, g])):
                    assert float(pl[row, 0, qh, 0]) == float("-inf")
                    continue
                torch.testing.assert_close(float(pl[row, 0, qh, 0]), float(l[qi, g]), atol=1e-2, rtol=0)
                torch.testing.assert_close(po[row, 0, qh].double(), o[qi, g], atol=ATOL, rtol=RTOL)
        checked += 1


def test_worklist_graph_capture_replays():
    case = make_case(batch=5, block_size=1024, num_query_heads=16, num_kv_heads=2, ctx_range=(1, 6000), seed=151)
    d = to_dev(case)
    pages = flat_pages(case)
    md = pd.get_pa_metadata(d["query"], d["key_cache"], d["context_lengths"], pages[1], 16, 2)
    out = torch.empty(d["query"].shape, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()

    def call():
        return pa_decode_ps_launch(out, d["query"], d["key_cache"], d["value_cache"], d["context_lengths"], pages[0],
                                   pages[1], d["softmax_scale"], d["key_scale"], d["value_scale"], metadata=md)

    with torch.cuda.stream(s):
        call()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.synchronize()
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        with torch.cuda.stream(s):
            call()
        torch.cuda.synchronize()


# The reference's own case set for this route (tests/kernels/test_pa.py:
# 1182-1207, normal_accuracy): 1024-token pages, context 1027 (or lengths
# drawn in [ql, 1027]), (8, 1) and (16, 1) heads, query lengths 1-4, both
# quantisation modes, batches 3 and 81; pages drawn with replacement
# (:713-716) and uniform(-1, 1) queries (:700).
REF_MATRIX = [(h, ql, q, b, v) for h in ((8, 1), (16, 1)) for ql in (1, 2, 3, 4) for q in ("per_token", "per_tensor")
              for b in (3, 81) for v in (False, True)]


@pytest.mark.parametrize("heads,ql,quant,batch,varlen", REF_MATRIX)
def test_reference_matrix_metadata_route(heads, ql, quant, batch, varlen):
    import random

    hq, hkv = heads
    rnd = random.Random(123 + ql * 7 + batch)
    ctx = [rnd.randint(ql, 1027) for _ in range(batch)] if varlen else [1027] * batch
    case = make_case(batch=batch, query_length=ql, num_query_heads=hq, num_kv_heads=hkv, block_size=1024, ctx=ctx,
                     per_token=quant == "per_token", seed=11 * ql + batch, dist="uniform",
                     extra_pages=3 * sum(math.ceil(c / 1024) for c in ctx))
    nb = case["key_cache"].shape[0]
    bt = case["block_tables"]
    case["block_tables"] = torch.tensor([[rnd.randrange(nb) for _ in range(bt.shape[1])] for _ in range(batch)],
                                        dtype=torch.int32)
    print(f"[ref-matrix] heads={heads} ql={ql} {quant} B={batch} varlen={varlen}", flush=True)
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    pages = flat_pages(case)
    md = pd.get_pa_metadata(d["query"], d["key_cache"], d["context_lengths"], pages[1], hq, hkv)
    assert md["num_sm"] == pd.metadata_bins(torch.cuda.get_device_properties(0).multi_processor_count, hkv)
    out, route = run(d, flat=True, metadata=md, pages=pages)
    assert route == "ps_split_reduce"
    assert_parity(out, ref, f"ref-matrix heads={heads} ql={ql} {quant} B={batch} varlen={varlen}")


def test_worklist_bins_with_many_works():
    """Three bins of ~70 works each (200 short sequences, one kv head): the
    bin kernel's pre-pass takes its works 64 at a time."""
    case = make_case(batch=200, num_query_heads=8, num_kv_heads=1, block_size=1024, ctx_range=(1, 600),
                     per_token=True, seed=171)
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    pages = flat_pages(case)
    md = pd.get_pa_metadata(d["query"], d["key_cache"], d["context_lengths"], pages[1], 8, 1, num_cu=1)
    assert md["num_sm"] == 3
    assert int(torch.diff(md["work_indptr"].cpu()).max()) > 64
    out, route = run(d, flat=True, metadata=md, pages=pages)
    assert_parity(out, ref, "worklist many works per bin")
