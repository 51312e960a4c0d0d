"""GPU parity of the HIP decode path against the CPU oracle.

Tolerance (from the target): bf16 outputs within atol 2e-2 / rtol 2e-2 of
the restated torch reference (torch.isclose semantics, every element, as
tests/kernels/test_pa.py:603-641 applies its tolerance).  Partition
intermediates (exp_sums, max_logits, tmp_out) are checked per slot against
the oracle's direct slot computation, which pins the slot indexing: an
empty slot must be exactly (0, -inf, 0).
"""

from __future__ import annotations

import contextlib
import math

import pytest
import torch

import ctypes

import flydsl_amd.pa_decode as pd
from flydsl_amd import _lib, pa_decode_ps_launch, prepare_pa_decode, workloads
from oracle import plan
from tests._cases import make_case, slot_partials, torch_oracle

pytestmark = pytest.mark.gpu

ATOL = 2e-2
RTOL = 2e-2
DEV = "cuda:0"


def to_dev(case, device=DEV):
    out = dict(case)
    for k, v in case.items():
        if isinstance(v, torch.Tensor):
            out[k] = v.to(device)
    return out


SCHEDULES = {
    "auto": None,
    "owner": lambda route, batch, kv_heads, P, eqgs, capacity, num_cu: P if (-(-eqgs // 16) == 1 or P <= 4) else 1,
    "slot": lambda *args: 1,
    "wave_slot": lambda route, batch, kv_heads, P, eqgs, capacity, num_cu: 4 if P >= 4 else 1,
}


@contextlib.contextmanager
def schedule(name):
    """Force the launcher's slots-per-workgroup choice (and, for a forced
    choice, keep the partition pass: no balanced stream split, and no switch
    of a generic-kernel owner launch to slots)."""
    saved = pd._schedule, pd._balanced_ok, pd._generic_owner_ok
    if SCHEDULES[name] is not None:
        pd._schedule = SCHEDULES[name]
        pd._balanced_ok = lambda *args: False
        pd._generic_owner_ok = lambda *args: True
    try:
        yield
    finally:
        pd._schedule, pd._balanced_ok, pd._generic_owner_ok = saved


def launch(case, *, P=0, out_dtype=torch.bfloat16, tmp_dtype=torch.bfloat16, flat=False, partials=False,
           sched="auto"):
    with schedule(sched):
        return _launch(case, P=P, out_dtype=out_dtype, tmp_dtype=tmp_dtype, flat=flat, partials=partials)


def _launch(case, *, P, out_dtype, tmp_dtype, flat, partials):
    q = case["query"]
    out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    kw = dict(
        sliding_window=case["sliding_window"],
        block_tables=None if flat else case["block_tables"],
        max_context_partition_num=P,
    )
    page_idx, indptr = None, None
    if flat:
        bt = case["block_tables"].cpu()
        ctx = case["context_lengths"].cpu().tolist()
        bs = case["key_cache"].shape[-2]
        rows = [bt[b, : math.ceil(c / bs)] for b, c in enumerate(ctx)]
        page_idx = torch.cat(rows).to(torch.int32).to(q.device)
        indptr = torch.tensor([0] + list(torch.tensor([len(r) for r in rows]).cumsum(0)), dtype=torch.int32,
                              device=q.device)
    es = ml = to = None
    if partials:
        b = case["context_lengths"].shape[0]
        hkv = case["key_cache"].shape[1]
        eq = case["query_length"] * (q.shape[1] // hkv)
        es = torch.full((b, hkv, P, eq), 7.0, device=q.device)
        ml = torch.full((b, hkv, P, eq), 7.0, device=q.device)
        to = torch.full((b, hkv, P, eq, q.shape[-1]), 7.0, device=q.device, dtype=tmp_dtype)
        kw.update(exp_sums=es, max_logits=ml, temporary_output=to)
    route = pa_decode_ps_launch(
        out, q, case["key_cache"], case["value_cache"], case["context_lengths"], page_idx, indptr,
        case["softmax_scale"], case["key_scale"], case["value_scale"], **kw
    )
    torch.cuda.synchronize()
    return out, route, (es, ml, to)


def launch_owner_with_partials(case, P, tmp_dtype=torch.float32):
    """Owner launch (one workgroup per (sequence, kv head) merging in LDS)
    whose C-ABI arguments carry the slot-partial buffers: the library then
    writes them as well.  The Python launcher treats caller partial buffers
    as workspace and leaves them out of owner launches, so this prepares the
    owner call and fills the partial fields of its arguments."""
    q = case["query"]
    b = case["context_lengths"].shape[0]
    hkv = case["key_cache"].shape[1]
    eq = case["query_length"] * (q.shape[1] // hkv)
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    es = torch.full((b, hkv, P, eq), 7.0, device=q.device)
    ml = torch.full((b, hkv, P, eq), 7.0, device=q.device)
    to = torch.full((b, hkv, P, eq, q.shape[-1]), 7.0, device=q.device, dtype=tmp_dtype)
    with schedule("owner"):
        call = prepare_pa_decode(out, q, case["key_cache"], case["value_cache"], case["context_lengths"], None, None,
                                 case["softmax_scale"], case["key_scale"], case["value_scale"],
                                 sliding_window=case["sliding_window"], block_tables=case["block_tables"],
                                 max_context_partition_num=P)
    pa = call._pa
    assert call._ra is None and pa.output is not None and pa.exp_sums is None
    pa.num_partitions = pa.slots_per_workgroup = P
    pa.exp_sums, pa.max_logits, pa.tmp_out = es.data_ptr(), ml.data_ptr(), to.data_ptr()
    pa.stride_es_seq, pa.stride_es_head, pa.stride_es_part = es.stride()[:3]
    pa.stride_to_seq, pa.stride_to_head, pa.stride_to_part, pa.stride_to_group = to.stride()[:4]
    pa.tmp_dtype = _lib.DTYPE_F32 if tmp_dtype == torch.float32 else _lib.DTYPE_BF16
    call.launch()
    torch.cuda.synchronize()
    return out, (es, ml, to)


def assert_parity(out, ref, what=""):
    out = out.float().cpu()
    ref = ref.float().cpu()
    bad = ~torch.isclose(out, ref, atol=ATOL, rtol=RTOL)
    err = (out - ref).abs().max().item()
    print(f"[parity] {what} max_abs_err={err:.3e} bad={int(bad.sum())}/{out.numel()}", flush=True)
    assert not torch.isnan(out).any(), what
    assert int(bad.sum()) == 0, f"{what}: {int(bad.sum())} elements outside atol/rtol {ATOL}; max err {err}"


CASES = {
    "c1_tiny": dict(config="c1_tiny"),
    "per_token": dict(per_token=True, ctx_range=(1, 700)),
    "ctx_edges": dict(ctx=[1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1023]),
    "mtp_ql4_gqa4": dict(query_length=4, num_query_heads=16, num_kv_heads=4, ctx_range=(4, 600)),
    "mtp_ql2_gqa8_pt": dict(query_length=2, num_query_heads=16, num_kv_heads=2, per_token=True, ctx_range=(2, 900)),
    "gqa16_ql4": dict(query_length=4, num_query_heads=16, num_kv_heads=1, ctx_range=(4, 1100)),
    "gqa8_ql3": dict(query_length=3, num_query_heads=8, num_kv_heads=1, ctx_range=(3, 1100), per_token=True),
    "page64": dict(block_size=64, ctx_range=(1, 2000)),
    "page64_mtp_pt": dict(block_size=64, query_length=4, num_query_heads=64, num_kv_heads=4, per_token=True,
                          ctx_range=(4, 1500)),
    "window": dict(sliding_window=300, ctx_range=(1, 2000)),
    "window_mtp_pt": dict(sliding_window=100, query_length=3, num_query_heads=16, num_kv_heads=4, per_token=True,
                          ctx_range=(3, 1500)),
    "window_page64": dict(sliding_window=513, block_size=64, ctx_range=(1, 3000)),
    "uniform_data": dict(dist="uniform", ctx_range=(1, 1500)),
}


def build(name):
    spec = dict(CASES[name])
    if "config" in spec:
        cfg = workloads.CONFIGS[spec["config"]]
        return workloads.build_inputs(cfg, device="cpu", seed=123)
    return make_case(batch=6, seed=len(name), **spec)


@pytest.mark.parametrize("sched", ["auto", "owner", "slot", "wave_slot"])
@pytest.mark.parametrize("name", sorted(CASES))
def test_decode_matches_oracle(name, sched):
    case = build(name)
    ref = torch_oracle(case, float_out=False)
    out, route, _ = launch(to_dev(case), sched=sched)
    exp_route = "ps_sw_partitioned" if case["sliding_window"] else "ps_small_block"
    assert route == exp_route
    assert_parity(out, ref, f"{name}/{sched}")


@pytest.mark.parametrize("sched", ["owner", "slot", "wave_slot"])
@pytest.mark.parametrize("P", [1, 2, 3, 5, 8, 13])
def test_any_partition_count(P, sched):
    case = make_case(batch=5, ctx_range=(1, 3000), per_token=True, seed=P)
    ref = torch_oracle(case, float_out=False)
    out, _, _ = launch(to_dev(case), P=P, sched=sched)
    assert_parity(out, ref, f"P={P}/{sched}")


FOUR_WAVE_VARIANTS = {
    "plain": dict(),
    "per_token": dict(per_token=True),
    "window": dict(sliding_window=150),
    "page64": dict(block_size=64),
}


@pytest.mark.parametrize("sched", ["owner", "slot", "wave_slot"])
@pytest.mark.parametrize("variant", sorted(FOUR_WAVE_VARIANTS))
def test_grids_beyond_one_workgroup_per_cu(variant, sched):
    """260+ workgroups (more than one per CU) keep two 4-wave workgroups per
    CU; the small cases above launch at most one workgroup per CU and so run
    8-wave workgroups."""
    case = make_case(batch=130, ctx_range=(1, 600), seed=47 + len(variant), **FOUR_WAVE_VARIANTS[variant])
    ref = torch_oracle(case, float_out=False)
    out, _, _ = launch(to_dev(case), P=8, sched=sched)
    assert_parity(out, ref, f"4-wave {variant}/{sched}")


@pytest.mark.parametrize("window", [2, 100, 700])
def test_window_fused_and_partitioned(window):
    case = make_case(batch=5, ctx=[1, 60, 255, 900, 2500], sliding_window=window, seed=21 + window)
    ref = torch_oracle(case, float_out=False)
    out, route, _ = launch(to_dev(case), P=1)
    assert route == "ps_sw_fused_partitioned"
    assert_parity(out, ref, f"fused W={window}")
    out2, route2, _ = launch(to_dev(case))
    assert route2 == "ps_sw_partitioned"
    assert_parity(out2, ref, f"window W={window} P=auto")


def test_flat_page_list_route():
    case = make_case(batch=5, block_size=1024, ctx_range=(1, 5000), per_token=True, seed=31)
    ref = torch_oracle(case, float_out=False)
    out, route, _ = launch(to_dev(case), flat=True)
    assert route == "ps_split_reduce"
    assert_parity(out, ref, "page1024 flat")


def test_plain_value_layout_and_dtypes():
    case = make_case(batch=4, block_size=64, ctx_range=(1, 1000), seed=41)
    ref = torch_oracle(case, float_out=True)
    from oracle.torch_ref import unshuffle_value_cache_layout

    d = to_dev(case)
    d["value_cache"] = unshuffle_value_cache_layout(case["value_cache"].view(torch.uint8)).view(
        torch.float8_e4m3fn).to(DEV)
    out, _, _ = launch(d, out_dtype=torch.float32, tmp_dtype=torch.float32, P=4, partials=True)
    assert_parity(out, ref, "plain V, f32 out/tmp")
    d["query"] = d["query"].to(torch.float16)
    out16, _, _ = launch(d, out_dtype=torch.float16)
    assert_parity(out16, ref, "f16 query/out")


@pytest.mark.parametrize("sched", ["owner", "slot", "wave_slot"])
@pytest.mark.parametrize("window,ql", [(0, 1), (0, 3), (200, 1), (150, 2)])
def test_slot_partials_match_oracle(window, ql, sched):
    """exp_sums / max_logits / tmp_out per slot: same cells as the oracle,
    whichever way the slots are spread over workgroups and waves."""
    case = make_case(batch=5, query_length=ql, num_query_heads=8, num_kv_heads=2, ctx=[ql, 100, 256, 700, 1500],
                     sliding_window=window, per_token=True, seed=51 + ql)
    P = plan.sw_partition_count(window, query_length=ql) if window else 6
    es_r, ml_r, to_r = slot_partials(case, P)
    if sched == "owner":
        _, (es, ml, to) = launch_owner_with_partials(to_dev(case), P)
    else:
        _, _, (es, ml, to) = launch(to_dev(case), P=P, partials=True, tmp_dtype=torch.float32, sched=sched)
    es, ml, to = es.cpu().double(), ml.cpu().double(), to.cpu().double()
    empty = torch.isinf(ml_r)
    assert torch.equal(torch.isinf(ml), empty), "non-empty slot set differs"
    assert bool((es[empty] == 0).all()) and bool((to[empty.unsqueeze(-1).expand_as(to)] == 0).all())
    full = ~empty
    torch.testing.assert_close(ml[full], ml_r[full], atol=1e-2, rtol=0)
    # exp_sums are relative to the slot max: compare the product s * e^m
    torch.testing.assert_close(es[full] * torch.exp(ml[full] - ml_r[full]), es_r[full], rtol=2e-2, atol=1e-3)
    torch.testing.assert_close(to[full.unsqueeze(-1).expand_as(to)], to_r[full.unsqueeze(-1).expand_as(to_r)],
                               atol=ATOL, rtol=RTOL)


def test_graph_capture_replays_match_eager():
    case = to_dev(make_case(batch=4, ctx_range=(1, 2000), seed=61))
    b = case["context_lengths"].shape[0]
    P = 8
    es = torch.empty((b, 2, P, 4), device=DEV)
    ml = torch.empty_like(es)
    to = torch.empty((b, 2, P, 4, 128), device=DEV, dtype=torch.bfloat16)
    out = torch.empty(case["query"].shape, dtype=torch.bfloat16, device=DEV)

    def call():
        pa_decode_ps_launch(out, case["query"], case["key_cache"], case["value_cache"], case["context_lengths"],
                            None, None, case["softmax_scale"], case["key_scale"], case["value_scale"],
                            block_tables=case["block_tables"], max_context_partition_num=P, exp_sums=es,
                            max_logits=ml, temporary_output=to)

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        call()  # eager work between replays
        torch.cuda.synchronize()


def _subcase(case, seqs):
    """Compact CPU copy of a few sequences (their pages only) for the oracle."""
    bs = case["key_cache"].shape[-2]
    ctx = case["context_lengths"].cpu()
    bt = case["block_tables"].cpu()
    ql = case["query_length"]
    pages, rows = [], []
    for b in seqs:
        n = math.ceil(int(ctx[b]) / bs)
        rows.append(list(range(len(pages), len(pages) + n)))
        pages.extend(bt[b, :n].tolist())
    idx = torch.tensor(pages, dtype=torch.long, device=case["key_cache"].device)
    width = max(len(r) for r in rows)
    sub = dict(case)
    sub["key_cache"] = case["key_cache"].index_select(0, idx).cpu()
    sub["value_cache"] = case["value_cache"].index_select(0, idx).cpu()
    if case["key_scale"].dim() > 1:
        sub["key_scale"] = case["key_scale"].index_select(0, idx).cpu()
        sub["value_scale"] = case["value_scale"].index_select(0, idx).cpu()
    else:
        sub["key_scale"] = case["key_scale"].cpu()
        sub["value_scale"] = case["value_scale"].cpu()
    sub["block_tables"] = torch.tensor([r + [0] * (width - len(r)) for r in rows], dtype=torch.int32)
    sub["context_lengths"] = ctx[list(seqs)].to(torch.int32)
    sub["query"] = torch.cat([case["query"][b * ql : (b + 1) * ql].cpu() for b in seqs])
    return sub


# Share of each full-size configuration's sequences checked against the
# oracle: every sequence of every configuration.
FULL_SIZE_SHARE = {"c2_llama8b": 1.0, "c3_ragged": 1.0, "c4_window": 1.0, "c5_mtp": 1.0}


@pytest.mark.parametrize("name", ["c2_llama8b", "c3_ragged", "c4_window", "c5_mtp"])
def test_benchmark_config_full_size(name):
    """Full BASELINE shapes on the GPU; the oracle checks FULL_SIZE_SHARE of
    the sequences (always the first, last, longest and shortest, the rest
    seeded at random), 16 sequences per oracle call."""
    cfg = workloads.CONFIGS[name]
    print(f"[full-size] {name}: building inputs", flush=True)
    case = workloads.build_inputs(cfg, device=DEV, seed=7)
    out, route, _ = launch(case)
    assert not torch.isnan(out).any()
    ctx = case["context_lengths"].cpu()
    want = math.ceil(FULL_SIZE_SHARE[name] * cfg.batch)
    pick = {0, cfg.batch - 1, int(ctx.argmax()), int(ctx.argmin())}
    order = torch.randperm(cfg.batch, generator=torch.Generator().manual_seed(0)).tolist()
    for b in order:
        if len(pick) >= want:
            break
        pick.add(b)
    seqs = sorted(pick)
    ql = cfg.query_length
    for i in range(0, len(seqs), 16):
        part = seqs[i : i + 16]
        ref = torch_oracle(_subcase(case, part), float_out=False)
        got = torch.cat([out[b * ql : (b + 1) * ql].cpu() for b in part])
        assert_parity(got, ref, f"{name} seqs={part}")
        print(f"[full-size] {name}: sequences {part[0]}..{part[-1]} match", flush=True)
    print(f"[full-size] {name}: route {route}, {len(seqs)} of {cfg.batch} sequences checked", flush=True)


@pytest.mark.parametrize("P", [4, 6, 9])
def test_owner_launch_matches_two_pass_reduce(P):
    """One launch that merges in LDS (owner workgroups) == partition pass
    with one slot per workgroup + pa_fp8_decode_reduce; same partials (the
    owner launch writes them when its C-ABI arguments carry them), and the
    Python launcher's owner launch leaves caller buffers untouched."""
    case = to_dev(make_case(batch=6, ctx_range=(1, 3000), per_token=P != 9, query_length=2 if P != 9 else 1,
                            num_query_heads=16 if P != 9 else 8, num_kv_heads=4 if P != 9 else 2, seed=71 + P))
    ref = torch_oracle({k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in case.items()},
                       float_out=False)
    out1, (es1, ml1, to1) = launch_owner_with_partials(case, P)
    out2, _, (es2, ml2, to2) = launch(case, P=P, partials=True, sched="slot", tmp_dtype=torch.float32)
    out3, _, (es3, ml3, to3) = launch(case, P=P, partials=True, sched="owner", tmp_dtype=torch.float32)
    assert_parity(out1, ref, f"owner P={P}")
    assert_parity(out3, ref, f"owner via launcher P={P}")
    assert bool((es3 == 7.0).all()) and bool((ml3 == 7.0).all()) and bool((to3 == 7.0).all())
    assert_parity(out2, ref, f"slot+reduce P={P}")
    assert torch.equal(torch.isinf(ml1), torch.isinf(ml2))
    fin = ~torch.isinf(ml1)
    torch.testing.assert_close(ml1[fin], ml2[fin], atol=1e-4, rtol=1e-5)
    torch.testing.assert_close(es1[fin], es2[fin], atol=1e-3, rtol=1e-3)
    torch.testing.assert_close(to1, to2, atol=2e-3, rtol=2e-3)


def test_owner_launch_without_partials_writes_only_output():
    case = to_dev(make_case(batch=4, ctx_range=(1, 2000), seed=77))
    ref = torch_oracle({k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in case.items()},
                       float_out=False)
    with schedule("owner"):
        call = prepare_pa_decode(torch.empty(case["query"].shape, dtype=torch.bfloat16, device=DEV), case["query"],
                                 case["key_cache"], case["value_cache"], case["context_lengths"], None, None,
                                 case["softmax_scale"], case["key_scale"], case["value_scale"],
                                 block_tables=case["block_tables"], max_context_partition_num=8)
    assert call._ra is None and call._pa.exp_sums is None
    call.launch()
    torch.cuda.synchronize()
    assert_parity(call._keep[0], ref, "owner, output only")


OWNER_PAIR_CASES = {
    # 768 (sequence, kv head) pairs, three per CU; empty sequences
    "pairs3_empty": dict(num_query_heads=32, num_kv_heads=8,
                         ctx=[0 if i % 7 == 3 else 1 + (37 * i) % 400 for i in range(96)]),
    # 2400 pairs, several dispatch rounds; per-token scales
    "pairs8_pt": dict(batch=300, num_query_heads=8, num_kv_heads=8, ctx_range=(1, 120), per_token=True),
    # 64-token pages under a window
    "pairs2_page64_window": dict(batch=70, num_query_heads=16, num_kv_heads=8, ctx_range=(1, 900), block_size=64,
                                 sliding_window=200),
    # two causal queries per sequence (four columns)
    "pairs5_ql2": dict(batch=150, query_length=2, num_query_heads=16, num_kv_heads=8, ctx_range=(2, 500)),
}


@pytest.mark.parametrize("name", sorted(OWNER_PAIR_CASES))
def test_fused_owner_many_pairs(name):
    """Fused owner calls (no partial buffers) with more (sequence, kv head)
    pairs than CUs, so several workgroups share a CU or run in later rounds.
    Empty sequences give zero rows."""
    spec = OWNER_PAIR_CASES[name]
    case = make_case(seed=len(name), **spec)
    ctx = case["context_lengths"]
    ref = torch_oracle(dict(case, context_lengths=ctx.clamp(min=1)), float_out=False)
    ql = case["query_length"]
    for b in torch.nonzero(ctx == 0).flatten().tolist():
        ref[b * ql:(b + 1) * ql] = 0
    out, route, _ = launch(to_dev(case), sched="owner")
    assert route == ("ps_sw_partitioned" if case["sliding_window"] else "ps_small_block")
    assert_parity(out, ref, f"owner pairs/{name}")


def test_fused_owner_graph_replays():
    """A captured fused owner launch replays bit for bit."""
    case = to_dev(make_case(batch=80, num_query_heads=32, num_kv_heads=8, ctx_range=(1, 700), seed=83))
    out = torch.empty(case["query"].shape, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    with schedule("owner"):
        call = prepare_pa_decode(out, case["query"], case["key_cache"], case["value_cache"], case["context_lengths"],
                                 None, None, case["softmax_scale"], case["key_scale"], case["value_scale"],
                                 block_tables=case["block_tables"], max_context_partition_num=8, stream=s)
    assert call._ra is None and call._pa.exp_sums is None
    with torch.cuda.stream(s):
        call.launch()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call.launch()
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        with torch.cuda.stream(s):
            call.launch()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"eager after replay {i}"


@pytest.mark.parametrize("sched", ["owner", "slot"])
def test_graph_capture_every_schedule(sched):
    case = to_dev(make_case(batch=5, ctx_range=(1, 2500), seed=81, per_token=True))
    P = 8
    b = 5
    es = torch.empty((b, 2, P, 4), device=DEV)
    ml = torch.empty_like(es)
    to = torch.empty((b, 2, P, 4, 128), device=DEV, dtype=torch.bfloat16)
    out = torch.empty(case["query"].shape, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()

    def call():
        return pa_decode_ps_launch(out, case["query"], case["key_cache"], case["value_cache"],
                                   case["context_lengths"], None, None, case["softmax_scale"], case["key_scale"],
                                   case["value_scale"], block_tables=case["block_tables"],
                                   max_context_partition_num=P, exp_sums=es, max_logits=ml, temporary_output=to)

    with schedule(sched):
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
        with schedule(sched):
            with torch.cuda.stream(s):
                call()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"eager after replay {i}"


@pytest.mark.parametrize("softmax_scale,neg_key_scale", [(-0.09, False), (0.0, False), (0.09, True), (-0.05, True)])
@pytest.mark.parametrize("shape", ["gqa4", "mtp_gqa16_pt"])
def test_negative_and_zero_logit_scales(softmax_scale, neg_key_scale, shape):
    """The logit factor (softmax scale x per-tensor key scale) may be negative
    or zero: the kernels fold its sign into the queries (and a zero factor
    gives uniform attention over the visible keys).  Every schedule, the
    balanced split and, for 64 columns, the cooperative kernel."""
    spec = dict(gqa4=dict(batch=5, ctx=[1, 40, 300, 2100, 5000]),
                mtp_gqa16_pt=dict(batch=4, query_length=4, num_query_heads=64, num_kv_heads=4, block_size=64,
                                  per_token=True, ctx=[4, 100, 1500, 4100]))[shape]
    case = make_case(seed=301, **spec)
    case["softmax_scale"] = softmax_scale
    if neg_key_scale and case["key_scale"].dim() == 1:
        case["key_scale"] = -case["key_scale"]
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    for sched in ("auto", "slot", "owner"):
        out, route, _ = launch(d, sched=sched)
        assert_parity(out, ref, f"scale={softmax_scale} negk={neg_key_scale} {shape} {sched} {route}")
