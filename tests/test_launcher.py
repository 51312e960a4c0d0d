"""Host-side launcher logic without a GPU: validation errors mirror the
reference launcher (kernels/pa_decode_fp8.py:1862-1919, 2859-2863,
3014-3018, 3030-3034), the schedule choice, and the C-ABI arguments it
marshals (checked field by field on a stub stream; nothing is launched)."""

from __future__ import annotations

import pytest
import torch

import flydsl_amd.pa_decode as pd
from flydsl_amd import prepare_pa_decode, workloads
from tests._cases import make_case


class StubStream:
    cuda_stream = 0


@pytest.fixture(autouse=True)
def no_device(monkeypatch):
    monkeypatch.setattr(pd, "_cu_count", lambda device=None: 256)


def prep(case, **kw):
    out = kw.pop("output", None)
    if out is None:
        out = torch.empty(case["query"].shape, dtype=torch.bfloat16)
    return prepare_pa_decode(out, case["query"], case["key_cache"], case["value_cache"], case["context_lengths"],
                             kw.pop("kv_page_indices", None), kw.pop("kv_indptr", None), case["softmax_scale"],
                             case["key_scale"], case["value_scale"], stream=StubStream(),
                             block_tables=kw.pop("block_tables", case["block_tables"]), **kw)


def test_small_block_slot_mode_marshalling():
    # 8 query columns per kv head: beyond the balanced split's limit
    case = make_case(batch=3, ctx=[10, 300, 1000], num_query_heads=16, per_token=True, seed=1)
    call = prep(case)
    a = call._pa
    assert call.route == "ps_small_block"
    assert a.num_partitions == 8 and a.slots_per_workgroup in (1, 4)
    assert call._ra is not None  # partials + reduce launch
    assert a.per_token_kv == 1 and a.trans_v == 1 and a.block_size == 16
    assert a.num_seqs == 3 and a.num_kv_heads == 2 and a.query_group_size == 8 and a.query_length == 1
    assert a.stride_k_block == case["key_cache"].stride(0)
    assert a.stride_ks_block == case["key_scale"].stride(0) and a.stride_ks_head == case["key_scale"].stride(1)
    assert a.output is None  # slot mode: the reduce writes the output
    assert call._ra.num_partitions == 8


def test_owner_mode_for_large_uniform_batch():
    cfg = workloads.DecodeConfig("x", 64, 1, 32, 8, 16, "fixed:64", False)
    case = workloads.build_inputs(cfg, device="cpu", seed=0, context_lengths=[4096] * 64)
    call = prep(case)
    # nobody observes the partials: four contiguous slots, one per wave
    assert call._pa.slots_per_workgroup == call._pa.num_partitions == 4
    assert call._ra is None and call._pa.output is not None
    assert call._pa.exp_sums is None  # caller passed no partial buffers


def test_owner_mode_leaves_caller_workspace_unused():
    """Caller partial buffers are workspace (the reference preallocates them
    for graph capture); an owner launch merges in LDS and needs none."""
    cfg = workloads.DecodeConfig("x", 64, 1, 32, 8, 16, "fixed:64", False)
    case = workloads.build_inputs(cfg, device="cpu", seed=0, context_lengths=[4096] * 64)
    es = torch.empty(64, 8, 8, 4)
    call = prep(case, max_context_partition_num=8, exp_sums=es, max_logits=torch.empty_like(es),
                temporary_output=torch.empty(64, 8, 8, 4, 128, dtype=torch.bfloat16))
    assert call._ra is None and call._pa.exp_sums is None and call._pa.output is not None
    # ... but they are validated as on the slot routes
    with pytest.raises(ValueError, match="exp_sums/max_logits must have shape"):
        prep(case, max_context_partition_num=8, exp_sums=es[:, :4], max_logits=torch.empty_like(es[:, :4]),
             temporary_output=torch.empty(64, 8, 8, 4, 128, dtype=torch.bfloat16))


def test_schedule_policy():
    # long contexts or few (sequence, kv head) pairs: slot mode
    assert pd._schedule("small", 128, 8, 8, 4, 27000, 256) == 1
    assert pd._schedule("small", 8, 8, 8, 4, 4096, 256) == 4
    assert pd._schedule("small", 64, 8, 8, 4, 4096, 256) == 8
    assert pd._schedule("sw", 32, 8, 17, 4, 32768, 256) == 17
    assert pd._schedule("sw", 16, 8, 17, 4, 32768, 256) == 4
    assert pd._schedule("small", 256, 4, 4, 64, 8192, 256) == 4
    assert pd._schedule("small", 256, 4, 8, 64, 8192, 256) == 1  # 4 column groups: no multi-slot waves
    assert pd._schedule("flat", 64, 8, 8, 4, None, 256) == 1
    assert pd._schedule("small", 4, 2, 1, 4, 512, 256) == 1


def test_window_route_and_fused_single_slot():
    case = make_case(batch=2, ctx=[500, 900], sliding_window=100, seed=2)
    call = prep(case, sliding_window=100)
    assert call.route == "ps_sw_partitioned" and call._pa.sliding_window == 100
    assert call._pa.num_partitions == 2  # cdiv(100 + 1 - 1, 256) + 1
    call1 = prep(case, sliding_window=100, max_context_partition_num=1)
    assert call1.route == "ps_sw_fused_partitioned" and call1._ra is None and call1._pa.exp_sums is None


def test_flat_route_uses_page_list():
    case = make_case(batch=2, block_size=1024, ctx=[100, 3000], seed=3)
    pages = torch.tensor([0, 1, 2, 3], dtype=torch.int32)
    indptr = torch.tensor([0, 1, 4], dtype=torch.int32)
    call = prep(case, block_tables=None, kv_page_indices=pages, kv_indptr=indptr)
    assert call.route == "ps_split_reduce"
    assert call._sa.kv_indptr == indptr.data_ptr() and call._sa.block_tables == pages.data_ptr()
    assert call._sa.max_blocks_per_seq == 4
    # with slot partials requested: the partition pass over the same list
    es = torch.empty(2, 2, 4, 4)
    call2 = prep(case, block_tables=None, kv_page_indices=pages, kv_indptr=indptr, max_context_partition_num=4,
                 exp_sums=es, max_logits=torch.empty_like(es),
                 temporary_output=torch.empty(2, 2, 4, 4, 128, dtype=torch.bfloat16))
    assert call2._pa.kv_indptr == indptr.data_ptr() and call2._pa.block_tables == pages.data_ptr()


def test_balanced_split_marshalling():
    """Ragged batch, nobody reads the slot partials: balanced stream split
    over every resident wave, workspace sized by the library."""
    from flydsl_amd import _lib

    case = make_case(batch=5, ctx=[3, 900, 17000, 40, 2500], per_token=True, seed=9)
    call = prep(case)
    assert call.route == "ps_small_block" and call._pa is None and call._wra is None
    sa = call._sa
    assert sa.num_workers == 256 * 2 * 4
    assert sa.kv_indptr is None and sa.stride_bt_seq == case["block_tables"].stride(0)
    assert sa.max_blocks_per_seq == case["block_tables"].shape[1]
    assert sa.per_token_kv == 1 and sa.query_group_size == 4 and sa.num_seqs == 5
    assert sa.stride_ks_block == case["key_scale"].stride(0)
    assert call._ws.numel() == _lib.balanced_workspace_bytes(5, 2, 1, 4, sa.num_workers)
    # requested partials, or more columns than the split takes: partition pass
    es = torch.empty(5, 2, 8, 4)
    call2 = prep(case, exp_sums=es, max_logits=torch.empty_like(es),
                 temporary_output=torch.empty(5, 2, 8, 4, 128, dtype=torch.bfloat16))
    assert call2._sa is None and call2._pa is not None


def test_worklist_route_marshalling():
    case = make_case(batch=3, block_size=1024, ctx=[100, 3000, 5000], seed=10)
    pages = torch.arange(0, 9, dtype=torch.int32)
    indptr = torch.tensor([0, 1, 4, 9], dtype=torch.int32)
    md = pd.get_pa_metadata(case["query"], case["key_cache"], case["context_lengths"], indptr, 8, 2)
    call = prep(case, block_tables=None, kv_page_indices=pages, kv_indptr=indptr, metadata=md)
    assert call.route == "ps_split_reduce"
    sa, wr = call._sa, call._wra
    assert sa.work_indptr == md["work_indptr"].data_ptr() and sa.work_info == md["work_info_flat"].data_ptr()
    assert sa.partition_indptr == md["partition_indptr"].data_ptr() and sa.num_workers == md["num_sm"]
    assert sa.stride_po_row == 8 * 128 and sa.stride_pl_row == 8
    # the reduce reads from partial row query_length on
    assert wr.partial_output == md["partial_output"].data_ptr() + 1 * 8 * 128 * 4
    assert wr.partial_lse == md["partial_lse"].data_ptr() + 1 * 8 * 4
    assert wr.num_groups == 3 and wr.num_query_heads == 8 and wr.max_query_length == 1
    with pytest.raises(ValueError, match="missing"):
        prep(case, block_tables=None, kv_page_indices=pages, kv_indptr=indptr, metadata={"num_sm": 4})


def test_rejects_packed_fp8_query():
    case = make_case(batch=1, ctx=[10], seed=4)
    case["query"] = case["query"].to(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="no longer accepts host query_scale"):
        prep(case)


def test_rejects_bad_dtypes_and_shapes():
    case = make_case(batch=1, ctx=[10], seed=5)
    with pytest.raises(ValueError, match="Unsupported query dtype"):
        c = dict(case)
        c["query"] = case["query"].float()
        prep(c)
    with pytest.raises(ValueError, match="Unsupported output dtype"):
        prep(case, output=torch.empty(case["query"].shape, dtype=torch.int32))
    with pytest.raises(ValueError, match="requires `block_tables`"):
        prep(case, block_tables=None)
    with pytest.raises(ValueError, match="must be int32"):
        prep(case, block_tables=case["block_tables"].long())
    c = dict(case)
    c["query"] = torch.zeros(1, 8, 64, dtype=torch.bfloat16)
    with pytest.raises((ValueError, NotImplementedError)):
        prep(c, output=torch.empty(1, 8, 64, dtype=torch.bfloat16))


def test_rejects_too_few_window_slots():
    case = make_case(batch=1, ctx=[5000], sliding_window=1000, seed=6)
    with pytest.raises(ValueError, match="cannot cover a window"):
        prep(case, sliding_window=1000, max_context_partition_num=2)


def test_partial_buffer_shape_checked():
    case = make_case(batch=2, ctx=[10, 20], seed=7)
    es = torch.empty(2, 2, 3, 4)
    with pytest.raises(ValueError, match="exp_sums/max_logits must have shape"):
        prep(case, max_context_partition_num=8, exp_sums=es, max_logits=torch.empty_like(es),
             temporary_output=torch.empty(2, 2, 3, 4, 128, dtype=torch.bfloat16))


def test_prepared_call_is_freed_without_the_cycle_collector():
    """A dropped call releases its buffers at once (its launch thunks do not
    refer back to it), so per-step workspaces are reused, not reallocated."""
    import gc
    import weakref

    case = make_case(batch=5, ctx=[3, 900, 17000, 40, 2500], seed=11)
    call = prep(case)
    assert call._ws is not None
    ref = weakref.ref(call._ws)
    gc.disable()
    try:
        del call
        assert ref() is None
    finally:
        gc.enable()


@pytest.mark.parametrize("d,ql,hq,hkv", [(64, 1, 8, 2), (256, 2, 16, 4), (128, 8, 32, 2), (192, 1, 64, 1)])
def test_generic_shapes_take_the_partition_routes(d, ql, hq, hkv):
    """Head sizes other than 128 and more than 64 columns per kv head are
    accepted (the library's generic kernels take them) and never use the
    balanced split, which is built for D = 128 and up to 64 columns."""
    case = make_case(batch=3, ctx=[ql, 300, 1000], query_length=ql, num_query_heads=hq, num_kv_heads=hkv,
                     head_size=d, seed=2)
    call = prep(case)
    assert call.route == "ps_small_block"
    assert call._pa is not None and call._pa.head_size == d
    assert getattr(call, "_sa", None) is None
    if call._ra is not None:
        assert call._ra.head_size == d
    call = prep(case, sliding_window=100)
    assert call.route in ("ps_sw_partitioned", "ps_sw_fused_partitioned") and call._pa.head_size == d


def test_generic_owner_needs_enough_waves(monkeypatch):
    """The generic kernels' owner launch runs one wave per (sequence, kv head,
    16-column block); below 8 such waves per CU the launcher takes slot mode
    plus the reduce instead, even where the D = 128 kernels would take owner."""
    assert not pd._generic_owner_ok(64, 8, 4, 256)  # C2's batch: 512 waves on 256 CUs
    assert pd._generic_owner_ok(256, 8, 4, 256)
    assert pd._generic_owner_ok(128, 8, 32, 256)  # 2 column blocks per pair
    # 512 (sequence, kv head) pairs with short contexts: owner for D = 128
    case = make_case(batch=64, ctx=[40] * 64, num_query_heads=32, num_kv_heads=8, seed=4, head_size=128)
    call = prep(case, max_context_partition_num=4)
    assert call._ra is None
    case = make_case(batch=64, ctx=[40] * 64, num_query_heads=32, num_kv_heads=8, seed=4, head_size=64)
    call = prep(case, max_context_partition_num=4)
    assert call._pa.head_size == 64 and call._ra is not None and call._ra.head_size == 64
    monkeypatch.setattr(pd, "_generic_owner_ok", lambda *args: True)
    call = prep(case, max_context_partition_num=4)
    assert call._ra is None


def test_unbuilt_head_size_is_not_implemented():
    case = make_case(batch=1, ctx=[10], seed=5, head_size=64)
    c = dict(case)
    c["query"] = torch.zeros(1, 8, 576, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="head_dim=576"):
        prep(c, output=torch.empty(1, 8, 576, dtype=torch.bfloat16))


@pytest.mark.parametrize("d", [320, 384, 448, 512])
def test_large_head_sizes_take_the_generic_routes(d):
    """Head sizes 320 .. 512 (multiples of 64, as the reference's routes
    take) run on the generic kernels through every route."""
    case = make_case(batch=2, ctx=[5, 700], head_size=d, seed=3)
    call = prep(case)
    assert call.route == "ps_small_block" and call._pa.head_size == d
    call = prep(case, sliding_window=100)
    assert call._pa.head_size == d


def _empty_case(**kw):
    """A validated case with its batch cut to zero sequences."""
    case = make_case(batch=1, ctx=[10], seed=8, **kw)
    hq, d = case["query"].shape[1:]
    case["query"] = torch.zeros(0, hq, d, dtype=torch.bfloat16)
    case["context_lengths"] = case["context_lengths"][:0]
    case["block_tables"] = case["block_tables"][:0]
    return case


@pytest.mark.parametrize("kw,route", [
    ({}, "ps_small_block"),
    ({"sliding_window": 100}, "ps_sw_partitioned"),
    ({"sliding_window": 100, "max_context_partition_num": 1}, "ps_sw_fused_partitioned"),
])
def test_empty_batch_launches_nothing(kw, route):
    """Zero sequences: validated as usual, no kernel, the route string back
    (the reference's launcher divides by the batch size there)."""
    case = _empty_case()
    call = prep(case, **kw)
    assert call.kernels() == [] if call._lib is not None else call._kernels == []
    assert call.launch() == route
    out = torch.empty(0, 8, 128, dtype=torch.bfloat16)
    got = pd.pa_decode_ps_launch(out, case["query"], case["key_cache"], case["value_cache"],
                                 case["context_lengths"], None, None, case["softmax_scale"], case["key_scale"],
                                 case["value_scale"], block_tables=case["block_tables"], stream=StubStream(), **kw)
    assert got == route
    # still validated: a query with rows but no sequences is an error
    c = dict(case)
    c["query"] = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="multiple of the batch size"):
        prep(c, output=torch.empty(2, 8, 128, dtype=torch.bfloat16))


def test_empty_batch_flat_route():
    case = _empty_case(block_size=1024)
    call = prep(case, block_tables=None, kv_page_indices=torch.zeros(0, dtype=torch.int32),
                kv_indptr=torch.zeros(1, dtype=torch.int32))
    assert call.launch() == "ps_split_reduce"


def test_empty_inputs_of_the_other_launchers():
    """The MLA decode, the KV-cache writer and the fused RMSNorm + RoPE
    return cleanly for zero rows / tokens, before touching a device."""
    from flydsl_amd import build_fused_rope_cache_module, flydsl_mla_fwd_decode, flydsl_qk_norm_rope_quant

    fp8 = torch.float8_e4m3fn
    q = torch.zeros(0, 128, 576, dtype=fp8)
    kv = torch.zeros(4, 1, 1, 576, dtype=fp8)
    i32 = torch.int32
    assert flydsl_mla_fwd_decode(q, kv, torch.zeros(0, dtype=i32), torch.zeros(2, dtype=i32),
                                 torch.zeros(1, 8, dtype=i32), torch.zeros(0, 128, 512, dtype=torch.bfloat16),
                                 torch.zeros(0, 1, 128, 512), torch.zeros(0, 1, 128, 1), 0.1) is None

    launch = build_fused_rope_cache_module(head_dim=128, num_q_heads=4, num_kv_heads=1, block_size=16,
                                           flash_layout=False, apply_scale=True)
    bf = torch.bfloat16
    z = lambda *s, dt=bf: torch.zeros(*s, dtype=dt)  # noqa: E731
    kc, vc = z(8, 1, 8, 16, 16, dt=fp8), z(8, 1, 1, 128, 16, dt=fp8)
    launch(z(0, 4, 128), z(0, 1, 128), z(0, 1, 128), z(0, dt=i32), z(64, 64), z(64, 64), z(0, dt=i32), kc, vc,
           z(0, 4, 128), z(0, 1, 128), 0, torch.ones(1), torch.ones(1))

    qo, kvo, qs, kvs = flydsl_qk_norm_rope_quant(
        z(0, 2 * 512), z(0, 512), torch.ones(512, dtype=bf), z(16, 32), z(16, 32), z(0, dt=torch.int64),
        num_q_heads=2, head_dim=512, rope_head_dim=64, quant=True, quant_group_size=128)
    assert qo.shape == (0, 2, 512) and kvo.shape == (0, 512) and qs.shape == (0, 2, 4) and kvs.shape == (0, 4)
