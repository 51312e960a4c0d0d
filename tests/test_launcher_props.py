"""Property tests of the launcher's host logic on the CPU: for random valid
shapes (head sizes 64-256, 1-4 query rows, GQA 1-32, windows, per-token
scales, partition counts, caller partials, CU counts), prepare_pa_decode
accepts the call, picks one of the reference's route strings, marshals the
head size into every kernel's arguments, keeps the balanced split to the
shapes it is built for, pairs every slot launch with a reduce over the
same slots, and launches the generic kernels as owners over several slots
only where their waves fill the GPU.  Nothing is launched."""

from __future__ import annotations

import math

import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import flydsl_amd.pa_decode as pd
from flydsl_amd import prepare_pa_decode
from tests._cases import make_case

ROUTES = {"ps_small_block", "ps_split_reduce", "ps_sw_partitioned", "ps_sw_fused_partitioned"}


class StubStream:
    cuda_stream = 0


@st.composite
def calls(draw):
    head = draw(st.sampled_from([64, 128, 192, 256]))
    hkv = draw(st.sampled_from([1, 2, 4, 8]))
    gqa = draw(st.sampled_from([1, 2, 4, 8, 16, 32]))
    ql = draw(st.integers(1, 4))
    batch = draw(st.integers(1, 12))
    bs = draw(st.sampled_from([16, 64]))
    ctx = draw(st.lists(st.integers(ql, 700), min_size=batch, max_size=batch))
    window = draw(st.sampled_from([0, 0, 1, 100, 600]))
    per_token = draw(st.booleans())
    partials = draw(st.booleans())
    p_req = draw(st.sampled_from([0, 0, 1, 2, 5, 8, 13]))
    num_cu = draw(st.sampled_from([1, 4, 32, 256]))
    seed = draw(st.integers(0, 1000))
    return dict(head=head, hkv=hkv, gqa=gqa, ql=ql, bs=bs, ctx=ctx, window=window, per_token=per_token,
                partials=partials, p_req=p_req, num_cu=num_cu, seed=seed)


@settings(max_examples=150, deadline=None, database=None, suppress_health_check=[HealthCheck.too_slow])
@given(calls())
def test_random_calls_marshal_consistently(c):
    case = make_case(batch=len(c["ctx"]), ctx=c["ctx"], query_length=c["ql"], num_query_heads=c["hkv"] * c["gqa"],
                     num_kv_heads=c["hkv"], block_size=c["bs"], per_token=c["per_token"],
                     sliding_window=c["window"], head_size=c["head"], seed=c["seed"])
    B, hkv, D, ql, W = len(c["ctx"]), c["hkv"], c["head"], c["ql"], c["window"]
    eq = ql * c["gqa"]
    P = c["p_req"]
    if W > 0:
        # the window route needs enough slots for the window (the launcher
        # raises otherwise, as tested elsewhere); 0 lets it choose
        need = math.ceil((W + ql - 1) / 256) + 1
        if 1 < P < need:
            P = need
    if c["partials"] and P == 0:
        # caller buffers are sized for an explicit slot count
        P = 4 if W == 0 else math.ceil((W + ql - 1) / 256) + 1
    kw = dict(max_context_partition_num=P, sliding_window=W)
    if c["partials"]:
        kw.update(exp_sums=torch.empty(B, hkv, P, eq), max_logits=torch.empty(B, hkv, P, eq),
                  temporary_output=torch.empty(B, hkv, P, eq, D, dtype=torch.bfloat16))
    saved = pd._cu_count
    pd._cu_count = lambda device=None: c["num_cu"]
    try:
        out = torch.empty(case["query"].shape, dtype=torch.bfloat16)
        call = prepare_pa_decode(out, case["query"], case["key_cache"], case["value_cache"],
                                 case["context_lengths"], None, None, case["softmax_scale"], case["key_scale"],
                                 case["value_scale"], stream=StubStream(), block_tables=case["block_tables"], **kw)
    finally:
        pd._cu_count = saved
    assert call.route in ROUTES
    assert call.route.startswith("ps_sw") == (W > 0)
    generic = D != 128 or eq > 64
    if generic:
        assert getattr(call, "_sa", None) is None, "the balanced split is built for D = 128, <= 64 columns"
    if call._sa is not None:
        return  # balanced split: its own checks (test_launcher.py)
    pa = call._pa
    assert pa is not None and pa.head_size == D
    owner = pa.slots_per_workgroup >= pa.num_partitions
    if call._ra is not None:
        # slot launch: the reduce merges exactly its slots
        assert not owner
        assert call._ra.head_size == D and call._ra.num_partitions == pa.num_partitions
    else:
        # no reduce: one owner launch per (sequence, kv head) writes the output
        assert owner
        if generic and pa.num_partitions > 1:
            # a generic owner launch over several slots only where its waves fill the GPU
            assert pd._generic_owner_ok(B, hkv, eq, c["num_cu"])
