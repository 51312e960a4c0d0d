"""The allocation-free balanced decode (pa_fp8_decode_balanced_static,
which takes its workspace from the library's static device scratch) against
the entry points it stands for (pa_fp8_decode_balanced + pa_fp8_merge_balanced
with a caller workspace): same kernels, so the same bits, on two calls in a
row with the second smaller (the scratch keeps the first call's contents),
and both within atol/rtol 2e-2 of the CPU oracle."""

from __future__ import annotations

import ctypes

import pytest
import torch

import flydsl_amd.pa_decode as pd
from flydsl_amd import _lib
from tests._cases import make_case, torch_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _call(case, static: bool):
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    q = d["query"]
    out = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    per_token = d["key_scale"].dim() > 1
    sa = pd._stream_args(out, q, d["key_cache"], d["value_cache"], d["context_lengths"], d["block_tables"], None,
                         d["softmax_scale"], d["key_scale"], d["value_scale"], per_token, True, "bf16",
                         _lib.DTYPE_BF16)
    hkv = d["key_cache"].shape[1]
    ql = case["query_length"]
    gqa = q.shape[1] // hkv
    sa.num_workers = _lib.stream_workers(pd._cu_count(), ql, gqa, per_token)
    lib = _lib.load()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if static:
        _lib.check(lib.pa_fp8_decode_balanced_static(ctypes.byref(sa), s), "pa_fp8_decode_balanced_static")
    else:
        n = _lib.balanced_workspace_bytes(len(case["context_lengths"]), hkv, ql, gqa, sa.num_workers)
        ws = torch.empty(n, dtype=torch.uint8, device=DEV)
        _lib.check(lib.pa_fp8_decode_balanced(ctypes.byref(sa), ws.data_ptr(), n, s), "pa_fp8_decode_balanced")
        _lib.check(lib.pa_fp8_merge_balanced(ctypes.byref(sa), ws.data_ptr(), n, s), "pa_fp8_merge_balanced")
    torch.cuda.synchronize()
    return out.cpu()


CASES = [
    # first call: a ragged batch, most pairs cut across waves
    dict(batch=48, per_token=True, ctx=None, ctx_range=(1, 9000), seed=201),
    # second call, smaller: fewer, shorter sequences, per-tensor scales
    dict(batch=5, per_token=False, ctx=[1, 33, 700, 2000, 257], seed=202),
]


def test_static_scratch_matches_workspace_entry_twice():
    for i, spec in enumerate(CASES):
        case = make_case(num_query_heads=32, num_kv_heads=8, **spec)
        print(f"[no-alloc] call {i}: B={len(case['context_lengths'])} per_token={spec['per_token']}", flush=True)
        got = _call(case, static=True)
        want = _call(case, static=False)
        assert not torch.isnan(got).any()
        assert torch.equal(got, want), f"call {i}: static scratch differs from the workspace entry"
        ref = torch_oracle(case, float_out=False).float()
        assert bool(torch.isclose(got.float(), ref, atol=2e-2, rtol=2e-2).all()), f"call {i}: oracle parity"


def test_static_scratch_refuses_oversized_calls():
    case = make_case(batch=4, query_length=4, num_query_heads=64, num_kv_heads=4, block_size=64, ctx_range=(4, 300),
                     seed=203)
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    out = torch.empty(d["query"].shape, dtype=torch.bfloat16, device=DEV)
    sa = pd._stream_args(out, d["query"], d["key_cache"], d["value_cache"], d["context_lengths"], d["block_tables"],
                         None, d["softmax_scale"], d["key_scale"], d["value_scale"], False, True, "bf16",
                         _lib.DTYPE_BF16)
    sa.num_workers = 4096  # 64 columns: 256 MiB of partial rows
    rc = _lib.load().pa_fp8_decode_balanced_static(ctypes.byref(sa), None)
    assert rc == -9


def test_static_scratch_on_a_side_stream_and_in_a_graph():
    """The entry point keys its scratch on the stream's device (here a
    non-default stream, so the library asks the stream), and a HIP graph
    that captured it replays to the same bits.  The capture follows an
    uncaptured call: a device's first call looks the scratch address up."""
    case = make_case(num_query_heads=32, num_kv_heads=8, batch=6, per_token=True, ctx=[1, 40, 3000, 700, 5000, 2],
                     seed=204)
    want = _call(case, static=False)
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    out = torch.full(d["query"].shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    sa = pd._stream_args(out, d["query"], d["key_cache"], d["value_cache"], d["context_lengths"], d["block_tables"],
                         None, d["softmax_scale"], d["key_scale"], d["value_scale"], True, True, "bf16",
                         _lib.DTYPE_BF16)
    sa.num_workers = _lib.stream_workers(pd._cu_count(), 1, 4, True)
    lib = _lib.load()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    print("[no-alloc] side stream", flush=True)
    with torch.cuda.stream(side):
        _lib.check(lib.pa_fp8_decode_balanced_static(ctypes.byref(sa), ctypes.c_void_p(side.cuda_stream)),
                   "pa_fp8_decode_balanced_static")
    side.synchronize()
    assert torch.equal(out.cpu(), want)
    print("[no-alloc] graph capture", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.pa_fp8_decode_balanced_static(ctypes.byref(sa), cap)
    _lib.check(rc, "pa_fp8_decode_balanced_static (captured)")
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want), f"replay {i}"
