"""The MLA launcher's argument checks (kernels/mla_fwd_decode.py:57-167) and
the host work-list calls, on the CPU (no kernel runs here)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from flydsl_amd import _lib
from flydsl_amd.mla_decode import (
    flydsl_mla_fwd_decode,
    get_mla_metadata_info_v1,
    get_mla_metadata_v1,
    mla_reduce_v1,
)

FP8 = torch.float8_e4m3fn


def args(B=2, heads=128, dim=576, pages=10, npart=4, qdt=FP8, kvdt=FP8, kv_shape=None):
    q = torch.zeros(B, heads, dim, dtype=qdt)
    kv = torch.zeros(kv_shape or (pages, 1, 1, 576), dtype=kvdt)
    return dict(query=q, kv_buffer=kv, kv_page_indices=torch.zeros(pages, dtype=torch.int32),
                work_indptr=torch.zeros(5, dtype=torch.int32), work_info_set=torch.zeros(4, 8, dtype=torch.int32),
                final_output=torch.zeros(B, heads, 512, dtype=torch.bfloat16),
                split_output=torch.zeros(npart, 1, heads, 512), split_lse=torch.zeros(npart, 1, heads, 1),
                softmax_scale=0.04)


def test_unsupported_shapes_raise_not_implemented():
    with pytest.raises(NotImplementedError, match="num_heads=64"):
        flydsl_mla_fwd_decode(**args(heads=64))
    with pytest.raises(NotImplementedError):
        flydsl_mla_fwd_decode(**args(qdt=torch.bfloat16))


@pytest.mark.parametrize("kw,msg", [
    (dict(dim=512), "head_dim=512"),
    (dict(kv_shape=(10, 2, 1, 576)), "page_size\\*num_kv_heads must be 1"),
    (dict(kv_shape=(10, 1, 1, 512)), "kv_buffer: head_dim=512"),
])
def test_shape_assertions(kw, msg):
    with pytest.raises(AssertionError, match=msg):
        flydsl_mla_fwd_decode(**args(**kw))


def test_output_checks():
    a = args()
    a["final_output"] = torch.zeros(3, 128, 512, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="final_output"):
        flydsl_mla_fwd_decode(**a)
    a = args()
    a["split_lse"] = torch.zeros(3, 1, 128, 1)
    with pytest.raises(AssertionError, match="split_lse batch dim"):
        flydsl_mla_fwd_decode(**a)
    a = args()
    a["final_output"] = torch.zeros(128, 2, 512, dtype=torch.bfloat16).transpose(0, 1)
    with pytest.raises(AssertionError, match="contiguous"):
        flydsl_mla_fwd_decode(**a)


def test_cpu_tensors_fail_loudly():
    with pytest.raises(RuntimeError, match="GPU"):
        flydsl_mla_fwd_decode(**args())


def test_metadata_info_sizes():
    sizes = get_mla_metadata_info_v1(33, 1, 128, FP8, FP8, num_cu=256)
    mw, mp = _lib.mla_plan_sizes(33, 256)
    assert [s for s, _ in sizes] == [(4,), (257,), (mw, 8), (34,), (33, 2), (mp,)]
    assert all(t == torch.int32 for _, t in sizes)
    with pytest.raises(NotImplementedError):
        get_mla_metadata_info_v1(4, 1, 64, FP8, FP8, num_cu=8)


def test_metadata_fill_matches_planner():
    lens = [700, 3, 0, 4000]
    B = len(lens)
    qo = torch.arange(B + 1, dtype=torch.int32)
    kv = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    sizes = get_mla_metadata_info_v1(B, 1, 128, FP8, FP8, num_cu=8)
    meta, wp, wi, ri, rf, rp = [torch.full(s, -5, dtype=t) for s, t in sizes]
    get_mla_metadata_v1(qo, kv, torch.ones(B, dtype=torch.int32), 128, 1, False, meta, wi, wp, ri, rf, rp)
    n, ng, npart, out = _lib.mla_plan(qo.numpy(), kv.numpy(), 8)
    assert meta.tolist() == [n, ng, npart, 8]
    assert wp.tolist() == out["work_indptr"].tolist()
    assert wi[:n].tolist() == out["work_info"][:n].tolist() and (wi[n:] == 0).all()
    assert ri.tolist() == out["reduce_indptr"].tolist()
    with pytest.raises(ValueError, match="kv_last_page_lens"):
        get_mla_metadata_v1(qo, kv, torch.full((B,), 2, dtype=torch.int32), 128, 1, False, meta, wi, wp, ri, rf,
                            rp)
    with pytest.raises(NotImplementedError):
        get_mla_metadata_v1(qo, kv, torch.ones(B, dtype=torch.int32), 64, 2, False, meta, wi, wp, ri, rf, rp)


def test_reduce_needs_gpu():
    with pytest.raises(RuntimeError, match="GPU"):
        mla_reduce_v1(torch.zeros(2, 1, 128, 512), torch.zeros(2, 1, 128, 1), torch.zeros(3, dtype=torch.int32),
                      torch.zeros(2, 2, dtype=torch.int32), torch.zeros(2, dtype=torch.int32), 1,
                      torch.zeros(2, 128, 512, dtype=torch.bfloat16))
