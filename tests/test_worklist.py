"""Work-list planner of the persistent route (kernels/pa_metadata.py).

The library's host planner (pa_fp8_plan_worklist, flydsl_amd/csrc/
pa_worklist.h) is compared bit for bit with the step-for-step Python
restatement in oracle/worklist.py.  Parity with aiter's C++
get_pa_metadata_v1 itself is unpinned (aiter is absent and the reference
holds no fixtures); what pins the restatement is: the invariants the
reference's design states (work_indptr monotone, each (sequence, kv head)
tiled exactly once, partial_qo_loc = -1 iff the sequence is not cut, one
reduce group per cut sequence, bins loaded to average or average + 1), and
a replay of the plan -- each work's partial attention merged through the
reduce maps -- that must equal unsplit attention.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from flydsl_amd import _lib
import flydsl_amd.pa_decode as pd
from oracle import torch_ref, worklist
from tests._cases import flat_scales, make_case, torch_oracle


def _ctxs(rng, B, kind):
    if kind == "uniform":
        return rng.integers(1, 3000, size=B).tolist()
    if kind == "ragged":
        return np.clip(np.round(np.exp(rng.normal(np.log(700), 1.2, size=B))), 1, 20000).astype(int).tolist()
    if kind == "zeros":
        c = rng.integers(0, 1500, size=B)
        c[rng.random(B) < 0.3] = 0
        return c.tolist()
    return [256 * int(x) for x in rng.integers(0, 6, size=B)]  # partition-aligned


CASES = list(itertools.product([1, 3, 17, 64], [1, 2, 8], [1, 4], ["uniform", "ragged", "zeros", "aligned"]))


@pytest.mark.parametrize("B,H,ql,kind", CASES)
def test_library_matches_restatement(B, H, ql, kind):
    rng = np.random.default_rng(B * 131 + H * 7 + ql)
    ctx = _ctxs(rng, B, kind)
    for bins_per_head in (1, 3, 8, 40, 256):
        num_cu = H * bins_per_head
        for gran in (256, 16):
            ref = worklist.pa_metadata_v1(ctx, H, 4, ql, num_cu, gran)
            n, got = _lib.plan_worklist(ctx, H, 4, ql, num_cu, gran)
            assert n == ref["num_works"]
            assert np.array_equal(got["work_indptr"], ref["work_indptr"])
            assert np.array_equal(got["work_info"][:n], ref["work_info"][:n])
            assert np.array_equal(got["reduce_indptr"], ref["reduce_indptr"])
            g = ref["num_groups"]
            assert np.array_equal(got["reduce_final_map"][:g], ref["reduce_final_map"][:g])
            used = int(ref["reduce_indptr"][-1])
            assert np.array_equal(got["reduce_partial_map"][:used], ref["reduce_partial_map"][:used])


@pytest.mark.parametrize("B,H,ql,kind", CASES)
def test_plan_invariants(B, H, ql, kind):
    rng = np.random.default_rng(B * 977 + H + ql)
    ctx = _ctxs(rng, B, kind)
    gqa, gran = 4, 256
    parts = [-(-c // gran) for c in ctx]
    pbase = np.concatenate([[0], np.cumsum(parts)]).astype(int)
    for bins_per_head in (1, 3, 40):
        num_cu = H * bins_per_head
        p = worklist.pa_metadata_v1(ctx, H, gqa, ql, num_cu, gran)
        n = p["num_works"]
        wi, info = p["work_indptr"], p["work_info"][:n]
        assert wi[0] == 0 and wi[-1] == n and np.all(np.diff(wi) >= 0)
        # bins load: average or average + 1 partitions per kv head's bins
        avg, rem = divmod(sum(parts), bins_per_head)
        for c in range(num_cu):
            load = sum(int(info[w, 5] - info[w, 4]) for w in range(wi[c], wi[c + 1]))
            assert load <= avg + 1, (c, load, avg)
        pieces = {}
        for w in range(n):
            b, ploc, qo0, qo1, kv0, kv1, z, qhr = (int(x) for x in info[w])
            kh = (qhr & 0xFFFF) // gqa
            assert (qhr >> 16) == (kh + 1) * gqa and z == 0
            assert (qo0, qo1) == (b * ql, (b + 1) * ql)
            assert pbase[b] <= kv0 <= kv1 <= pbase[b + 1]
            pieces.setdefault((b, kh), []).append((kv0, kv1, ploc))
        for b in range(B):
            for kh in range(H):
                ps = sorted(pieces[(b, kh)])
                # tiled exactly once, in order
                assert ps[0][0] == pbase[b] and ps[-1][1] == pbase[b + 1]
                assert all(ps[i][1] == ps[i + 1][0] for i in range(len(ps) - 1))
                if len(ps) == 1:
                    assert ps[0][2] == -1
                else:
                    assert all(x[2] >= 0 for x in ps)
        # reduce groups: the cut sequences (their structure is the same for
        # every kv head), partial rows = the pieces' partial_qo_loc
        cut = sorted(b for b in range(B) if len(pieces[(b, H - 1)]) > 1)
        assert p["num_groups"] == len(cut)
        for gi, b in enumerate(cut):
            assert tuple(p["reduce_final_map"][gi]) == (b * ql, (b + 1) * ql)
            rows = p["reduce_partial_map"][p["reduce_indptr"][gi]:p["reduce_indptr"][gi + 1]].tolist()
            assert rows == [x[2] for x in sorted(pieces[(b, H - 1)])]


@pytest.mark.parametrize("ql,bins_per_head", [(1, 3), (2, 5), (1, 64)])
def test_plan_replay_equals_attention(ql, bins_per_head):
    """Each work's partial (oracle attention over its partition range) merged
    through the reduce maps is unsplit attention."""
    case = make_case(batch=5, query_length=ql, ctx=[ql, 300, 700, 1300, 2100], per_token=True, seed=91 + ql)
    H = case["key_cache"].shape[1]
    hq = case["query"].shape[1]
    gqa = hq // H
    ctx = case["context_lengths"].tolist()
    p = worklist.pa_metadata_v1(ctx, H, gqa, ql, H * bins_per_head, 256)
    parts = [-(-c // 256) for c in ctx]
    p["partition_base"] = np.concatenate([[0], np.cumsum(parts)]).astype(int)
    ks, vs = flat_scales(case)
    bt = case["block_tables"]

    def partial_fn(b, kh, t0, t1):
        o, l = torch_ref.range_partial(case["query"], case["key_cache"], case["value_cache"], bt[b].tolist(),
                                       ctx[b], ks, vs, b, kh, t0, t1, case["softmax_scale"], query_length=ql)
        return o.numpy(), l.numpy()

    got = worklist.merge_plan(p, partial_fn, ql, hq, gqa)
    ref = torch_oracle(case, float_out=True).double().numpy()
    for b in range(len(ctx)):
        for qi in range(ql):
            for qh in range(hq):
                np.testing.assert_allclose(got[(b * ql + qi, qh)], ref[b * ql + qi, qh], atol=2e-5, rtol=1e-5)


def test_planted_mistakes_break_the_replay():
    """A plan whose reduce map drops a piece, or whose work misreads its
    range, no longer reproduces attention."""
    case = make_case(batch=3, ctx=[700, 1300, 2100], seed=93)
    H = case["key_cache"].shape[1]
    hq = case["query"].shape[1]
    ctx = case["context_lengths"].tolist()
    ks, vs = flat_scales(case)
    ref = torch_oracle(case, float_out=True).double().numpy()

    def run(p, shift=0):
        p["partition_base"] = np.concatenate([[0], np.cumsum([-(-c // 256) for c in ctx])]).astype(int)

        def partial_fn(b, kh, t0, t1):
            o, l = torch_ref.range_partial(case["query"], case["key_cache"], case["value_cache"],
                                           case["block_tables"][b].tolist(), ctx[b], ks, vs, b, kh, t0 + shift,
                                           t1 + shift, case["softmax_scale"])
            return o.numpy(), l.numpy()

        got = worklist.merge_plan(p, partial_fn, 1, hq, hq // H)
        return max(np.abs(got[(b, qh)] - ref[b, qh]).max() for b in range(3) for qh in range(hq))

    p = worklist.pa_metadata_v1(ctx, H, hq // H, 1, H * 4, 256)
    assert run(dict(p)) < 1e-4
    assert run(dict(p), shift=16) > 1e-3
    bad = dict(p)
    bad["reduce_indptr"] = p["reduce_indptr"].copy()
    bad["reduce_indptr"][1:] -= 1  # first group loses its last piece
    bad["reduce_indptr"][0] = 0
    assert run(bad) > 1e-3


def test_sizes_match_reference_sizing():
    for B, H, cu in [(1, 1, 4), (64, 8, 2048), (300, 4, 768)]:
        assert _lib.worklist_sizes(B, H, cu) == worklist.worklist_sizes(B, H, cu)


def test_planner_rejects_bad_arguments():
    lib = _lib.load()
    z = np.zeros(64, np.int32)
    ptr = z.ctypes.data_as(_lib.ctypes.c_void_p)
    # num_cu not a multiple of the kv heads; granularity not a power of two
    assert lib.pa_fp8_plan_worklist(ptr, 1, 3, 4, 1, 8, 256, ptr, ptr, ptr, ptr, ptr) == -6
    assert lib.pa_fp8_plan_worklist(ptr, 1, 1, 4, 1, 8, 100, ptr, ptr, ptr, ptr, ptr) == -6
    assert lib.pa_fp8_plan_worklist(None, 1, 1, 4, 1, 8, 256, ptr, ptr, ptr, ptr, ptr) == -1


def test_get_pa_metadata_keys_and_buffers(monkeypatch):
    """get_pa_metadata on CPU tensors: the reference's keys, buffers sized
    from the plan, bins = resident waves rounded to the kv heads."""
    monkeypatch.setattr(pd, "_cu_count", lambda device=None: 256)
    case = make_case(batch=4, block_size=1024, ctx=[100, 3000, 5000, 700], seed=95)
    md = pd.get_pa_metadata(case["query"], case["key_cache"], case["context_lengths"], None, 8, 2)
    for k in ("work_indptr", "work_info_flat", "partition_indptr", "reduce_indptr", "reduce_final_map",
              "reduce_partial_map", "num_sm", "partial_output", "partial_lse", "stride_po_partial",
              "stride_pl_partial", "stride_po_ql", "stride_pl_ql", "query_length"):
        assert k in md, k
    assert md["num_sm"] == _lib.stream_workers(256, 1, 4, True) == 2048
    assert md["partition_indptr"].tolist() == [0, 1, 13, 33, 36]
    ref = worklist.pa_metadata_v1(case["context_lengths"].tolist(), 2, 4, 1, md["num_sm"], 256)
    n = ref["num_works"]
    assert torch.equal(md["work_info_flat"][: 8 * n], torch.from_numpy(ref["work_info"][:n].reshape(-1)))
    npart = int(ref["reduce_indptr"][-1])
    assert tuple(md["partial_output"].shape) == ((npart + 1) * 1, 1, 8, 128)
    assert tuple(md["partial_lse"].shape) == ((npart + 1) * 1, 1, 8, 1)
    assert md["stride_po_ql"] == 8 * 128 and md["stride_pl_ql"] == 8
