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


def test_get_pa_metadata_keys_and_buffers():
    """get_pa_metadata on CPU tensors: the reference's keys, buffers sized
    from the plan, the reference's CU * 3 bins rounded to the kv heads."""
    case = make_case(batch=4, block_size=1024, ctx=[100, 3000, 5000, 700], seed=95)
    md = pd.get_pa_metadata(case["query"], case["key_cache"], case["context_lengths"], None, 8, 2, num_cu=256)
    for k in ("work_indptr", "work_info_flat", "partition_indptr", "reduce_indptr", "reduce_final_map",
              "reduce_partial_map", "num_sm", "partial_output", "partial_lse", "stride_po_partial",
              "stride_pl_partial", "stride_po_ql", "stride_pl_ql", "query_length"):
        assert k in md, k
    assert md["num_sm"] == 768
    assert md["partition_indptr"].tolist() == [0, 1, 13, 33, 36]
    ref = worklist.pa_metadata_v1(case["context_lengths"].tolist(), 2, 4, 1, md["num_sm"], 256)
    n = ref["num_works"]
    assert torch.equal(md["work_info_flat"][: 8 * n], torch.from_numpy(ref["work_info"][:n].reshape(-1)))
    npart = int(ref["reduce_indptr"][-1])
    assert tuple(md["partial_output"].shape) == ((npart + 1) * 1, 1, 8, 128)
    assert tuple(md["partial_lse"].shape) == ((npart + 1) * 1, 1, 8, 1)
    assert md["stride_po_ql"] == 8 * 128 and md["stride_pl_ql"] == 8


def test_metadata_bins_are_the_references():
    """(CU * 3 // Hkv) * Hkv (kernels/pa_decode_fp8.py:1766-1771): 768 on a
    256-CU MI355X for 1, 2, 3, 4, 8 kv heads; 765 for 5."""
    for h, want in [(1, 768), (2, 768), (3, 768), (4, 768), (5, 765), (8, 768), (7, 763)]:
        assert pd.metadata_bins(256, h) == want
    assert pd.metadata_bins(304, 8) == 912  # MI300X
    assert pd.metadata_bins(1, 8) == 8


@pytest.mark.parametrize("H,ql,kind", [(8, 1, "ragged"), (4, 4, "uniform"), (1, 2, "zeros"), (2, 1, "aligned")])
def test_get_pa_metadata_bits_at_reference_bins(H, ql, kind):
    """Every buffer get_pa_metadata returns equals the restatement planned
    over 768 bins, bit for bit (valid prefixes), on a ragged 1024-page
    batch."""
    rng = np.random.default_rng(H * 31 + ql)
    B = 97
    ctx = [max(c, ql) for c in _ctxs(rng, B, kind)] if kind != "zeros" else _ctxs(rng, B, kind)
    q = torch.zeros(B * ql, H * 4, 128, dtype=torch.bfloat16)
    kc = torch.zeros(1, H, 8, 1024, 16, dtype=torch.uint8)
    cl = torch.tensor(ctx, dtype=torch.int32)
    md = pd.get_pa_metadata(q, kc, cl, None, H * 4, H, num_cu=256)
    ref = worklist.pa_metadata_v1(ctx, H, 4, ql, 768, 256)
    n = ref["num_works"]
    assert md["num_sm"] == 768
    assert torch.equal(md["work_indptr"], torch.from_numpy(ref["work_indptr"]))
    assert int(md["work_indptr"][-1]) == n
    assert torch.equal(md["work_info_flat"][: 8 * n], torch.from_numpy(ref["work_info"][:n].reshape(-1)))
    assert torch.equal(md["reduce_indptr"], torch.from_numpy(ref["reduce_indptr"]))
    g = ref["num_groups"]
    assert torch.equal(md["reduce_final_map"][:g], torch.from_numpy(ref["reduce_final_map"][:g]))
    used = int(ref["reduce_indptr"][-1])
    assert torch.equal(md["reduce_partial_map"][:used], torch.from_numpy(ref["reduce_partial_map"][:used]))
    parts = [-(-c // 256) for c in ctx]
    assert md["partition_indptr"].tolist() == [0] + np.cumsum(parts).tolist()
    assert capacity_violations(ref, ctx, H, 768, 256) == []


# ---------------------------------------------------------------------------
# Exact capacities.  kernels/pa_metadata.py:196-221 gives bin c the capacity
# average + (c % nspk < reminder) partitions (nspk = bins per kv head); the
# loop at :228-398 fills bins in order, each kv head's partitions laid end
# to end, closing a bin when its capacity is spent (a finished sequence
# leaves the rest of the capacity to the next one, :300-318), and starts the
# next kv head at the bin after its last (:411-417).  So every bin holds
# exactly min(capacity, partitions still unplaced) of one kv head, in order,
# and only a sequence with no partition yields an empty work.
# ---------------------------------------------------------------------------


def capacity_violations(plan, ctx, H, num_cu, gran):
    parts = [-(-max(c, 0) // gran) for c in ctx]
    pbase = np.concatenate([[0], np.cumsum(parts)]).astype(int)
    S = int(sum(parts))
    nspk = num_cu // H
    avg, rem = divmod(S, nspk)
    cap = lambda c: avg + (1 if c % nspk < rem else 0)
    n = plan["num_works"]
    wi, info = plan["work_indptr"], plan["work_info"][:n]
    out = []
    # expected: (kv head, load) per bin
    want = [(None, 0)] * num_cu
    c = 0
    for kh in range(H):
        left = S
        while left > 0 and c < num_cu:
            take = min(cap(c), left)
            want[c] = (kh, take)
            left -= take
            if left > 0:
                c += 1
        c += 1
    pos = [0] * H  # next cumulative partition expected, per kv head
    for c in range(num_cu):
        ws = range(int(wi[c]), int(wi[c + 1]))
        load = sum(int(info[w, 5] - info[w, 4]) for w in ws)
        if load != want[c][1]:
            out.append(("load", c, load, want[c][1]))
        for w in ws:
            b, kv0, kv1 = int(info[w, 0]), int(info[w, 4]), int(info[w, 5])
            kh = (int(info[w, 7]) & 0xFFFF) // 4
            if kv1 <= kv0:
                if parts[b] != 0:
                    out.append(("empty work", c, w, b))
                continue
            if kh != want[c][0]:
                out.append(("head", c, w, kh, want[c][0]))
            if kv0 != pos[kh]:
                out.append(("order", c, w, kv0, pos[kh]))
            pos[kh] = kv1
    for kh in range(H):
        if pos[kh] != pbase[-1]:
            out.append(("placed", kh, pos[kh], int(pbase[-1])))
    return out


@pytest.mark.parametrize("B,H,ql,kind", CASES)
def test_plan_exact_capacities(B, H, ql, kind):
    rng = np.random.default_rng(B * 7 + H * 3 + ql)
    ctx = _ctxs(rng, B, kind)
    for bins_per_head in (1, 2, 3, 7, 40, 96, 768):
        for gran in (256, 16):
            num_cu = H * bins_per_head
            p = worklist.pa_metadata_v1(ctx, H, 4, ql, num_cu, gran)
            assert capacity_violations(p, ctx, H, num_cu, gran) == [], (bins_per_head, gran)


def _mutant(old, new):
    """The restated planner with one planted mistake (test-only)."""
    import inspect
    import textwrap

    src = textwrap.dedent(inspect.getsource(worklist.pa_metadata_v1))
    assert src.count(old) == 1, old
    ns = dict(vars(worklist))
    exec(compile(src.replace(old, new), "<mutant>", "exec"), ns)
    return ns["pa_metadata_v1"]


@pytest.mark.parametrize("old,new", [
    ("do_finish = remain >= remain_kv", "do_finish = remain > remain_kv"),            # finish test slip
    ("return average + (1 if c % nspk < reminder else 0)",
     "return average + (1 if c % nspk <= reminder else 0)"),                          # one extra +1 bin
    ("return average + (1 if c % nspk < reminder else 0)",
     "return average + (1 if c < reminder else 0)"),                                  # +1 bins of head 0 only
    ("s_kv_end = min(kv_start + remain, kvend)", "s_kv_end = min(kv_start + remain + 1, kvend)"),
])
def test_capacity_invariants_catch_planted_mistakes(old, new):
    """Each planted slip breaks the exact-capacity invariants on some batch
    (the load-only bound and the tiling checks let the first three pass)."""
    bad = _mutant(old, new)
    rng = np.random.default_rng(5)
    caught = False
    for trial in range(40):
        B = int(rng.integers(3, 40))
        H = int(rng.choice([1, 2, 4, 8]))
        ctx = _ctxs(rng, B, ["uniform", "ragged", "aligned"][trial % 3])
        for bph in (3, 7, 40):
            try:
                p = bad(ctx, H, 4, 1, H * bph, 256)
            except (IndexError, ValueError):
                caught = True
                break
            if capacity_violations(p, ctx, H, H * bph, 256):
                caught = True
                break
        if caught:
            break
    assert caught
