"""Work-list scheduler of the persistent decode route (test infrastructure).

Pure-Python restatement of ``pa_metadata_v1_kernel``
(kernels/pa_metadata.py:145-420) and its buffer sizing
(kernels/pa_metadata.py:53-79), step for step: each loop iteration computes
the "finish" branch (the bin completes the sequence) and the "split" branch
(the bin takes what it can and closes) and selects one, as the reference
does, and every store the reference makes unconditionally is made here too.
Buffers start at zero (the reference's are uninitialised; only the valid
prefixes are meaningful).

Also: ``merge_plan``, which replays a work list on the CPU -- each work's
partial attention over its partition range, merged per reduce group through
the reduce maps -- so tests can check that a plan computes attention.
"""

from __future__ import annotations

from typing import Dict, List, Sequence

import numpy as np

WORK_INFO_FIELDS = 8


def worklist_sizes(batch_size: int, num_head_k: int, num_cu: int):
    """(max_works, max_split_tiles) of kernels/pa_metadata.py:53-79."""
    max_work = (batch_size + num_cu - 1) * num_head_k
    max_split_tiles = min(batch_size + num_cu - 1, (num_cu - 1) * 2)
    return max_work, max_split_tiles


def pa_metadata_v1(
    context_lens: Sequence[int],
    num_heads_k: int,
    gqa: int,
    query_length: int,
    num_cu: int,
    kv_granularity: int = 256,
) -> Dict[str, np.ndarray]:
    """Work list for ``num_cu`` bins (kernels/pa_metadata.py:145-420)."""
    assert num_cu % num_heads_k == 0, "num_cu must be divisible by num_heads_k"
    B = len(context_lens)
    max_work, max_split = worklist_sizes(B, num_heads_k, num_cu)
    work_indptr = np.zeros(num_cu + 1, np.int32)
    work_info = np.zeros((max(max_work, 0), WORK_INFO_FIELDS), np.int32)
    reduce_indptr = np.zeros(B + 1, np.int32)
    reduce_final_map = np.zeros((B, 2), np.int32)
    reduce_partial_map = np.zeros(max(max_split, 0), np.int32)
    out = dict(work_indptr=work_indptr, work_info=work_info, reduce_indptr=reduce_indptr,
               reduce_final_map=reduce_final_map, reduce_partial_map=reduce_partial_map, num_works=0)
    if B == 0:
        return out
    qo_indptr = [b * query_length for b in range(B + 1)]  # uniform qo lengths

    def num_part(b):  # partitions of sequence b (:173-177)
        return -(-max(int(context_lens[b]), 0) // kv_granularity)

    nspk = num_cu // num_heads_k
    sum_blocks = sum(num_part(b) for b in range(B))  # phase 1 (:196-214)
    average, reminder = divmod(sum_blocks, nspk)

    def remain_for(c):  # (:218-221)
        return average + (1 if c % nspk < reminder else 0)

    cid = 0
    num_works = 0
    lri = grt = 0
    for khead in range(num_heads_k):  # phase 2 (:228-398)
        qhr = ((khead + 1) * gqa << 16) | ((khead * gqa) & 0xFFFF)
        batch = kvblk = nsplit = pidx = kvbeg = 0
        kvend = num_part(0)
        remain = remain_for(cid)
        lri = grt = 0
        while cid < num_cu and batch < B:
            pages = kvend - kvbeg
            remain_kv = pages - kvblk
            do_finish = remain >= remain_kv
            qo_start, qo_end = qo_indptr[batch], qo_indptr[batch + 1]
            kv_start = kvbeg + kvblk
            # finish branch (:300-318)
            f_ploc = pidx if nsplit > 0 else -1
            f_pidx2 = pidx + query_length if nsplit > 0 else pidx
            f_nworks2 = num_works + 1
            f_remain2 = remain - remain_kv
            f_batch2 = batch + 1
            f_kvbeg2 = kvend
            f_kvend2 = kvend + (num_part(f_batch2) if f_batch2 < B else 0)
            # split branch (:320-329)
            s_emit = remain > 0
            s_kv_end = min(kv_start + remain, kvend)
            s_nworks2 = num_works + 1 if s_emit else num_works
            s_pidx2 = pidx + query_length if s_emit else pidx
            s_kvblk2 = kvblk + remain if s_emit else kvblk
            s_nsplit2 = nsplit + 1 if s_emit else nsplit
            s_cid2 = cid + 1
            s_remain2 = remain_for(s_cid2)
            # the work entry at slot num_works, stored every iteration (:331-343)
            work_info[num_works] = (batch, f_ploc if do_finish else pidx, qo_start, qo_end, kv_start,
                                    kvend if do_finish else s_kv_end, 0, qhr)
            # reduce maps (:345-374)
            do_reduce = do_finish and nsplit > 0
            num_splits = nsplit + 1
            reduce_indptr[grt + 1] = lri + num_splits
            reduce_final_map[grt] = (qo_start, qo_end)
            if do_reduce:
                for s in range(num_splits):
                    reduce_partial_map[lri + s] = pidx - (nsplit - s) * query_length
            n_lri = lri + (num_splits if do_reduce else 0)
            n_grt = grt + (1 if do_reduce else 0)
            # select (:376-393)
            cid_old = cid
            if do_finish:
                batch, kvblk, nsplit, num_works = f_batch2, 0, 0, f_nworks2
                pidx, kvbeg, kvend, remain = f_pidx2, f_kvbeg2, f_kvend2, f_remain2
            else:
                cid, kvblk, nsplit, num_works = s_cid2, s_kvblk2, s_nsplit2, s_nworks2
                pidx, remain = s_pidx2, s_remain2
            lri, grt = n_lri, n_grt
            work_indptr[cid_old + 1] = num_works  # (:395-401)
        if cid < num_cu:  # (:411-417)
            cid += 1
    for i in range(cid, num_cu + 1):  # tails (:419-437)
        work_indptr[i] = num_works
    for i in range(grt, B + 1):
        reduce_indptr[i] = lri
    # the slot after the last work may hold a non-emitted candidate; clear it
    if num_works < len(work_info):
        work_info[num_works:] = 0
    out["num_works"] = num_works
    out["num_groups"] = grt
    return out


def valid_final_map(plan) -> np.ndarray:
    return plan["reduce_final_map"][: plan["num_groups"]]


def merge_plan(plan, partial_fn, query_length: int, num_query_heads: int, gqa: int, kv_granularity: int = 256):
    """Replay a work list: returns ``out[row][qhead] -> vector`` of the
    final output, computing each work through ``partial_fn(batch, kvhead,
    tok0, tok1) -> (out [ql, gqa, D] normalised, lse [ql, gqa])`` and merging
    split works through the reduce maps as pa_reduce_v1 would."""
    work_info = plan["work_info"]
    part_base = plan["partition_base"]
    direct = {}
    partial_rows = {}
    for w in range(plan["num_works"]):
        b, ploc, qo0, _qo1, kv0, kv1, _z, qhr = (int(x) for x in work_info[w])
        qh0 = qhr & 0xFFFF
        kh = qh0 // gqa
        t0 = (kv0 - part_base[b]) * kv_granularity
        t1 = (kv1 - part_base[b]) * kv_granularity
        o, lse = partial_fn(b, kh, t0, t1)
        for qi in range(query_length):
            for g in range(gqa):
                if ploc < 0:
                    direct[(qo0 + qi, qh0 + g)] = o[qi, g]
                else:
                    partial_rows[(ploc + qi, qh0 + g)] = (o[qi, g], lse[qi, g])
    rip, fmap, pmap = plan["reduce_indptr"], plan["reduce_final_map"], plan["reduce_partial_map"]
    out = dict(direct)
    for gidx in range(plan["num_groups"]):
        qo0, qo1 = int(fmap[gidx, 0]), int(fmap[gidx, 1])
        rows = [int(pmap[i]) for i in range(rip[gidx], rip[gidx + 1])]
        for qi in range(qo1 - qo0):
            for qh in range(num_query_heads):
                items = [partial_rows[(r + qi, qh)] for r in rows if (r + qi, qh) in partial_rows]
                if not items:
                    continue
                lses = np.array([l for _, l in items], np.float64)
                m = lses.max()
                if not np.isfinite(m):
                    out[(qo0 + qi, qh)] = np.zeros_like(items[0][0])
                    continue
                w = np.exp(lses - m)
                acc = sum(wi * o for wi, (o, _) in zip(w, items))
                out[(qo0 + qi, qh)] = acc / w.sum()
    return out
