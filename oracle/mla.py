"""CPU restatement of the MLA fp8 decode (test infrastructure only).

Follows the reference test's oracle, tests/kernels/test_mla_decode.py:
  * ``ref_masked_attention`` (:77-97): logits = softmax_scale * q.k over all
    576 dims of the fp8 query and key (values taken as exact floats);
    lse = logsumexp(logits); out = softmax(logits) @ v with v the first 512
    dims of the key row;
  * ``torch_mla_extend`` (:100-131): query rows qo_indptr[b] .. qo_indptr[b+1]
    of sequence b attend kv_indices[kv_indptr[b] : kv_indptr[b+1]] (page
    size 1), no causal mask.
computed in float64 with numpy.  ``mla_split_ref`` gives the normalised
partial output and log-sum-exp of every work record (the decode's split
outputs, kernels/mla_fwd_decode_m16x8_fp8_fp8.py:1831-1838), and
``mla_reduce_ref`` the log-sum-exp merge of those partials.

Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline use this.
"""

from __future__ import annotations

import numpy as np

QK_HEAD_DIM = 576
V_HEAD_DIM = 512
NUM_HEADS = 128


def fp8_to_f64(t) -> np.ndarray:
    """torch float8_e4m3fn tensor -> float64 numpy (exact)."""
    import torch

    return t.to(torch.float32).cpu().numpy().astype(np.float64)


def attend(q: np.ndarray, k: np.ndarray, sm_scale: float):
    """q [R, H, 576], k [N, 576] float64 -> (out [R, H, 512], lse [R, H],
    wabs [R, H, 512]) where wabs = softmax-weighted mean of |v| (the scale
    of the probability-rounding error of the decode)."""
    r, h, _ = q.shape
    n = k.shape[0]
    if n == 0:
        z = np.zeros((r, h, V_HEAD_DIM))
        return z, np.full((r, h), -np.inf), z
    logits = (q.reshape(r * h, -1) @ k.T) * sm_scale  # [R*H, N]
    m = logits.max(-1, keepdims=True)
    e = np.exp(logits - m)
    s = e.sum(-1, keepdims=True)
    w = e / s
    v = k[:, :V_HEAD_DIM]
    out = (w @ v).reshape(r, h, V_HEAD_DIM)
    wabs = (w @ np.abs(v)).reshape(r, h, V_HEAD_DIM)
    lse = (m + np.log(s)).reshape(r, h)
    return out, lse, wabs


def mla_decode_ref(q, kv, qo_indptr, kv_indptr, kv_indices, sm_scale: float):
    """q [rows, 128, 576] and kv [pages, 576] float64 numpy; index arrays
    int; returns out [rows, 128, 512], lse [rows, 128], wabs."""
    rows = q.shape[0]
    out = np.zeros((rows, NUM_HEADS, V_HEAD_DIM))
    wabs = np.zeros_like(out)
    lse = np.full((rows, NUM_HEADS), -np.inf)
    for b in range(len(qo_indptr) - 1):
        r0, r1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        pages = np.asarray(kv_indices[int(kv_indptr[b]) : int(kv_indptr[b + 1])], dtype=np.int64)
        o, l, wa = attend(q[r0:r1], kv[pages], sm_scale)
        out[r0:r1], lse[r0:r1], wabs[r0:r1] = o, l, wa
    return out, lse, wabs


def mla_split_ref(q, kv, kv_indices, work_info, num_works: int, sm_scale: float):
    """Per work record w (batch, partial row, row, row + 1, kv0, kv1, ...):
    returns list of (row, partial row, out [128, 512], lse [128], wabs)."""
    res = []
    for w in range(num_works):
        _, pql, row, _, kv0, kv1 = (int(x) for x in work_info[w][:6])
        pages = np.asarray(kv_indices[kv0:kv1], dtype=np.int64)
        o, l, wa = attend(q[row : row + 1], kv[pages], sm_scale)
        res.append((row, pql, o[0], l[0], wa[0]))
    return res


def mla_reduce_ref(split_out, split_lse, reduce_indptr, reduce_final_map, reduce_partial_map, num_groups: int):
    """Merge of partial rows: returns {row: (out [128, 512], lse [128])}."""
    res = {}
    for g in range(num_groups):
        p0, p1 = int(reduce_indptr[g]), int(reduce_indptr[g + 1])
        row0, row1 = int(reduce_final_map[g][0]), int(reduce_final_map[g][1])
        for row in range(row0, row1):
            parts = [int(reduce_partial_map[i]) + row - row0 for i in range(p0, p1)]
            lses = np.stack([split_lse[p] for p in parts])  # [n, 128]
            outs = np.stack([split_out[p] for p in parts])  # [n, 128, 512]
            m = lses.max(0)
            w = np.exp(lses - m)
            s = w.sum(0)
            res[row] = ((w[..., None] * outs).sum(0) / s[:, None], m + np.log(s))
    return res
