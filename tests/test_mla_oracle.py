"""The MLA oracle (oracle/mla.py) and the host work-list planner, on the CPU.

The reference's MLA test holds no fixed vectors (it draws random inputs on
the GPU and compares with its torch oracle), so the oracle is pinned here by
what the mathematics fixes: one token returns its value row and its logit as
lse; identical keys give the mean of the values and lse = s + ln N; two
tokens give the closed-form two-way softmax; a brute-force scalar loop
agrees on a small case; and a split into pieces merged by the log-sum-exp
reduce equals the unsplit result.  The planner is checked by its
invariants: every query row's page range covered once, in order, by works
of balanced workers, with partial rows and reduce groups exactly for the
rows that were cut.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from flydsl_amd import _lib
from oracle import mla as om


def rand(shape, rng):
    return rng.standard_normal(shape)


def test_single_token_returns_its_value_row():
    rng = np.random.default_rng(1)
    q = rand((2, 128, 576), rng)
    k = rand((1, 576), rng)
    out, lse, _ = om.attend(q, k, 0.05)
    np.testing.assert_allclose(out, np.broadcast_to(k[0, :512], out.shape), rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, (q @ k[0]) * 0.05, rtol=1e-12, atol=1e-12)


def test_identical_keys_give_uniform_weights():
    rng = np.random.default_rng(2)
    q = rand((1, 128, 576), rng)
    k = np.repeat(rand((1, 576), rng), 37, axis=0)
    out, lse, _ = om.attend(q, k, 0.1)
    s = (q[0] @ k[0]) * 0.1
    np.testing.assert_allclose(lse[0], s + math.log(37), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out[0], np.broadcast_to(k[0, :512], (128, 512)), atol=1e-12)


def test_two_tokens_closed_form():
    rng = np.random.default_rng(3)
    q = rand((1, 128, 576), rng)
    k = rand((2, 576), rng)
    sc = 1.0 / math.sqrt(576)
    out, lse, wabs = om.attend(q, k, sc)
    a = (q[0] @ k[0]) * sc
    b = (q[0] @ k[1]) * sc
    wa = 1.0 / (1.0 + np.exp(b - a))
    want = wa[:, None] * k[0, :512] + (1 - wa)[:, None] * k[1, :512]
    np.testing.assert_allclose(out[0], want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse[0], np.logaddexp(a, b), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(wabs[0], wa[:, None] * np.abs(k[0, :512]) + (1 - wa)[:, None] * np.abs(k[1, :512]),
                               atol=1e-12)


def test_brute_force_scalar_loop():
    rng = np.random.default_rng(4)
    n = 5
    q = rand((1, 128, 576), rng)
    k = rand((n, 576), rng)
    out, lse, _ = om.attend(q, k, 0.07)
    for h in (0, 77, 127):
        logits = [0.07 * sum(float(q[0, h, d]) * float(k[t, d]) for d in range(576)) for t in range(n)]
        m = max(logits)
        ws = [math.exp(x - m) for x in logits]
        tot = sum(ws)
        assert abs(lse[0, h] - (m + math.log(tot))) < 1e-10
        for d in (0, 255, 511):
            ref = sum(ws[t] * float(k[t, d]) for t in range(n)) / tot
            assert abs(out[0, h, d] - ref) < 1e-10


def plan_case(lens, rows_per_seq, workers):
    qo = np.concatenate([[0], np.cumsum(rows_per_seq)]).astype(np.int32)
    kv = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n, ng, npart, out = _lib.mla_plan(qo, kv, workers)
    return qo, kv, n, ng, npart, out


@pytest.mark.parametrize("lens,workers", [
    ([63], 256), ([64], 256), ([128], 256), ([2048] * 4, 256), ([2333] * 33, 256), ([8192] * 32, 256),
    ([1, 127, 128, 129, 0, 5000, 77], 3), ([300, 10, 4096], 1), ([0, 0, 0], 4), ([129] * 50, 7),
])
def test_planner_invariants(lens, workers):
    qo, kv, n, ng, npart, out = plan_case(lens, [1] * len(lens), workers)
    wp, wi = out["work_indptr"], out["work_info"][:n]
    assert wp[0] == 0 and wp[-1] == n and np.all(np.diff(wp) >= 0)
    # coverage: per row, the pieces tile [kv[b], kv[b+1]) in order
    per_row = {}
    for w in wi:
        b, pql, r0, r1, k0, k1 = (int(x) for x in w[:6])
        assert r1 == r0 + 1 and qo[b] <= r0 < qo[b + 1]
        assert w[7] == (128 << 16)
        per_row.setdefault(r0, []).append((k0, k1, pql))
    assert sorted(per_row) == list(range(int(qo[-1])))
    blocks = []
    for b in range(len(lens)):
        pieces = per_row[b]
        assert pieces[0][0] == kv[b] and pieces[-1][1] == kv[b + 1]
        for (a0, a1, _), (b0, _, _) in zip(pieces, pieces[1:]):
            assert a1 == b0 and a1 > a0
        if len(pieces) == 1:
            assert pieces[0][2] == -1
        else:
            assert all(p[2] >= 0 for p in pieces)
        blocks.append(sum(max(1, -(-(k1 - k0) // 128)) for k0, k1, _ in pieces))
    # partial rows unique, groups = cut rows
    pq = [p for ps in per_row.values() for _, _, p in ps if p >= 0]
    assert sorted(pq) == list(range(npart))
    assert ng == sum(1 for ps in per_row.values() if len(ps) > 1)
    ri, fm, pm = out["reduce_indptr"], out["reduce_final_map"], out["reduce_partial_map"]
    assert ri[0] == 0 and ri[ng] == npart and np.all(ri[ng:] == npart)
    for g in range(ng):
        row = int(fm[g][0])
        assert fm[g][1] == row + 1
        assert [int(pm[i]) for i in range(ri[g], ri[g + 1])] == [p for _, _, p in per_row[row]]
    # balance: every worker but the last takes at most ceil(total / workers)
    # blocks (a piece never exceeds its worker's quota)
    total = sum(max(1, -(-l // 128)) for l in lens)
    quota = -(-total // workers)
    for c in range(workers - 1):
        load = sum(max(1, -(-(int(w[5]) - int(w[4])) // 128)) for w in wi[wp[c]:wp[c + 1]])
        assert load <= quota


def test_split_and_reduce_equal_unsplit():
    rng = np.random.default_rng(5)
    lens = [700, 1, 300]
    qo, kv, n, ng, npart, out = plan_case(lens, [1] * 3, 5)
    pages = int(kv[-1]) + 9
    kvbuf = rand((pages, 576), rng)
    kv_indices = rng.permutation(pages)[: int(kv[-1])]
    q = rand((3, 128, 576), rng)
    want, want_lse, _ = om.mla_decode_ref(q, kvbuf, qo, kv, kv_indices, 0.04)
    pieces = om.mla_split_ref(q, kvbuf, kv_indices, out["work_info"], n, 0.04)
    split_out = np.zeros((max(npart, 1), 128, 512))
    split_lse = np.zeros((max(npart, 1), 128))
    direct = {}
    for row, pql, o, l, _ in pieces:
        if pql < 0:
            direct[row] = (o, l)
        else:
            split_out[pql], split_lse[pql] = o, l
    merged = om.mla_reduce_ref(split_out, split_lse, out["reduce_indptr"], out["reduce_final_map"],
                               out["reduce_partial_map"], ng)
    assert ng >= 1 and set(merged) | set(direct) == {0, 1, 2}
    for row, (o, l) in {**direct, **merged}.items():
        np.testing.assert_allclose(o, want[row], rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(l, want_lse[row], rtol=1e-12, atol=1e-12)
