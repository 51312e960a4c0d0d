"""Indexing of the work-list decode's bins, modelled on the CPU.

pa_fp8_bin_kernel (flydsl_amd/csrc/pa_fp8.hip) gives each of its G
workgroups an equal run of consecutive bins of the persistent route's work
list (G = the CU count for 8-wave workgroups, so 3 bins each at the
reference's CU * 3 bins): the run's works laid end to end form one sequence
of N 32-token chunks, wave r of W takes chunks [rN/W, (r+1)N/W), and a
work cut between waves is merged in LDS by the wave that holds its last
chunk, from the first merge slot of every later wave and the second slot
(or the first, when its run starts at the work) of the work's first wave.
This model restates the kernel's integer steps (bin runs, chunk counts, run
bounds, start search, walk, slot choice) and checks, over many plans of the
reference's scheduler at the reference's bin counts and smaller ones, that
every visible chunk of every work is read exactly once and that every
work's result is written exactly once, from exactly its own pieces.  The
GPU tests then check the numbers.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import plan, worklist

CHUNK = 32


def work_chunks(ctx, lo_all, hi_all, last_page, pb, kv0, kv1):
    a0 = max((kv0 - pb) * 256, lo_all)
    a1 = min(min((kv1 - pb) * 256, ctx), lo_all if last_page < 0 else hi_all)
    if a1 > a0:
        tb0 = a0 & ~(CHUNK - 1)
        return tb0, -(-(a1 - tb0) // CHUNK)
    return 0, 0


def group_bins(num_bins, num_cu, waves):
    """[bin0, bin1) of each workgroup (pa_fp8.hip bin_workgroups and the
    kernel's bin run)."""
    per_cu = 1 if waves >= 8 else (2 if waves >= 4 else 3)
    G = min(num_bins, num_cu * per_cu)
    return [(g * num_bins // G, (g + 1) * num_bins // G) for g in range(G)]


def bin_works(p, bins, ctx, ql, window, bs, pbase):
    """(tb0, n, wstart) of each work of the bin run [bins[0], bins[1]), as
    the kernel's pre-pass and walk compute them."""
    info = p["work_info"]
    out, pos = [], 0
    for w in range(int(p["work_indptr"][bins[0]]), int(p["work_indptr"][bins[1]])):
        b, kv0, kv1 = int(info[w, 0]), int(info[w, 4]), int(info[w, 5])
        lo_all = plan.visible_token_range(ctx[b], 0, ql, window)[0]
        hi_all = plan.visible_token_range(ctx[b], ql - 1, ql, window)[1]
        last_page = -(-ctx[b] // bs) - 1
        tb0, n = work_chunks(ctx[b], lo_all, hi_all, last_page, pbase[b], kv0, kv1)
        out.append((w, tb0, n, pos))
        pos += n
    return out, pos


def walk_wave(works, N, r, W):
    """The pieces of wave r: (work, first chunk index in the work, chunks,
    cut flags)."""
    R0, R1 = r * N // W, (r + 1) * N // W
    start = len(works)
    for i, (_, _, n, s) in enumerate(works):  # start search
        if s + n > R0 or (n == 0 and s >= R0):
            start = i
            break
    pieces = []
    for w, tb0, n, s in works[start:]:
        e = s + n
        if s > R1:
            break
        if n == 0:
            if (R0 <= s < R1) or (r == W - 1 and s == R1):
                pieces.append((w, 0, 0, 0, s))
            continue
        c0, c1 = max(s, R0), min(e, R1)
        if c1 <= c0:
            continue
        pieces.append((w, c0 - s, c1 - c0, (1 if c0 > s else 0) | (2 if c1 < e else 0), s))
    return pieces


def check_bin(works, N, W):
    read = {w: [0] * n for w, _, n, _ in works}
    written = {w: 0 for w, _, _, _ in works}
    slots = {}  # (wave, slot) -> work
    mergers = []
    for r in range(W):
        pieces = walk_wave(works, N, r, W)
        first = True
        for w, c0, n, cut, s in pieces:
            for k in range(c0, c0 + n):
                read[w][k] += 1
            if cut == 0:
                written[w] += 1
            elif first:
                slots[(r, 0)] = w
                if cut == 1:
                    mergers.append((r, w, s))
            else:
                assert cut == 2, "a cut piece after the first ends the run"
                assert pieces[-1][0] == w, "the second slot is the wave's last piece"
                slots[(r, 1)] = w
            if n > 0:
                first = False  # an empty work does not count as the first piece
    for r, w, s in mergers:  # the merger's contributors
        got = []
        for q in range(r + 1):
            Rq, Rn = q * N // W, (q + 1) * N // W
            if Rn <= s or Rn <= Rq:
                continue
            got.append(slots.get((q, 0 if Rq >= s else 1)))
        assert got and all(g == w for g in got), (r, w, got)
        # exactly the waves holding pieces of w
        holders = {q for q in range(W) for (ww, _, nn, _, _) in walk_wave(works, N, q, W) if ww == w and nn > 0}
        assert len(got) == len(holders)
        written[w] += 1
    for w, cnt in read.items():
        assert all(x == 1 for x in cnt), (w, cnt)
    for w, cnt in written.items():
        assert cnt == 1, (w, cnt)


def _ctx(rng, B, kind, ql):
    if kind == "ragged":
        c = np.clip(np.round(np.exp(rng.normal(np.log(2048), 1.0, size=B))), 16, 32768).astype(int)
    elif kind == "short":
        c = rng.integers(1, 400, size=B)
    elif kind == "zeros":
        c = rng.integers(0, 3000, size=B)
        c[rng.random(B) < 0.3] = 0
    else:
        c = rng.integers(1, 9000, size=B)
    return [int(max(x, ql)) if kind != "zeros" else int(x) for x in c]


@pytest.mark.parametrize("kind", ["ragged", "short", "zeros", "uniform"])
@pytest.mark.parametrize("ql,window", [(1, 0), (4, 0), (1, 700), (2, 3000)])
def test_bin_walk_reads_every_chunk_once_and_writes_every_work_once(kind, ql, window):
    rng = np.random.default_rng(hash((kind, ql, window)) % 2**32)
    for trial in range(12):
        B = int(rng.integers(1, 300))
        H = int(rng.choice([1, 2, 4, 8]))
        ctx = _ctx(rng, B, kind, ql)
        pbase = np.concatenate([[0], np.cumsum([-(-c // 256) for c in ctx])]).astype(int)
        for bins, cus in ((768, 256), (H * int(rng.integers(1, 12)), int(rng.integers(1, 9)))):
            bins = (bins // H) * H or H
            p = worklist.pa_metadata_v1(ctx, H, 4, ql, bins, 256)
            for W in (8, 3):
                for run in group_bins(bins, cus, W):
                    works, N = bin_works(p, run, ctx, ql, window, 1024, pbase)
                    check_bin(works, N, W)


def test_more_than_64_works_in_a_bin():
    """The pre-pass handles 64 works per pass; a bin of many short sequences
    needs several."""
    ctx = [40 + (i * 37) % 500 for i in range(700)]
    pbase = np.concatenate([[0], np.cumsum([-(-c // 256) for c in ctx])]).astype(int)
    p = worklist.pa_metadata_v1(ctx, 1, 4, 1, 3, 256)
    counts = np.diff(p["work_indptr"])
    assert counts.max() > 128
    for run in group_bins(3, 1, 8):
        works, N = bin_works(p, run, ctx, 1, 0, 1024, pbase)
        assert len(works) > 640
        check_bin(works, N, 8)
