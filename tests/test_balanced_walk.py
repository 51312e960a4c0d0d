"""CPU model of the balanced split's indexing (the walk of
pa_fp8_stream_kernel / pa_fp8_coop_kernel and the partial ids that
pa_fp8_segment_merge_kernel reads), with head groups.

The split lays the chunks of every (sequence, head group of G adjacent kv
heads) end to end, each group preceded by A units of start cost (1 for the
per-wave kernel, 4 for the cooperative one), and cuts them into equal runs;
the G waves of a run walk head i of each group in step.  The model restates the kernel's start
search, walk and merge addressing on random batches and checks what the
GPU results depend on: every chunk of every (sequence, kv head) pair is
computed exactly once, a pair held whole writes its output row, and for a
cut pair the partial ids the merge reads (the first piece's id, then 2w for
the pair's wave w in each later run, G wave ids apart) are exactly the ids
its pieces were written to, in chunk order.  The GPU tests check the
numbers.
"""

from __future__ import annotations

import random

import pytest

from oracle import plan

CHUNK = 32
MIN_CHUNKS_PER_WAVE = 8


def seq_chunks(ctx, ql, window):
    lo, _ = plan.visible_token_range(ctx, 0, ql, window)
    _, hi = plan.visible_token_range(ctx, ql - 1, ql, window)
    if hi <= lo:
        return 0
    return -(-(hi - (lo & ~(CHUNK - 1))) // CHUNK)


def run_of_chunk(g, T, nw):
    return ((g + 1) * nw + T - 1) // T - 1


def run_begin(w, T, nw):
    return w * T // nw


def stream_waves(nq, waves=4):
    return waves if nq == 1 else 4


def stream_nq(eq):
    return 1 if eq <= 4 else (2 if eq <= 8 else 4)


def balanced_group(H, workers, eq):
    if eq > 16:  # cooperative workgroup runs: no head groups
        return 1
    g = stream_waves(stream_nq(eq))
    while g > 1 and (H % g or workers % g):
        g //= 2
    return g


def walk(nbs, H, workers, G, wid, A=0):
    """Pieces (b, h, c, n, target, desc_cnt) of worker wid; each (sequence,
    head group) costs A before its chunks in the split's order."""
    Hg = H // G
    T = sum(n + A for n in nbs if n) * Hg
    nw = min(max(1, T // MIN_CHUNKS_PER_WAVE), workers // G)
    run = wid // G
    if run >= nw:
        return []
    g0, g1 = run_begin(run, T, nw), run_begin(run + 1, T, nw)
    if g1 <= g0:
        return []
    S = 0
    for b0, n0 in enumerate(nbs):
        q = n0 + A if n0 else 0
        if n0 > 0 and (S + q) * Hg > g0:
            break
        S += q
    off = g0 - S * Hg
    hg, o = divmod(off, n0 + A)
    b, nb, h, c = b0, n0, hg * G + (wid - run * G), max(o - A, 0)
    P = S * Hg + hg * (n0 + A)
    pos, end, first = P + A + c, g1, True
    out = []
    while pos < end:
        n = min(nb - c, end - pos)
        whole = c == 0 and n == nb
        target = -1 if whole else 2 * wid + (0 if first else 1)
        desc = 0 if c else (1 if whole else run_of_chunk(P + A + nb - 1, T, nw) - run + 1)
        out.append((b, h, c, n, target, desc))
        first = False
        c += n
        pos += n
        if pos < end and c == nb:
            c = 0
            P += nb + A
            pos = P + A
            h += G
            if h >= H:
                h -= H
                while True:
                    if b + 1 >= len(nbs):
                        pos = end
                        break
                    b += 1
                    nb = nbs[b]
                    if nb:
                        break
    return out


def check(ctxs, H, ql, window, workers, eq, A=0):
    nbs = [seq_chunks(c, ql, window) for c in ctxs]
    G = balanced_group(H, workers, eq)
    pieces = {}
    for wid in range(workers):
        for b, h, c, n, target, desc in walk(nbs, H, workers, G, wid, A):
            pieces.setdefault((b, h), []).append((c, n, target, desc))
    for b, nb in enumerate(nbs):
        for h in range(H):
            got = sorted(pieces.get((b, h), []))
            covered = [c for c0, n, _, _ in got for c in range(c0, c0 + n)]
            assert covered == list(range(nb)), (b, h, got)
            if nb == 0:
                continue
            if len(got) == 1:
                assert got[0][2] == -1 and got[0][3] == 1  # whole: straight to the output
                continue
            pid0, cnt = got[0][2], got[0][3]
            assert cnt == len(got) and pid0 >= 0
            merge_reads = [pid0] + [2 * ((pid0 >> 1) + i * G) for i in range(1, cnt)]
            assert merge_reads == [t for _, _, t, _ in got], (b, h, got)
            assert all(t < 2 * workers for t in merge_reads)
    return G


@pytest.mark.parametrize("seed", range(40))
def test_every_chunk_once_and_merge_reads_the_written_pieces(seed):
    rng = random.Random(seed)
    B = rng.randint(1, 40)
    ctxs = [rng.choice([0, 1, 2, 17, 31, 32, 33]) if rng.random() < 0.2 else rng.randint(1, 6000) for _ in range(B)]
    H = rng.choice([1, 2, 3, 4, 6, 8, 12, 16])
    ql = rng.choice([1, 1, 2, 4])
    window = rng.choice([0, 0, 100, 1000])
    eq = ql * rng.choice([1, 2, 4, 8, 16])
    workers = rng.choice([4, 6, 8, 12, 16, 64, 2048])
    check(ctxs, H, ql, window, workers, eq, A=rng.choice([0, 1, 2, 4, 5]))


def test_head_groups_of_the_benchmark_shapes():
    # C3: 8 kv heads, 4 query columns, 2048 waves: groups of 4 adjacent heads
    assert check([2048, 17, 32768, 1, 700] * 8, 8, 1, 0, 2048, 4) == 4
    # 2 kv heads: groups of 2; 3 kv heads or odd worker counts: no groups
    assert check([900, 3000, 5], 2, 1, 0, 64, 4) == 2
    assert check([900, 3000, 5], 3, 1, 0, 64, 4) == 1
    assert check([900, 3000, 5], 4, 1, 0, 6, 4) == 2
    assert check([900, 3000, 5], 4, 1, 0, 7, 4) == 1
    # more than 4 columns (two query images per wave) keep 4-wave groups
    assert check([900, 3000, 5], 8, 2, 0, 64, 8) == 4
    # the shipped start costs: per-wave runs (A = 1), cooperative workgroup runs (A = 4, no groups)
    assert check([2048, 17, 32768, 1, 700] * 8, 8, 1, 0, 2048, 4, A=1) == 4
    assert check([4096, 8000, 5000, 6144] * 16, 4, 4, 0, 512, 64, A=4) == 1
