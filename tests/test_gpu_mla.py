"""MLA fp8 decode on the GPU against the oracle (oracle/mla.py).

Mirrors tests/kernels/test_mla_decode.py: fp8 query [rows, 128, 576] and
fp8 KV buffer [pages, 1, 1, 576] from standard normals, pages in random
order, softmax scale 1/sqrt(576); work list from get_mla_metadata_v1, the
decode, then mla_reduce_v1.  Each case checks
  * every work's split output and lse (or, for uncut rows, the final
    output) against the oracle's per-work attention, and
  * the final bf16 output and the reduced lse against the oracle's
    unsplit attention.
Bar (floating point): the logits are exact (fp8 x fp8 products summed in
float32), so the error comes from the probabilities carried in fp8 for the
value product.  With one fp8 term per probability (the reference's
arithmetic) each p has relative error <= 2^-4, so
    |out - ref| <= 2^-4 * wabs + 2^-8 * |ref| + 1e-5
per element, wabs = the softmax-weighted mean of |v| (2^-8 |ref| covers the
bf16 output); with precise_p (two fp8 terms) 2^-7 * wabs instead of
2^-4 * wabs (the low term's own rounding is 2^-8 relative, plus the flush of
low terms below the e4m3fn subnormal range, 2^-9 of the block maximum).  lse within 2e-5 + 1e-5 |lse|.  The reference test's own bar is
a cosine difference < 3e-2; the tests also assert that, and a much tighter
cosine difference.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from flydsl_amd.mla_decode import (
    QK_HEAD_DIM,
    V_HEAD_DIM,
    flydsl_mla_fwd_decode,
    get_mla_metadata_info_v1,
    get_mla_metadata_v1,
    mla_reduce_v1,
)
from oracle import mla as om

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
FP8 = torch.float8_e4m3fn


def make_case(lens, seed, extra_pages=7, wide=None, nan_page0=False):
    """wide = (boost, fractions): rows at those fractions of each sequence get
    keys aligned with the (head-shared) query direction, scaled so their
    logits reach about `boost` nats.  nan_page0: no sequence uses page 0,
    whose bytes are all 0x7f (e4m3fn NaN)."""
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    kv_indptr = torch.zeros(B + 1, dtype=torch.int32)
    kv_indptr[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    total = int(kv_indptr[-1])
    num_pages = total + extra_pages
    first = 1 if nan_page0 else 0
    kv_indices = (torch.randperm(num_pages - first, generator=g)[:total] + first).to(torch.int32)
    kv = torch.randn(num_pages, 1, 1, QK_HEAD_DIM, generator=g)
    q = torch.randn(B, 128, QK_HEAD_DIM, generator=g)
    if wide is not None:
        boost, fracs = wide
        # one query direction for every head (plus a little noise), and keys
        # along its sign pattern: logit ~ a * sum |q| / 24
        base = torch.randn(QK_HEAD_DIM, generator=g)
        q = base + 0.05 * torch.randn(B, 128, QK_HEAD_DIM, generator=g)
        a = boost * 24.0 / float(base.abs().sum())
        a = float(torch.tensor(a).to(torch.bfloat16).to(FP8).float())
        for b in range(B):
            n = lens[b]
            for f0, f1 in fracs:
                for t in range(int(f0 * n), max(int(f1 * n), int(f0 * n) + 1)):
                    kv[int(kv_indices[int(kv_indptr[b]) + t]), 0, 0] = a * torch.sign(base)
    kv = kv.to(torch.bfloat16).to(FP8)
    q = q.to(torch.bfloat16).to(FP8)
    if nan_page0:
        kv.view(torch.uint8)[0].fill_(0x7F)
    qo_indptr = torch.arange(B + 1, dtype=torch.int32)
    last = torch.ones(B, dtype=torch.int32)
    return q, kv, qo_indptr, kv_indptr, kv_indices, last


def run(lens, seed=0, num_cu=None, precise=False, fnuz=False, sm=None, **case_kw):
    q, kv, qo_indptr, kv_indptr, kv_indices, last = make_case(lens, seed, **case_kw)
    q_val, kv_val = om.fp8_to_f64(q), om.fp8_to_f64(kv.view(-1, QK_HEAD_DIM))
    if fnuz:  # the same values as float8_e4m3fnuz tensors (every e4m3fn value below 240 is one)
        q = q.float().to(torch.float8_e4m3fnuz)
        kv = kv.float().to(torch.float8_e4m3fnuz)
        assert np.array_equal(q.to(torch.float64).numpy(), q_val)
    B = len(lens)
    sizes = get_mla_metadata_info_v1(B, 1, 128, FP8, FP8, num_cu=num_cu)
    bufs = [torch.empty(s, dtype=t, device=DEV) for s, t in sizes]
    meta, work_indptr, work_info, reduce_indptr, reduce_final_map, reduce_partial_map = bufs
    get_mla_metadata_v1(qo_indptr.to(DEV), kv_indptr.to(DEV), last.to(DEV), 128, 1, False, meta, work_info,
                        work_indptr, reduce_indptr, reduce_final_map, reduce_partial_map, kv_granularity=16,
                        max_seqlen_qo=1, uni_seqlen_qo=1)
    npart = reduce_partial_map.size(0)
    out = torch.full((B, 128, V_HEAD_DIM), -1.0, dtype=torch.bfloat16, device=DEV)
    split_o = torch.full((npart, 1, 128, V_HEAD_DIM), float("nan"), dtype=torch.float32, device=DEV)
    split_l = torch.full((npart, 1, 128, 1), float("nan"), dtype=torch.float32, device=DEV)
    final_lse = torch.full((B, 128), float("nan"), dtype=torch.float32, device=DEV)
    sm = 1.0 / QK_HEAD_DIM ** 0.5 if sm is None else float(sm)
    qd, kvd, kid = q.to(DEV), kv.to(DEV), kv_indices.to(DEV)
    print(f"mla case lens={lens[:4]}{'...' if len(lens) > 4 else ''} B={B} seed={seed} num_cu={num_cu} "
          f"precise={precise}", flush=True)
    flydsl_mla_fwd_decode(qd, kvd, kid, work_indptr, work_info, out, split_o, split_l, sm, precise_p=precise)
    torch.cuda.synchronize()
    split_snapshot = (split_o.clone(), split_l.clone(), out.clone())
    mla_reduce_v1(split_o, split_l, reduce_indptr, reduce_final_map, reduce_partial_map, 1, out, final_lse)
    torch.cuda.synchronize()
    meta_h = meta.cpu().numpy()
    return dict(q=q_val, kv=kv_val, qo=qo_indptr.numpy(),
                kvp=kv_indptr.numpy(), kvi=kv_indices.numpy(), sm=sm, out=out.float().cpu().numpy(),
                lse=final_lse.cpu().numpy(), split=[t.cpu() for t in split_snapshot],
                work_info=work_info.cpu().numpy(), n=int(meta_h[0]), ng=int(meta_h[1]), npart=int(meta_h[2]))


def tolerance(wabs, ref, precise):
    return (2.0 ** -7 if precise else 2.0 ** -4) * wabs + 2.0 ** -8 * np.abs(ref) + 1e-5


def check(r, precise=False):
    want, want_lse, wabs = om.mla_decode_ref(r["q"], r["kv"], r["qo"], r["kvp"], r["kvi"], r["sm"])
    tol = tolerance(wabs, want, precise)
    err = np.abs(r["out"] - want)
    assert np.all(err <= tol), f"final output: worst excess {np.max(err - tol):.3g} at {np.unravel_index(np.argmax(err - tol), err.shape)}"
    cos = 1 - 2 * float((r["out"] * want).sum()) / max(float((r["out"] ** 2 + want ** 2).sum()), 1e-12)
    assert cos < 3e-2  # the reference test's bar
    assert cos < (1e-5 if precise else 2e-3)
    # per work: split rows (float32, normalised) or direct rows
    so, sl, direct_out = r["split"]
    so = so.numpy()[:, 0]
    sl = sl.numpy()[:, 0, :, 0]
    for row, pql, o, l, wa in om.mla_split_ref(r["q"], r["kv"], r["kvi"], r["work_info"], r["n"], r["sm"]):
        if pql < 0:
            got = direct_out[row].float().numpy()
            assert np.all(np.abs(got - o) <= tolerance(wa, o, precise)), f"direct row {row}"
        else:
            e = np.abs(so[pql] - o) - tolerance(wa, o, precise)
            assert np.all(e <= 0), f"split row {pql}: worst excess {e.max():.3g}"
            fin = np.isfinite(l)
            assert np.array_equal(fin, np.isfinite(sl[pql]))
            assert np.all(np.abs(sl[pql][fin] - l[fin]) <= 2e-5 + 1e-5 * np.abs(l[fin])), f"split lse {pql}"
    # reduced lse for the cut rows
    cut = sorted({int(w[2]) for w in r["work_info"][: r["n"]] if w[1] >= 0})
    for row in cut:
        assert np.all(np.abs(r["lse"][row] - want_lse[row]) <= 2e-5 + 1e-5 * np.abs(want_lse[row])), f"lse row {row}"


# the reference test's configurations (tests/kernels/test_mla_decode.py:60-68)
@pytest.mark.parametrize("batch,ctx", [(1, 63), (1, 64), (1, 128), (4, 2048), (33, 2333), (32, 8192)])
def test_reference_configs(batch, ctx):
    check(run([ctx] * batch, seed=batch * 1000003 + ctx))


@pytest.mark.parametrize("batch,ctx", [(1, 128), (4, 2048), (33, 2333)])
def test_precise_probabilities(batch, ctx):
    check(run([ctx] * batch, seed=7 + ctx, precise=True), precise=True)


def test_ragged_with_few_workers():
    # several works per worker (cross-work prefetch), cut and uncut rows,
    # partial last blocks of every length class
    check(run([1, 127, 128, 129, 255, 5000, 77, 640, 2], seed=11, num_cu=3))


def test_one_worker_no_splits():
    check(run([300, 10, 4096, 1], seed=12, num_cu=1))


def test_many_small_pieces():
    # more workers than blocks: every block its own piece, long merges
    check(run([1100, 40], seed=13, num_cu=64))


def test_fnuz_inputs():
    """float8_e4m3fnuz query and kv tensors (accepted, as the reference's
    launcher accepts them) decode to the oracle's result on their values."""
    check(run([700, 33, 2000], seed=17, fnuz=True))


def test_empty_sequence_writes_zeros():
    """Empty ranges write zeros even when the page their DMA touches (page 0)
    holds NaN bytes."""
    r = run([0, 200, 0], seed=14, num_cu=2, nan_page0=True)
    assert np.all(r["out"][0] == 0) and np.all(r["out"][2] == 0)
    want, _, wabs = om.mla_decode_ref(r["q"], r["kv"], r["qo"], r["kvp"], r["kvi"], r["sm"])
    assert np.all(np.abs(r["out"][1] - want[1]) <= tolerance(wabs[1], want[1], False))


def test_rerun_is_deterministic():
    a = run([3000, 900], seed=15, num_cu=16)
    b = run([3000, 900], seed=15, num_cu=16)
    assert np.array_equal(a["out"], b["out"])


@pytest.mark.parametrize("precise", [False, True])
def test_wide_logits_with_late_maxima(precise):
    """Logits spanning ~150 nats whose maxima sit late in a work (the last
    tenth of every sequence, and a run in the middle that ends pieces when
    the rows are cut): the reference exponent set on a work's first block
    has to move (the softmax's rare rescale), and nothing overflows."""
    lens = [5000, 3000, 777, 9000]
    r = run(lens, seed=21, num_cu=5, precise=precise, wide=(150.0, [(0.9, 1.0), (0.45, 0.5)]))
    assert np.all(np.isfinite(r["out"]))
    want, want_lse, _ = om.mla_decode_ref(r["q"], r["kv"], r["qo"], r["kvp"], r["kvi"], r["sm"])
    assert float(np.min(want_lse)) > 120.0  # the boosted rows dominate every head
    check(r, precise=precise)


@pytest.mark.parametrize("sm", [-1.0 / QK_HEAD_DIM ** 0.5, 0.0])
def test_softmax_scales(sm):
    """Negative (carried by the query signs) and zero (a uniform softmax)
    scales: the kernel takes its maxima on the raw logits and folds the
    scale into the exponent."""
    check(run([1500, 64, 3000], seed=23, num_cu=4, sm=sm))


def _quantized_softmax_out(q, kv, kvp, kvi, sm, b):
    """float64 model of the kernel's fp8 probabilities for row b: one block
    exponent e = ceil(max) per 32-token group (tokens 16t + 0..7 or
    16t + 8..15 of the four 16-token tiles of a 64-token half block),
    p = 2^(x - e) rounded to e4m3fn in the numerator, exact p in the
    denominator."""
    idx = kvi[kvp[b]:kvp[b + 1]]
    K = kv[idx]
    V = K[:, :V_HEAD_DIM]
    x = (K @ q[b].T) * sm * np.log2(np.e)  # [tokens, heads]
    pos = np.arange(len(idx))
    grp = (pos // 64) * 2 + (pos % 16) // 8
    num = np.zeros((q.shape[1], V_HEAD_DIM))
    den = np.zeros(q.shape[1])
    for G in np.unique(grp):
        m = grp == G
        e = np.ceil(x[m].max(axis=0))
        p = 2.0 ** (x[m] - e)
        pq = torch.from_numpy(p.astype(np.float32)).to(FP8).to(torch.float64).numpy()
        num += (pq * 2.0 ** e).T @ V[m]
        den += (p * 2.0 ** e).sum(axis=0)
    return num / den[:, None]


def test_large_softmax_scale():
    """Scale 0.5 (12x the usual): a very peaked softmax.  Probabilities more
    than 2^6 below their 32-token group's maximum fall in the fp8 subnormal
    range, where rounding is absolute (2^-10 of the group's block exponent),
    so an element whose |v|-weight sits on such tokens can be far off in
    relative terms -- the arithmetic of one fp8 term per probability (the
    reference's), not a fault.  The bound: the distance of a float64 model
    of that quantization from the exact result, plus the usual bound."""
    r = run([1500, 64, 3000], seed=23, num_cu=4, sm=0.5)
    want, _, wabs = om.mla_decode_ref(r["q"], r["kv"], r["qo"], r["kvp"], r["kvi"], r["sm"])
    for b in range(3):
        model = _quantized_softmax_out(r["q"], r["kv"], r["kvp"], r["kvi"], r["sm"], b)
        tol = np.abs(model - want[b]) + tolerance(wabs[b], want[b], False)
        assert np.all(np.abs(r["out"][b] - want[b]) <= tol), f"row {b}"


def test_fnuz_conversion_every_code():
    """The library's byte-wise e4m3fnuz -> e4m3fn pass equals torch's
    conversion through float32 for all 256 codes (NaN to NaN), gathering
    rows by index with out-of-range indices clamped."""
    from flydsl_amd import mla_decode as md

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    src = codes.repeat(9).view(4, 576)  # four rows, every code 2.25 times per row
    src[1] = src[1].roll(37)
    src[2] = src[2].flip(0)
    src = src.view(torch.float8_e4m3fnuz)
    rows = torch.tensor([3, 0, -5, 2, 99, 1], dtype=torch.int32)
    got = md._fnuz_rows_to_fn(src.to(DEV), rows.to(DEV), (6, 576)).cpu()
    want = src.float()[rows.clamp(0, 3).long()].to(torch.float8_e4m3fn)
    g, w = got.view(torch.uint8), want.view(torch.uint8)
    nan = torch.isnan(want.float())
    assert torch.equal(torch.isnan(got.float()), nan)
    assert torch.equal(g[~nan], w[~nan])


def test_fnuz_large_pool_converts_only_used_pages():
    """A pool far larger than the pages the call uses: the fnuz path converts
    only the listed rows (memory bounded by them, not by the pool) and
    decodes as the e4m3fn tensors of the same values do."""
    lens = [300, 5, 1200]
    q, kv, qo_indptr, kv_indptr, kv_indices, last = make_case(lens, 31)
    n_used = kv.size(0)
    pool_pages = 400_000  # 230 MB of fp8 rows
    big = torch.zeros(pool_pages, 1, 1, QK_HEAD_DIM, dtype=torch.float8_e4m3fnuz, device=DEV)
    where = torch.randperm(pool_pages, generator=torch.Generator().manual_seed(5))[:n_used].to(torch.int32)
    big[where.long().to(DEV)] = kv.float().to(torch.float8_e4m3fnuz).to(DEV)
    idx_big = where[kv_indices.long()].to(DEV)
    B = len(lens)

    def decode(qd, kvd, kid):
        sizes = get_mla_metadata_info_v1(B, 1, 128, FP8, FP8)
        bufs = [torch.empty(s, dtype=t, device=DEV) for s, t in sizes]
        meta, work_indptr, work_info, reduce_indptr, reduce_final_map, reduce_partial_map = bufs
        get_mla_metadata_v1(qo_indptr.to(DEV), kv_indptr.to(DEV), last.to(DEV), 128, 1, False, meta, work_info,
                            work_indptr, reduce_indptr, reduce_final_map, reduce_partial_map)
        out = torch.empty(B, 128, V_HEAD_DIM, dtype=torch.bfloat16, device=DEV)
        npart = reduce_partial_map.size(0)
        so = torch.empty(npart, 1, 128, V_HEAD_DIM, device=DEV)
        sl = torch.empty(npart, 1, 128, 1, device=DEV)
        flydsl_mla_fwd_decode(qd, kvd, kid, work_indptr, work_info, out, so, sl, 1.0 / QK_HEAD_DIM ** 0.5)
        mla_reduce_v1(so, sl, reduce_indptr, reduce_final_map, reduce_partial_map, 1, out)
        torch.cuda.synchronize()
        return out.cpu()

    def peak_extra(fn, *args):
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        r = fn(*args)
        return r, torch.cuda.max_memory_allocated() - base

    qd, kvd, kid = q.to(DEV), kv.to(DEV), kv_indices.to(DEV)
    want, fn_extra = peak_extra(decode, qd, kvd, kid)
    qz = q.float().to(torch.float8_e4m3fnuz).to(DEV)
    got, fnuz_extra = peak_extra(decode, qz, big, idx_big)
    assert torch.equal(got, want)
    # the work list and split rows are the same for both; the conversion adds
    # the query and the listed rows (about 1 MB here), not the 230 MB pool
    assert fnuz_extra - fn_extra < 8 << 20, (fnuz_extra, fn_extra)
