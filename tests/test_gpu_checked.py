"""The checked build (libpa_fp8_checked.so: the library's sources compiled
with -DPA_FP8_CHECKED) on the GPU.

Every kernel clamps the indices it reads from caller data -- block-table and
page-list entries, MLA work records, rope positions, cache slots -- into
range before it forms an address, in both builds.  The checked build also
records each value it had to clamp (pa_fp8_debug_violations).  Here clean
calls record nothing and match the CPU oracle at the usual tolerances;
calls with entries outside their range run on the clamped values (the
oracle's result for the clamped inputs) and leave the matching bit.  The
out-of-range values are ones the kernels' own bounds checks clamp, so these
calls read and write only inside their buffers.
"""

from __future__ import annotations

import pytest
import torch

from flydsl_amd import (
    _lib,
    build_fused_rope_cache_module,
    flydsl_mla_fwd_decode,
    flydsl_qk_norm_rope_quant,
    get_mla_metadata_info_v1,
    get_mla_metadata_v1,
    mla_reduce_v1,
)
from oracle import rope_cache as rc
from tests._cases import make_case, torch_oracle
from tests.test_gpu_parity import assert_parity, launch
from tests.test_gpu_stream import balanced, run, to_dev

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture
def checked(monkeypatch):
    """The checked library in place of the release one for the test."""
    lib = _lib.load(_lib.CHECKED_LIB_PATH)
    assert lib.pa_fp8_checked_build() == 1
    monkeypatch.setattr(_lib, "_LIB", lib)
    _lib.debug_violations(lib)  # start clean
    return lib


def paged_routes(d):
    """(label, output) of the partition schedules and the balanced split."""
    for sched in ("auto", "owner", "slot"):
        out, route, _ = launch(d, sched=sched)
        yield f"{sched} {route}", out
    for num_cu in (None, 2):
        with balanced(num_cu):
            out, route = run(d)
        yield f"balanced cu={num_cu} {route}", out


PAGED_CASES = {
    "gqa4_pt": dict(batch=5, per_token=True, ctx=[1, 300, 2000, 17, 5000]),
    "coop_ql4_gqa16_pt": dict(batch=4, query_length=4, num_query_heads=64, num_kv_heads=4, per_token=True,
                              ctx=[4, 700, 2100, 3000]),
}


@pytest.mark.parametrize("name", sorted(PAGED_CASES))
def test_paged_decode_clean_and_out_of_range_pages(checked, name):
    case = make_case(seed=301, **PAGED_CASES[name])
    d = to_dev(case)
    ref = torch_oracle(case, float_out=False)
    for label, out in paged_routes(d):
        assert_parity(out, ref, f"checked {name} {label}")
        assert _lib.debug_violations(checked) == 0, label
    # entries inside the sequences' visible pages, below 0 and past the pool
    bt = case["block_tables"].clone()
    nb = case["key_cache"].shape[0]
    bs = case["key_cache"].shape[-2]
    ctx = case["context_lengths"].tolist()
    long1, long2 = sorted(range(len(ctx)), key=lambda b: -ctx[b])[:2]
    bt[long1, (ctx[long1] - 1) // bs // 2] = -7
    bt[long2, (ctx[long2] - 1) // bs] = nb + 11
    print(f"[checked] {name}: pages -7 and {nb + 11} in sequences {long1}, {long2}", flush=True)
    ref_clamped = torch_oracle(dict(case, block_tables=bt.clamp(0, nb - 1)), float_out=False)
    d_bad = dict(d, block_tables=bt.to(DEV))
    for label, out in paged_routes(d_bad):
        assert_parity(out, ref_clamped, f"checked {name} clamped pages {label}")
        assert _lib.debug_violations(checked) == _lib.VIOLATION_PAGE, label


def _mla_inputs(lens, seed):
    from tests.test_gpu_mla import make_case as mla_case

    q, kv, qo_indptr, kv_indptr, kv_indices, last = mla_case(lens, seed)
    B = len(lens)
    sizes = get_mla_metadata_info_v1(B, 1, 128, q.dtype, kv.dtype)
    bufs = [torch.empty(s, dtype=t, device=DEV) for s, t in sizes]
    meta, work_indptr, work_info, reduce_indptr, reduce_final_map, reduce_partial_map = bufs
    get_mla_metadata_v1(qo_indptr.to(DEV), kv_indptr.to(DEV), last.to(DEV), 128, 1, False, meta, work_info,
                        work_indptr, reduce_indptr, reduce_final_map, reduce_partial_map)
    return dict(q=q.to(DEV), kv=kv.to(DEV), kv_indices=kv_indices.to(DEV), work_indptr=work_indptr,
                work_info=work_info, reduce=(reduce_indptr, reduce_final_map, reduce_partial_map), B=B)


def _mla_decode(m, kv_indices=None, work_info=None):
    B = m["B"]
    npart = m["reduce"][2].size(0)
    out = torch.full((B, 128, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    so = torch.empty(npart, 1, 128, 512, device=DEV)
    sl = torch.empty(npart, 1, 128, 1, device=DEV)
    flydsl_mla_fwd_decode(m["q"], m["kv"], m["kv_indices"] if kv_indices is None else kv_indices, m["work_indptr"],
                          m["work_info"] if work_info is None else work_info, out, so, sl, 576 ** -0.5)
    mla_reduce_v1(so, sl, *m["reduce"], 1, out)
    torch.cuda.synchronize()
    return out.cpu()


def test_mla_clean_and_out_of_range_entries(checked):
    m = _mla_inputs([63, 700, 1500, 300], seed=5)
    rel = _lib.load(_lib.LIB_PATH)
    want = _mla_decode(m)
    assert _lib.debug_violations(checked) == 0
    nan = torch.isnan(want.float())
    print(f"[checked] mla clean: NaN at (row, head) {nan.any(-1).nonzero()[:8].tolist()} of {int(nan.sum())}", flush=True)
    assert not nan.any()
    num_pages = m["kv"].shape[0]
    idx = m["kv_indices"].clone()
    idx[5] = num_pages + 3
    idx[900] = -2
    got = _mla_decode(m, kv_indices=idx)
    assert _lib.debug_violations(checked) == _lib.VIOLATION_PAGE
    assert not torch.isnan(got.float()).any()
    # the same call on the page list clamped by hand: the same bits
    same = _mla_decode(m, kv_indices=idx.clamp(0, num_pages - 1))
    assert _lib.debug_violations(checked) == 0
    assert torch.equal(got, same)
    # a work whose kv range runs past the page list
    wi = m["work_info"].clone().view(-1, 8)
    wi[0, 5] = m["kv_indices"].numel() + 50
    _mla_decode(m, work_info=wi.view(m["work_info"].shape))
    assert _lib.debug_violations(checked) & _lib.VIOLATION_WORK
    assert rel.pa_fp8_checked_build() == 0


def test_rope_cache_positions_and_slots(checked):
    T, QH, KH, D, bs = 16, 8, 2, 128, 16
    nb = 4
    torch.manual_seed(7)
    q = torch.randn(T, QH, D, dtype=torch.bfloat16, device=DEV)
    k = torch.randn(T, KH, D, dtype=torch.bfloat16, device=DEV)
    v = torch.randn(T, KH, D, dtype=torch.bfloat16, device=DEV)
    max_pos = 64
    cos = torch.randn(max_pos, D // 2, dtype=torch.bfloat16, device=DEV)
    sin = torch.randn(max_pos, D // 2, dtype=torch.bfloat16, device=DEV)
    launch_rc = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs,
                                              flash_layout=True, dtype_str="bf16", apply_scale=False,
                                              reuse_freqs_front_part=True, pos_dtype="i32")

    def call(pos, slots):
        kc = torch.zeros(nb, bs, KH, D, dtype=torch.bfloat16, device=DEV)
        vc = torch.zeros_like(kc)
        qo, ko = torch.empty_like(q), torch.empty_like(k)
        ones = torch.ones(1, dtype=torch.float32, device=DEV)
        launch_rc(q, k, v, pos, cos, sin, slots, kc, vc, qo, ko, T, ones, ones)
        torch.cuda.synchronize()
        return qo, ko, kc, vc

    pos = torch.arange(T, dtype=torch.int32, device=DEV) * 3
    slots = torch.arange(T, dtype=torch.int32, device=DEV) * 2
    clean = call(pos, slots)
    assert _lib.debug_violations(checked) == 0
    rq, rk, rkc, rvc = rc.rope_cache_ref(q.cpu(), k.cpu(), v.cpu(), pos.cpu(), cos.cpu(), sin.cpu(), slots.cpu(),
                                         torch.zeros(nb, bs, KH, D, dtype=torch.bfloat16),
                                         torch.zeros(nb, bs, KH, D, dtype=torch.bfloat16), block_size=bs,
                                         layout=rc.FLASH, reuse_freqs_front_part=True)
    assert torch.equal(clean[0].cpu(), rq) and torch.equal(clean[2].cpu(), rkc)
    bad_pos = pos.clone()
    bad_pos[3] = max_pos + 9
    call(bad_pos, slots)
    assert _lib.debug_violations(checked) == _lib.VIOLATION_POSITION
    bad_slots = slots.clone()
    bad_slots[5] = nb * bs + 40  # block 6 of a 4-block cache: not written
    _, _, kc, _ = call(pos, bad_slots)
    assert _lib.debug_violations(checked) == _lib.VIOLATION_SLOT
    keep = torch.ones(T, dtype=torch.bool)
    keep[5] = False
    want_kc = rc.rope_cache_ref(q.cpu(), k.cpu(), v.cpu(), pos.cpu(), cos.cpu(), sin.cpu(),
                                torch.where(keep.to(DEV), slots, -1).cpu(),
                                torch.zeros(nb, bs, KH, D, dtype=torch.bfloat16),
                                torch.zeros(nb, bs, KH, D, dtype=torch.bfloat16), block_size=bs, layout=rc.FLASH,
                                reuse_freqs_front_part=True)[2]
    assert torch.equal(kc.cpu(), want_kc)


def test_qk_norm_rope_positions(checked):
    from tests.test_qk_norm_rope_oracle import make_inputs

    H, D, RD, T = 4, 128, 64, 6
    inp = make_inputs(T, H, D, RD, seed=11)
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}

    def call(positions):
        out = flydsl_qk_norm_rope_quant(d["q"], d["kv"], d["kv_weight"], d["cos_cache"], d["sin_cache"], positions,
                                        num_q_heads=H, head_dim=D, rope_head_dim=RD, q_weight=d["q_weight"])
        torch.cuda.synchronize()
        return out

    call(d["positions"])
    assert _lib.debug_violations(checked) == 0
    bad = d["positions"].clone()
    bad[2] = d["cos_cache"].shape[0] + 5
    call(bad)
    assert _lib.debug_violations(checked) == _lib.VIOLATION_POSITION
