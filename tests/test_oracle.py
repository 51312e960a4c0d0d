"""Pins the CPU oracle before anything is compared against it.

Each restated function is checked against something independent of its
own formula: torch's fp8 cast (a library routine), the float64 NumPy brute
force (separate gather, decode and mask code), closed-form special cases,
torch's scaled_dot_product_attention, and identities (page permutation,
log-sum-exp merge of any split, window >= context).  The mutation tests at
the end plant plausible mistakes in the oracle's inputs or wiring and show
the brute-force comparison catches each one.
"""

from __future__ import annotations

import math
import zlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fp8, plan, torch_ref
from tests._cases import flat_scales, indptr, make_case, numpy_oracle, slot_partials, torch_oracle

FP8 = torch.float8_e4m3fn


# ---------------------------------------------------------------- fp8 format


def test_fp8_decode_table_matches_torch():
    ours = fp8.decode_table()
    lib = torch.arange(256, dtype=torch.uint8).view(FP8).to(torch.float64).numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(lib))
    ok = ~np.isnan(lib)
    assert np.array_equal(ours[ok], lib[ok])
    assert np.nanmax(ours) == 448.0
    assert ours[1] == 2.0**-9  # smallest subnormal


def test_fp8_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    vals = np.concatenate(
        [
            rng.normal(size=4000) * 10.0 ** rng.uniform(-4, 2.7, size=4000),
            fp8.decode_table()[~np.isnan(fp8.decode_table())],
            # midpoints between neighbours (ties to even) and the overflow edge
            (fp8.decode_table()[:126] + fp8.decode_table()[1:127]) / 2,
            [448.0, 463.9, 464.0, 464.1, 480.0, 1e6, 2.0**-10, 1.5 * 2.0**-10, 3 * 2.0**-11],
        ]
    ).astype(np.float32)
    vals = np.concatenate([vals, -vals])
    ours = fp8.encode(vals.astype(np.float64))
    lib = torch.from_numpy(vals).to(FP8).view(torch.uint8).numpy()
    nan_o, nan_l = np.isnan(fp8.decode(ours)), np.isnan(fp8.decode(lib))
    assert np.array_equal(nan_o, nan_l)
    assert np.array_equal(ours[~nan_o], lib[~nan_l])


# ------------------------------------------------------------- quantisers


def test_pertoken_quant_scale_and_roundtrip():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 7, 128, generator=g) * torch.rand(5, 7, 1, generator=g) * 10
    x[2, 3] = 0.0
    q, s = torch_ref.pertoken_quant(x)
    amax = x.abs().amax(-1, keepdim=True)
    exp = torch.where(amax == 0, torch.ones_like(amax), amax / 448.0)
    assert torch.equal(s, exp)
    deq = q.float() * s
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 above the
    # subnormal range, absolute error <= 2^-10 * scale below it.
    err = (deq - x).abs()
    bound = torch.maximum(x.abs() * 2.0**-4, s * 2.0**-10)
    assert bool((err <= bound + 1e-12).all())
    assert bool((q[2, 3].float() == 0).all())


def test_per_tensor_quant_uses_global_amax():
    x = torch.tensor([[1.0, -3.5], [0.25, 2.0]])
    q, s = torch_ref.per_tensor_quant(x)
    assert s.shape == (1,) and float(s) == pytest.approx(3.5 / 448.0)
    assert float(q.float().abs().max()) == 448.0


def test_value_shuffle_roundtrip():
    v = torch.arange(3 * 2 * 128 * 64, dtype=torch.int32).reshape(3, 2, 128, 64).to(torch.uint8)
    t = torch_ref.shuffle_value_cache_layout(v)
    assert t.shape == (3, 2, 4, 128, 16)
    assert torch.equal(t[1, 1, 2, 5, 7], v[1, 1, 5, 2 * 16 + 7])
    assert torch.equal(torch_ref.unshuffle_value_cache_layout(t), v)


# ------------------------------------------- torch oracle vs float64 brute force

VARIANTS = {
    "per_tensor": dict(),
    "per_token": dict(per_token=True),
    "mtp_causal": dict(query_length=4, num_query_heads=16, num_kv_heads=4),
    "window": dict(sliding_window=40, ctx_range=(1, 150)),
    "window_mtp": dict(sliding_window=23, query_length=3, ctx_range=(3, 120)),
    "page64": dict(block_size=64, ctx_range=(1, 300)),
    "gqa16_ql2": dict(query_length=2, num_query_heads=32, num_kv_heads=2, per_token=True),
    "uniform_dist": dict(dist="uniform"),
    # the generic kernels' shapes: head sizes other than 128, > 64 columns
    "d64": dict(head_size=64),
    "d192_mtp": dict(head_size=192, query_length=2, num_query_heads=8, num_kv_heads=2, per_token=True),
    "d256_pt": dict(head_size=256, per_token=True),
    "eq128": dict(query_length=8, num_query_heads=32, num_kv_heads=2, ctx_range=(8, 120)),
    # head sizes above 256 (the generic kernels' single-buffer form)
    "d320_window": dict(head_size=320, sliding_window=31, ctx_range=(1, 120)),
    "d384_mtp": dict(head_size=384, query_length=2, num_query_heads=8, num_kv_heads=2),
    "d448_pt": dict(head_size=448, per_token=True, ctx_range=(1, 90)),
    "d512_pt_mtp": dict(head_size=512, per_token=True, query_length=3, num_query_heads=12, num_kv_heads=3,
                        ctx_range=(3, 100)),
}


@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_torch_oracle_matches_float64_bruteforce(name):
    kw = dict(VARIANTS[name])
    ql = kw.get("query_length", 1)
    kw.setdefault("ctx_range", (ql, 160))
    case = make_case(seed=zlib.crc32(name.encode()) % 1000, **kw)
    ours = torch_oracle(case).double().numpy()
    ref = numpy_oracle(case)
    np.testing.assert_allclose(ours, ref, atol=2e-6, rtol=0)


# ----------------------------------------------------------- closed forms


def test_single_token_context_returns_the_value():
    case = make_case(ctx=[1, 1], seed=3, per_token=True)
    out = torch_oracle(case)
    ks, vs = flat_scales(case)
    for b in range(2):
        page = int(case["block_tables"][b, 0])
        v = torch_ref.unshuffle_value_cache_layout(case["value_cache"])[page, :, :, 0].float()  # [H, D]
        v = v * vs[:, page * 16].unsqueeze(-1)
        exp = v.repeat_interleave(4, dim=0)
        assert torch.equal(out[b], exp)


def test_equal_keys_give_mean_of_values():
    case = make_case(ctx=[37, 200], seed=4)
    kc = case["key_cache"].view(torch.uint8)
    kc[:] = kc[0, :, :, 0:1, :].clone()  # every token of every page = one key per head
    out = torch_oracle(case)
    ks, vs = flat_scales(case)
    for b, ctx in enumerate([37, 200]):
        _, v = torch_ref.gather_tokens(
            case["key_cache"], case["value_cache"], case["block_tables"][b].tolist(), ctx, ks, vs
        )
        exp = v.mean(0).repeat_interleave(4, dim=0)
        torch.testing.assert_close(out[b], exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("ql,window,d", [(1, 0, 128), (3, 0, 128), (2, 17, 128), (1, 0, 64), (2, 9, 256), (1, 0, 320),
                                         (2, 13, 512)])
def test_sdpa_library_routine(ql, window, d):
    """Each sequence reduces to torch's scaled_dot_product_attention."""
    case = make_case(query_length=ql, num_query_heads=8, num_kv_heads=2, ctx=[ql + 5, 90, 161], seed=5,
                     sliding_window=window, head_size=d)
    out = torch_oracle(case)
    ks, vs = flat_scales(case)
    for b, ctx in enumerate(case["context_lengths"].tolist()):
        k, v = torch_ref.gather_tokens(case["key_cache"], case["value_cache"], case["block_tables"][b].tolist(), ctx, ks, vs)
        q = case["query"][b * ql : (b + 1) * ql].float()  # [ql, Hq, D]
        qpos = torch.arange(ctx - ql, ctx)[:, None]
        kpos = torch.arange(ctx)[None, :]
        allowed = kpos <= qpos
        if window:
            allowed &= qpos - kpos <= window
        ref = F.scaled_dot_product_attention(
            q.transpose(0, 1),
            k.repeat_interleave(4, dim=1).transpose(0, 1),
            v.repeat_interleave(4, dim=1).transpose(0, 1),
            attn_mask=allowed,
            scale=case["softmax_scale"],
        ).transpose(0, 1)
        torch.testing.assert_close(out[b * ql : (b + 1) * ql], ref, atol=2e-6, rtol=1e-5)


# ------------------------------------------------------------- identities


def test_page_permutation_invariance():
    case = make_case(ctx=[100, 50, 170], seed=6, per_token=True)
    base = torch_oracle(case)
    nb = case["key_cache"].shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(0))
    inv = torch.argsort(perm)
    case2 = dict(case)
    case2["key_cache"] = case["key_cache"][perm]
    case2["value_cache"] = case["value_cache"][perm]
    case2["key_scale"] = case["key_scale"][perm]
    case2["value_scale"] = case["value_scale"][perm]
    case2["block_tables"] = inv[case["block_tables"].long()].to(torch.int32)
    assert torch.equal(torch_oracle(case2), base)


def test_window_at_least_context_equals_full():
    case = make_case(ctx=[30, 64, 99], seed=7, query_length=2)
    full = torch_oracle(case)
    case["sliding_window"] = 99
    assert torch.equal(torch_oracle(case), full)


def test_gqa_heads_only_see_their_kv_head():
    case = make_case(ctx=[80, 120], seed=8)
    base = torch_oracle(case)
    case["key_cache"].view(torch.uint8)[:, 1] ^= 0x11  # perturb kv head 1
    out = torch_oracle(case)
    assert torch.equal(out[:, :4], base[:, :4])
    assert not torch.equal(out[:, 4:], base[:, 4:])


@pytest.mark.parametrize("P,window,ql,d", [(1, 0, 1, 128), (3, 0, 1, 128), (8, 0, 2, 128), (6, 300, 1, 128),
                                           (4, 77, 3, 128), (5, 0, 2, 256), (6, 120, 1, 64), (3, 0, 1, 320),
                                           (4, 50, 2, 512)])
def test_slot_partials_merge_to_full_attention(P, window, ql, d):
    """Any slot split, merged by LSE, reproduces the unsplit attention."""
    case = make_case(ctx=[ql, 255, 256, 257, 700, 1100][: 6], query_length=ql, seed=9, sliding_window=window,
                     per_token=True, head_size=d)
    if window:
        P = max(P, plan.sw_partition_count(window, query_length=ql))
    es, ml, to = slot_partials(case, P)
    merged = torch_ref.lse_merge(es, ml, to)  # [B, Hkv, ql*gqa, D]
    b, hkv, eq, d = merged.shape
    gqa = eq // ql
    out = merged.reshape(b, hkv, ql, gqa, d).permute(0, 2, 1, 3, 4).reshape(b * ql, hkv * gqa, d)
    ref = torch_oracle(case).double()
    torch.testing.assert_close(out, ref, atol=2e-6, rtol=1e-5)


def test_lse_merge_empty_rows_are_zero():
    es = torch.zeros(2, 3, 5)
    ml = torch.full((2, 3, 5), float("-inf"))
    to = torch.randn(2, 3, 5, 7)
    assert torch.equal(torch_ref.lse_merge(es, ml, to), torch.zeros(2, 5, 7, dtype=torch.float64))


# ------------------------------------------------------ planted mistakes


def _max_err(a, b):
    return float(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64)).max())


def test_brute_force_catches_off_by_one_causal_bound():
    case = make_case(query_length=3, ctx=[10, 40], seed=10)
    ref = numpy_oracle(case)
    # a causal bound one token too wide == attending with ctx+1 keys visible
    bad = dict(case)
    bad["query_length"] = 3
    ks, vs = flat_scales(case)
    q = case["query"].float()
    out = torch_ref.reference_masked_attention  # noqa: F841 (documented path)
    wrong = []
    for b, ctx in enumerate([10, 40]):
        k, v = torch_ref.gather_tokens(case["key_cache"], case["value_cache"], case["block_tables"][b].tolist(), ctx, ks, vs)
        logits = torch.einsum("qhd,khd->hqk", q[3 * b : 3 * b + 3], k.repeat_interleave(4, 1)) * case["softmax_scale"]
        allowed = torch.ones(3, ctx, dtype=torch.bool).tril(diagonal=ctx - 3 + 1)
        w = torch.softmax(logits.masked_fill(~allowed, float("-inf")), -1)
        wrong.append(torch.einsum("hqk,khd->qhd", w, v.repeat_interleave(4, 1)))
    assert _max_err(torch.cat(wrong), ref) > 1e-2


def test_brute_force_catches_window_off_by_one():
    case = make_case(ctx=[60, 90], seed=11, sliding_window=20)
    ref = numpy_oracle(case)
    case["sliding_window"] = 19
    assert _max_err(torch_oracle(case), ref) > 1e-2


def test_brute_force_catches_transposed_gqa_mapping():
    case = make_case(ctx=[50, 70], seed=12)
    ref = numpy_oracle(case)
    out = torch_oracle(case)
    # head hh read kv head hh % Hkv instead of hh // gqa
    perm = torch.tensor([(hh % 4) * 2 + hh // 4 for hh in range(8)])
    case_bad = dict(case)
    case_bad["query"] = case["query"][:, perm]
    bad = torch_oracle(case_bad)[:, torch.argsort(perm)]
    assert _max_err(out, ref) < 1e-5
    assert _max_err(bad, ref) > 1e-2


def test_brute_force_catches_wrong_page_walk():
    case = make_case(ctx=[70, 100], seed=13)
    ref = numpy_oracle(case)
    bad = dict(case)
    bad["block_tables"] = case["block_tables"].roll(1, dims=1)
    assert _max_err(torch_oracle(bad), ref) > 1e-2


def test_brute_force_catches_dropped_value_scale():
    case = make_case(ctx=[70, 100], seed=14, per_token=True)
    ref = numpy_oracle(case)
    bad = dict(case)
    bad["value_scale"] = torch.ones_like(case["value_scale"]) * case["value_scale"].mean()
    assert _max_err(torch_oracle(bad), ref) > 1e-3
