"""The fused RMSNorm + GPT-J RoPE + fp8 quant restatement (oracle/qk_norm_rope.py), pinned.

The reference ships no test and no fixtures for kernels/qk_norm_rope_quant.py.
What pins the restatement here:
  * an independent float64 loop over rows, elements and pairs written from
    the kernel's algebra (:330-474), compared to within the bf16 / fp8
    rounding of the outputs;
  * closed forms: a constant row normalises to +-1; cos = 1, sin = 0 (position
    0 of a real table) leaves the row unrotated; a rotation keeps pair norms;
    dequantised fp8 (value * scale) reproduces the normalised row; the
    element at a group's amax quantises to fp8(448 / sqrt2) = 320; an e8m0
    byte equals the biased exponent of amax * rstd * sqrt2 rounded up at
    significand 1.5, minus 7;
  * edge rules: positions outside the cos/sin table rotate with zeros;
    values in (-2^-8, 0) store as +0.
Planted mistakes (NeoX pairing, a weighted norm statistic, swapped cos and
sin, no epsilon) fail the float64 comparison.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import qk_norm_rope as qnr

SQRT2 = math.sqrt(2.0)


def make_inputs(T=5, H=3, D=128, RD=64, seed=0, max_pos=64, q_weighted=False, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(T, H * D, generator=g) * scale).to(torch.bfloat16)
    kv = (torch.randn(T, D, generator=g) * scale).to(torch.bfloat16)
    kvw = (1.0 + 0.5 * torch.randn(D, generator=g)).to(torch.bfloat16)
    qw = (1.0 + 0.5 * torch.randn(D, generator=g)).to(torch.bfloat16) if q_weighted else None
    cos, sin = qnr.rope_table(max_pos, RD) if RD else (torch.ones(max_pos, 0, dtype=torch.bfloat16),) * 2
    pos = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int64)
    return dict(q=q, kv=kv, kv_weight=kvw, cos_cache=cos, sin_cache=sin, positions=pos, q_weight=qw)


def f64_reference(inp, H, D, RD, quant=False, G=None, e8m0=False, pairing="gptj", weighted_norm=False,
                  swap_cs=False, eps=1e-6):
    """Float64 loops over rows, written from the kernel's algebra.  Returns
    (q rows [T, H, D], kv rows [T, D]) of unquantised values (for quant:
    the values before fp8 rounding), and the scales as float64 (e8m0 as the
    byte values)."""
    G = G or D
    T = inp["q"].shape[0]
    xq = inp["q"].double().reshape(T, H, D).numpy()
    xkv = inp["kv"].double().numpy()
    wkv = inp["kv_weight"].double().numpy()
    wq = inp["q_weight"].double().numpy() if inp["q_weight"] is not None else None
    cos = inp["cos_cache"].double().reshape(inp["cos_cache"].shape[0], RD // 2).numpy()
    sin = inp["sin_cache"].double().reshape(inp["sin_cache"].shape[0], RD // 2).numpy()
    out_q = np.zeros((T, H, D))
    out_kv = np.zeros((T, D))
    sc_q = np.zeros((T, H, D // G))
    sc_kv = np.zeros((T, D // G))
    for t in range(T):
        p = int(inp["positions"][t])
        for r in range(H + 1):
            x = xq[t, r] if r < H else xkv[t]
            w = (wq if r < H else wkv)
            w = w if w is not None else np.ones(D)
            xw = x * w
            stat = xw if weighted_norm else x
            rstd = 1.0 / math.sqrt(float(np.mean(stat * stat)) + eps)
            y = np.zeros(D)
            scales = np.zeros(D // G)
            for gi in range(D // G):
                seg = slice(gi * G, (gi + 1) * G)
                if quant:
                    am = max(float(np.max(np.abs(xw[seg]))), 1e-12)
                    if e8m0:
                        post = am * rstd * SQRT2
                        m, ex = math.frexp(post)  # post = m * 2^ex, m in [0.5, 1)
                        e = (ex - 1 + 127) + (1 if m >= 0.75 else 0) - 7
                        e = min(max(e, 0), 255)
                        factor = rstd * 2.0 ** (127 - e)
                        scales[gi] = e
                    else:
                        factor = 448.0 / (SQRT2 * am)
                        scales[gi] = am * rstd * SQRT2 / 448.0
                    y[seg] = xw[seg] * factor
                else:
                    y[seg] = xw[seg] * rstd
            nope = D - RD
            c = cos[p] if 0 <= p < cos.shape[0] else np.zeros(RD // 2)
            s = sin[p] if 0 <= p < cos.shape[0] else np.zeros(RD // 2)
            if swap_cs:
                c, s = s, c
            z = y.copy()
            for k in range(RD // 2):
                if pairing == "gptj":
                    i0, i1 = nope + 2 * k, nope + 2 * k + 1
                else:  # NeoX: halves of the rope part
                    i0, i1 = nope + k, nope + RD // 2 + k
                e_, o_ = y[i0], y[i1]
                z[i0] = e_ * c[k] - o_ * s[k]
                z[i1] = e_ * s[k] + o_ * c[k]
            if r < H:
                out_q[t, r] = z
                sc_q[t, r] = scales
            else:
                out_kv[t] = z
                sc_kv[t] = scales
    return out_q, out_kv, sc_q, sc_kv


def run_oracle(inp, H, D, RD, **kw):
    return qnr.qk_norm_rope_quant(inp["q"], inp["kv"], inp["kv_weight"], inp["cos_cache"], inp["sin_cache"],
                                  inp["positions"], num_q_heads=H, head_dim=D, rope_head_dim=RD,
                                  q_weight=inp["q_weight"], **kw)


def fp8_values(b: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(b)).view(torch.float8_e4m3fn).float().numpy()


def close_bf16(got, ref, atol=1e-30):
    """Within one bf16 step of ref (8 significant bits), plus atol."""
    return np.abs(got - ref) <= 2.0**-7 * np.abs(ref) + atol


def close_fp8(got, ref):
    """Within one e4m3fn step of ref (4 significant bits); values in (-2^-8, 0)
    may store as +0 (the reference's clamp), hence the 2^-8 floor."""
    return np.abs(got - ref) <= 2.0**-3 * np.abs(ref) + 2.0**-8


@pytest.mark.parametrize("D,RD,H,qw", [(128, 64, 3, False), (512, 64, 2, True), (256, 256, 1, False), (128, 0, 2, True)])
def test_bf16_matches_float64_loops(D, RD, H, qw):
    inp = make_inputs(T=4, H=H, D=D, RD=RD, seed=D + RD + H, q_weighted=qw)
    q, kv, sq, skv = run_oracle(inp, H, D, RD)
    rq, rkv, _, _ = f64_reference(inp, H, D, RD)
    assert sq is None and skv is None
    assert close_bf16(q, rq).all() and close_bf16(kv, rkv).all()


@pytest.mark.parametrize("G,e8m0", [(128, False), (32, False), (64, True), (512, True)])
def test_fp8_matches_float64_loops(G, e8m0):
    D, RD, H = 512, 64, 3
    inp = make_inputs(T=4, H=H, D=D, RD=RD, seed=G + e8m0, q_weighted=True)
    q, kv, sq, skv = run_oracle(inp, H, D, RD, quant=True, quant_group_size=G, scale_dtype="e8m0" if e8m0 else "fp32")
    rq, rkv, rsq, rskv = f64_reference(inp, H, D, RD, quant=True, G=G, e8m0=e8m0)
    assert close_fp8(fp8_values(q), rq).all() and close_fp8(fp8_values(kv), rkv).all()
    if e8m0:
        assert sq.dtype == np.uint8 and (sq == rsq).all() and (skv == rskv).all()
    else:
        assert np.allclose(sq, rsq, rtol=1e-6, atol=0) and np.allclose(skv, rskv, rtol=1e-6, atol=0)


@pytest.mark.parametrize("mistake", [dict(pairing="neox"), dict(weighted_norm=True), dict(swap_cs=True),
                                     dict(eps=0.0)])
def test_planted_mistakes_fail(mistake):
    D, RD, H = 128, 64, 2
    # small-magnitude rows make the missing epsilon visible
    inp = make_inputs(T=4, H=H, D=D, RD=RD, seed=9, q_weighted=True, scale=2e-3 if "eps" in mistake else 1.0)
    q, kv, _, _ = run_oracle(inp, H, D, RD)
    rq, rkv, _, _ = f64_reference(inp, H, D, RD, **mistake)
    assert not (close_bf16(q, rq).all() and close_bf16(kv, rkv).all())


def test_constant_rows_normalise_to_unit():
    D, RD, H = 256, 0, 2
    inp = make_inputs(T=3, H=H, D=D, RD=RD)
    inp["q"] = torch.full_like(inp["q"], -3.0)
    inp["kv"] = torch.full_like(inp["kv"], 0.5)
    inp["kv_weight"] = torch.ones_like(inp["kv_weight"])
    q, kv, _, _ = run_oracle(inp, H, D, RD)
    assert np.allclose(q, -1.0, atol=2**-8) and np.allclose(kv, 1.0, atol=2**-7)


def test_position_zero_is_unrotated_and_pairs_keep_norms():
    D, RD, H = 128, 128, 3
    inp = make_inputs(T=6, H=H, D=D, RD=RD, seed=3)
    empty = torch.ones(4, 0, dtype=torch.bfloat16)
    q_plain, kv_plain, _, _ = run_oracle(dict(inp, cos_cache=empty, sin_cache=empty), H, D, 0)
    # cos(0) = 1, sin(0) = 0: the rotation is the identity
    q0, kv0, _, _ = run_oracle(dict(inp, positions=torch.zeros_like(inp["positions"])), H, D, RD)
    assert np.array_equal(q0, q_plain) and np.array_equal(kv0, kv_plain)
    # any position keeps each pair's norm (bf16 cos/sin: |c^2 + s^2 - 1| < 2^-7)
    q, kv, _, _ = run_oracle(inp, H, D, RD)
    pn = lambda a: np.hypot(a[..., 0::2], a[..., 1::2])  # noqa: E731
    assert np.allclose(pn(q), pn(q_plain), rtol=2**-6, atol=1e-6)
    assert np.allclose(pn(kv), pn(kv_plain), rtol=2**-6, atol=1e-6)


def test_dequantised_fp8_reproduces_normalised_rows():
    D, RD, H, G = 512, 64, 4, 64
    inp = make_inputs(T=3, H=H, D=D, RD=RD, seed=5, q_weighted=True)
    qb, kvb, sq, skv = run_oracle(inp, H, D, RD)
    qf, kvf, sqf, skvf = run_oracle(inp, H, D, RD, quant=True, quant_group_size=G)
    deq_q = fp8_values(qf) * np.repeat(sqf, G, axis=-1)
    deq_kv = fp8_values(kvf) * np.repeat(skvf, G, axis=-1)
    # fp8 keeps 4 significant bits; compare against the group's largest value
    big_q = np.repeat(np.abs(qb).reshape(3, H, D // G, G).max(-1), G, axis=-1)
    assert (np.abs(deq_q - qb) <= 2**-4 * np.abs(qb) + 2**-8 * big_q + 1e-6).all()
    assert np.abs(deq_kv - kvb).max() <= 2**-4 * np.abs(kvb).max()
    # the nope element at a group's amax is quantised to fp8(448 / sqrt2) = 320
    nope_groups = fp8_values(qf)[..., : D - RD].reshape(3, H, -1, G)
    assert np.allclose(np.abs(nope_groups).max(-1), 320.0)


def test_out_of_table_positions_rotate_with_zeros():
    D, RD, H = 128, 64, 2
    inp = make_inputs(T=4, H=H, D=D, RD=RD, seed=11, max_pos=16)
    inp["positions"] = torch.tensor([-1, 16, 2**40 + 3, 3], dtype=torch.int64)
    q, kv, _, _ = run_oracle(inp, H, D, RD)
    assert (q[:2, :, D - RD:] == 0).all() and (kv[:2, D - RD:] == 0).all()
    assert (q[:2, :, : D - RD] != 0).any()
    # int64 positions are read as their low 32-bit words: 2^40 + 3 acts as 3
    q3, kv3, _, _ = run_oracle(dict(inp, positions=torch.tensor([-1, 16, 3, 3], dtype=torch.int64)), H, D, RD)
    assert np.array_equal(q, q3) and np.array_equal(kv, kv3)


def test_small_negatives_store_as_positive_zero():
    y = np.array([-1e-3, -0.0039, -0.004, 1e-3, -0.0], dtype=np.float32)
    b = qnr.fp8_bytes(y)
    assert b[0] == 0 and b[1] == 0 and b[2] == 0x82 and b[3] != 0 and b[4] == 0x80
