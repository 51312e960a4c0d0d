"""The fused RMSNorm + GPT-J RoPE + fp8 quant kernel against the oracle.

Each case runs flydsl_qk_norm_rope_quant (one launch of the C ABI's
pa_fp8_qk_norm_rope_quant) and compares with oracle/qk_norm_rope.py on the
same seeded inputs, and the golden fixtures without the oracle.  Bar:
  * bf16 outputs within one bf16 step (2^-7 relative) of the oracle, plus
    2e-5 absolute: the kernel uses the hardware rsqrt, a different sum order
    and fused multiply-adds, so a value on a rounding boundary may round the
    other way, and a rotated value that nearly cancels (e*c - o*s) carries
    the float32 error of its O(1) terms;
  * fp8 outputs within one e4m3fn step (2^-3 relative, 2^-8 floor for the
    (-2^-8, 0) clamp); the hardware reciprocal in the factor moves values by
    an ulp;
  * float32 scales within 1e-5 relative; e8m0 scale bytes equal.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from flydsl_amd import flydsl_qk_norm_rope_quant
from tests.golden import make_golden as mg
from tests.test_golden import load
from tests.test_qk_norm_rope_oracle import close_bf16, close_fp8, fp8_values, make_inputs, run_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def run_gpu(inp, H, D, RD, kv_stride=None, **kw):
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    if kv_stride is not None and kv_stride != D:
        wide = torch.zeros(d["kv"].shape[0], kv_stride, dtype=torch.bfloat16, device=DEV)
        wide[:, :D] = d["kv"]
        d["kv"] = wide[:, :D]
    q, kv, qs, kvs = flydsl_qk_norm_rope_quant(d["q"], d["kv"], d["kv_weight"], d["cos_cache"], d["sin_cache"],
                                               d["positions"], num_q_heads=H, head_dim=D, rope_head_dim=RD,
                                               q_weight=d["q_weight"], **kw)
    torch.cuda.synchronize()
    return q.cpu(), kv.cpu(), None if qs is None else qs.cpu(), None if kvs is None else kvs.cpu()


def check(got, want, quant, e8m0, tag):
    gq, gkv, gqs, gkvs = got
    wq, wkv, wqs, wkvs = want
    if quant:
        assert gq.dtype == torch.float8_e4m3fn and gkv.dtype == torch.float8_e4m3fn
        for g, w, n in ((gq, wq, "q_out"), (gkv, wkv, "kv_out")):
            gv = fp8_values(g.view(torch.uint8).numpy())
            wv = fp8_values(np.asarray(w).reshape(gv.shape))
            bad = ~close_fp8(gv, wv)
            assert not bad.any(), f"{tag} {n}: {int(bad.sum())} of {bad.size} off, e.g. {gv[bad][:4]} vs {wv[bad][:4]}"
        for g, w, n in ((gqs, wqs, "q_scale"), (gkvs, wkvs, "kv_scale")):
            g = g.numpy()
            w = np.asarray(w).reshape(g.shape)
            if e8m0:
                assert g.dtype == np.uint8 and np.array_equal(g, w), f"{tag} {n}"
            else:
                assert np.allclose(g, w, rtol=1e-5, atol=0), f"{tag} {n}: max rel {np.max(np.abs(g / w - 1)):.2e}"
    else:
        assert gq.dtype == torch.bfloat16 and gqs is None and gkvs is None
        for g, w, n in ((gq, wq, "q_out"), (gkv, wkv, "kv_out")):
            gv = g.float().numpy()
            wv = np.asarray(w).reshape(gv.shape)
            bad = ~close_bf16(gv, wv, atol=2e-5)
            assert not bad.any(), f"{tag} {n}: {int(bad.sum())} of {bad.size} off, e.g. {gv[bad][:4]} vs {wv[bad][:4]}"


CASES = [
    # (T, H, D, RD, quant, G, scale_dtype, q_weighted, kv_stride)
    (1, 16, 512, 64, False, None, "fp32", False, 512),
    (7, 16, 512, 64, True, None, "fp32", False, 1024),
    (33, 8, 512, 64, True, 128, "fp32", True, 512),
    (33, 8, 512, 64, True, 32, "e8m0", False, 576),
    (5, 3, 512, 64, True, 64, "e8m0", True, 512),
    (257, 1, 512, 64, False, None, "fp32", True, 512),
    (9, 4, 256, 64, True, 64, "fp32", False, 256),
    (9, 4, 256, 256, False, None, "fp32", False, 320),
    (9, 5, 128, 128, True, 32, "e8m0", True, 128),
    (9, 5, 128, 0, True, 128, "fp32", False, 130),
    (3, 0, 512, 64, True, 128, "fp32", False, 512),
    (1000, 2, 128, 64, False, None, "fp32", False, 128),
]


@pytest.mark.parametrize("T,H,D,RD,quant,G,sd,qw,kv_stride", CASES,
                         ids=[f"T{c[0]}_H{c[1]}_D{c[2]}_RD{c[3]}_{'q' + str(c[5] or c[2]) + c[6] if c[4] else 'bf16'}"
                              f"{'_qw' if c[7] else ''}_s{c[8]}" for c in CASES])
def test_matches_oracle(T, H, D, RD, quant, G, sd, qw, kv_stride):
    inp = make_inputs(T=T, H=H, D=D, RD=RD, seed=T * 7 + H + D + RD, q_weighted=qw, max_pos=128)
    kw = dict(quant=quant, quant_group_size=G, scale_dtype=sd)
    got = run_gpu(inp, H, D, RD, kv_stride=kv_stride, **kw)
    want = run_oracle(inp, H, D, RD, **kw)
    check(got, want, quant, sd == "e8m0", f"T{T} H{H} D{D}")


def test_edge_rows_and_positions():
    """Zero rows, huge and tiny rows, positions outside the table (-1, past
    the end, int64 with high bits), the small-negative fp8 clamp."""
    T, H, D, RD = 8, 3, 512, 64
    inp = make_inputs(T=T, H=H, D=D, RD=RD, seed=77, max_pos=32, q_weighted=True)
    q = inp["q"].reshape(T, H, D).clone()
    q[0] = 0.0
    q[1] *= 1e4
    q[2] *= 1e-4
    inp["q"] = q.reshape(T, H * D)
    inp["kv"][3] = 0.0
    inp["positions"] = torch.tensor([0, -1, 32, 2**40 + 5, 5, 31, 7, -(2**35)], dtype=torch.int64)
    for quant, sd in ((False, "fp32"), (True, "fp32"), (True, "e8m0")):
        kw = dict(quant=quant, quant_group_size=128 if quant else None, scale_dtype=sd)
        check(run_gpu(inp, H, D, RD, **kw), run_oracle(inp, H, D, RD, **kw), quant, sd == "e8m0", f"edge {sd} {quant}")


def test_preallocated_outputs_and_stream():
    T, H, D, RD = 12, 4, 512, 64
    inp = make_inputs(T=T, H=H, D=D, RD=RD, seed=5)
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    q_out = torch.full((T, H, D), 7, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
    kv_out = torch.empty((T, D), dtype=torch.float8_e4m3fn, device=DEV)
    q_scale = torch.empty((T, H, 4), dtype=torch.float32, device=DEV)
    kv_scale = torch.empty((T, 4), dtype=torch.float32, device=DEV)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        r = flydsl_qk_norm_rope_quant(d["q"], d["kv"], d["kv_weight"], d["cos_cache"], d["sin_cache"], d["positions"],
                                      num_q_heads=H, head_dim=D, rope_head_dim=RD, quant=True, quant_group_size=128,
                                      q_out=q_out, kv_out=kv_out, q_scale=q_scale, kv_scale=kv_scale, stream=s)
    s.synchronize()
    assert r[0] is q_out and r[1] is kv_out and r[2] is q_scale and r[3] is kv_scale
    want = run_oracle(inp, H, D, RD, quant=True, quant_group_size=128)
    check((q_out.cpu(), kv_out.cpu(), q_scale.cpu(), kv_scale.cpu()), want, True, False, "prealloc")


@pytest.mark.parametrize("name", list(mg.QKNR_CASES))
def test_matches_fixture(name):
    fx = load("qk_norm_rope.npz")
    T, H, D, RD, quant, G, sd, qw, max_pos, kv_stride = mg.QKNR_CASES[name]
    shapes = mg.qknr_inputs(name)  # dtypes and shapes; values come from the fixture
    inp = {}
    for k, t in shapes.items():
        if t is None:
            inp[k] = None
        elif t.is_floating_point():
            inp[k] = torch.from_numpy(fx[f"{name}/{k}"].view(np.int16)).view(torch.bfloat16).reshape(t.shape)
        else:
            inp[k] = torch.from_numpy(fx[f"{name}/{k}"]).reshape(t.shape)
    got = run_gpu(inp, H, D, RD, kv_stride=kv_stride, quant=quant, quant_group_size=G, scale_dtype=sd)
    want = tuple(fx.get(f"{name}/{k}") for k in ("q_out", "kv_out", "q_scale", "kv_scale"))
    check(got, want, quant, sd == "e8m0", name)
